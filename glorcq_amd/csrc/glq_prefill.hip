// Prefill (many tokens): grouped dequant-to-fp16 MFMA GEMM with the low-rank
// correction, for one projection (glq_gemm_lora; the reference's
// gptq_dequant_gemm_kernel, inference/kernels/gptq_matmul.cu:111-213, taken
// for B > 4, plus the LoRA tail of GLoRCQLinear.forward,
// inference/quantized_linear.py:338-349) and for the routed experts of a MoE
// block over a prompt (glq_moe_prefill; the reference's _forward_sparse,
// inference/moe_block.py:704-740: each active expert's projections on its
// gathered tokens).
//
// pf_gemm_kernel<BITS, TM, RT, MODE, SYM, ZF, DEEP>: a workgroup of 4 waves
// owns TM token rows x (4 * 16 RT) weight rows (MODE gate/up: 4 * 8 RT row
// indices of the gate AND the up matrix) and a range of K.
//  * Per 128-code group one LDS slot receives, by direct global->LDS loads,
//    the TM rows of A (16-byte piece c of slot row r at c ^ (r % 16), so 16
//    lanes reading one piece of 16 rows hit 16 distinct bank groups), each
//    wave's codes, and its rows' scales and zero-points.  A ring of D slots
//    keeps D - 1 groups in flight; each thread waits for its own loads of a
//    group (vmcnt), one barrier makes them everyone's and frees the oldest
//    slot for the next issue.  DEEP rings give half the CU's LDS to one
//    workgroup (for small launches); others take 2 or 3 slots.
//  * A: the dense form reads the caller's x in natural order and builds each
//    MFMA operand in the decode's order with v_perm (pf_nat_a); the MoE forms
//    read rows that their producers already wrote in decode order
//    (glq_gemv_core.h perm_src), gathered through an index list.
//  * B: codes decode into exact fp16 MFMA operands q - zi (zi the
//    zero-point's nearest integer): one v_and_or per code pair lands q under
//    an exponent chosen per bit position (exactly 2^e + q), one packed fp16
//    add removes 2^e + zi.  Each group's fp32 MFMA sum is scaled once,
//    y += s (acc - zf c2), zf = z - zi and c2 the group's sum of x (only for
//    non-integer zero-points: an MFMA of A against ones in the dense form),
//    so W = s (q - z) enters exactly, as in the reference's fp32 kernel.
//    Lane group kb of a wave holds code words 2kb, 2kb+1 (2-bit) or
//    4kb..4kb+3 (4-bit) of a group; k-step t uses slice t of them.
//  * v_mfma_f32_16x16x32_f16 with A = 16 token rows, B = 16 weight rows: each
//    A operand feeds RT MFMAs and each decoded B operand TM/16.
//  * Split K (ks > 1, the MoE launches): each (tile, split) workgroup writes
//    an fp32 partial tile; the last of a tile's splits to arrive (a per-tile
//    counter, left zero again) sums the partials in split order and runs the
//    epilogue, so the result does not depend on arrival order.
//  * Epilogues: DENSE y = fp16(acc + a SV^T + bias); GATE/UP inter =
//    fp16(fp16(silu(fp16 g)) * fp16 u) with each projection's own a SV^T,
//    stored in the down projection's decode order; DOWN fp32 y + a SV^T.
//
// pf_lowrank_kernel: a = x U for the low-rank term (fp32 accumulation, one
// fp16 rounding), 16 rows per workgroup with U staged in LDS.
#include <algorithm>
#include <cstdio>

#include "glq_handoff.h"
#include "glq_stream.h"

namespace glq {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

enum PfMode { kPfDense = 0, kPfGateUp = 1, kPfDown = 2 };

constexpr int kPfThreads = 256;  // 4 waves

struct PfArgs {
  const __half* xp;          // A rows in decode order, K halves each
  const int32_t* arow;       // A row of sorted row p (null: p)
  const uint32_t* codes[2];  // matrix m: (E, N, kw) words
  const __half* scales[2];   // (E, N, G)
  const __half* zeros[2];    // (E, N, G) (unused with SYM)
  int64_t codes_es, sz_es;   // expert strides (elements)
  const __half* a;           // low-rank a (rows, a_ld) fp16: matrix m at column m*rank, or null
  int a_ld;
  const __half* sv[2];       // (E, N, rank)
  int64_t sv_es;
  const __half* bias;        // (N,) or null (dense)
  __half* y;                 // DENSE: (M, N); GATE/UP: inter (rows, N) in decode order
  int64_t y_ld;
  float* yf;                 // DOWN: (rows, N) fp32
  int64_t yf_ld;
  const float* c2;           // ZF: per (group, row) sum of x, (G, c2_ld) fp32
  int64_t c2_ld;
  float* part;               // split-K partial tiles (ks, tiles, TM, ntn*WGROWS) fp32, or null
  unsigned* cnt;             // split-K arrival counters (tiles * ntn), zero between launches
  const int32_t* tiles;      // (max_tiles, 3): expert, first sorted row, rows; null: dense
  const int32_t* ntiles;     // device count of valid tiles
  int M, K, N, G, kw, rank;
  int ntn;                   // weight-row tiles of a workgroup along N
  int ks, gps;               // K splits, groups per split
  int out_bits;              // GATE/UP: decode order of inter's consumer (2 or 4)
  int max_tiles;             // token tiles in the grid (y dimension)
  float zoff;                // added to every zero-point (signed codes stored offset by 2^(b-1))
  // a = x U formed in the same launch (dense form, no K split; pf_xu_job):
  // row-block jobs fill the first xu_rows rows of the grid, and the epilogue
  // waits for its token rows' blocks (a read coherently).  xu_rows == 0: a
  // is given (or absent).
  int xu_rows, xu_nrb, xu_ns, xu_rpad;
  const __half* xu_u;        // U (K, rank)
  float* xu_part;            // (nrb, ns, 16, rpad) fp32 slice partials
  unsigned* xu_cnt;          // (nrb) words: arrivals | ready bit | readers << 16; zero between launches
  uint64_t xu_spin;          // the epilogue's wait bound (100 MHz real-time counter ticks)
};

// The x U jobs of the fused dense launch (see PfArgs).  A row block's word:
// low bits the slices that arrived, kXuReady once its last slice has
// written a, then 1 << 16 per GEMM workgroup that has read it; whichever
// event completes the final word sets it back to zero.
constexpr unsigned kXuReady = 0x8000u;
constexpr size_t kXuJobLds = (4 * 4 * 64) * 4 + 16 * kLowrankRows * 2 +
                             64 * kLowrankUtStride * 2 + 16 * 128 * 4;

__device__ __forceinline__ unsigned pf_xu_final(const PfArgs& g) {
  return ((unsigned)g.ntn << 16) | kXuReady | (unsigned)g.xu_ns;
}

// Job (row block rb, K slice sp): lowrank_partial<4> over the slice, handed
// over; the block's last slice sums the slices in slice order and writes
// a = fp16 (agent-scope stores), then marks the block ready.
__device__ void pf_xu_job(const PfArgs& g, int job, unsigned char* smem, int* flag) {
  const int rb = job / g.xu_ns, sp = job - rb * g.xu_ns, tid = threadIdx.x;
  const int r0 = 16 * rb, rows = min(16, g.M - r0), rank = g.rank, rpad = g.xu_rpad;
  float* red = (float*)smem;
  __half* xl = (__half*)(red + 4 * 4 * 64);
  __half* ut = xl + 16 * kLowrankRows;
  const __half* xb = g.xp + (int64_t)r0 * g.K;
  auto xrow = [&](int m) { return xb + (int64_t)m * g.K; };
  float* slices = g.xu_part + (int64_t)rb * g.xu_ns * 16 * rpad;
  lowrank_partial<4, decltype(xrow), true>(xrow, rows, g.K, rank, rpad, g.xu_u, sp,
                                           slices + (int64_t)sp * 16 * rpad, red, xl, tid, ut);
  if (!handoff_arrive(g.xu_cnt + rb, (unsigned)g.xu_ns, flag)) return;
  for (int i = tid; i < rows * rank; i += kPfThreads) {
    const int m = i / rank, j = i - m * rank;
    const __half v = __float2half(sum_strided_coh(slices + m * rpad + j, 16 * rpad, g.xu_ns));
    handoff_put((uint16_t*)g.a + (int64_t)(r0 + m) * g.a_ld + j, __half_as_ushort(v));
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(g.xu_cnt + rb, kXuReady, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (old + kXuReady == pf_xu_final(g)) handoff_reset(g.xu_cnt + rb);
  }
}

// The epilogue's wait for the row blocks of token rows [p0, p0 + rows): a
// block not ready within xu_spin is formed here, slice by slice in the
// jobs' order (the same bits), and written as the jobs write it.  Every
// thread calls it; smem is free (the ring has drained).
__device__ void pf_xu_wait(const PfArgs& g, int p0, int rows, unsigned char* smem, int* flag) {
  const int rb0 = p0 / 16, rb1 = (p0 + rows - 1) / 16, tid = threadIdx.x;
  if (tid == 0) {
    int missing = 0;
    for (int rb = rb0; rb <= rb1; ++rb) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      while (!(handoff_get(g.xu_cnt + rb) & kXuReady)) {
        if (__builtin_amdgcn_s_memrealtime() - t0 > g.xu_spin) {
          missing |= 1 << (rb - rb0);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    *flag = missing;
  }
  __syncthreads();
  const int missing = *flag;
  __syncthreads();
  for (int rb = rb0; rb <= rb1; ++rb) {
    if (!(missing & (1 << (rb - rb0)))) continue;  // uniform
    const int r0 = 16 * rb, brows = min(16, g.M - r0), rank = g.rank, rpad = g.xu_rpad;
    float* red = (float*)smem;
    __half* xl = (__half*)(red + 4 * 4 * 64);
    __half* ut = xl + 16 * kLowrankRows;
    float* out = (float*)(ut + 64 * kLowrankUtStride);  // 16 x rpad
    const __half* xb = g.xp + (int64_t)r0 * g.K;
    auto xrow = [&](int m) { return xb + (int64_t)m * g.K; };
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // elements tid + 256 q of the block
    for (int sp = 0; sp < g.xu_ns; ++sp) {
      lowrank_partial<4>(xrow, brows, g.K, rank, rpad, g.xu_u, sp, out, red, xl, tid, ut);
      __syncthreads();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = tid + kPfThreads * q, m = i / rpad, j = i - m * rpad;
        if (m < brows && j < rank) acc[q] += out[m * rpad + j];
      }
      __syncthreads();
    }
    const int pad = (8 - g.xu_ns % 8) % 8;  // sum_strided's zeros after the last batch
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      for (int z = 0; z < pad; ++z) acc[q] += 0.f;
      const int i = tid + kPfThreads * q, m = i / rpad, j = i - m * rpad;
      if (m < brows && j < rank)
        handoff_put((uint16_t*)g.a + (int64_t)(r0 + m) * g.a_ld + j,
                    __half_as_ushort(__float2half(acc[q])));
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
}

// 8 halves of a written inside this launch (agent-scope loads).
__device__ __forceinline__ f16x8 pf_load8_coh(const __half* p) {
  const unsigned long long lo = handoff_get((const unsigned long long*)p);
  const unsigned long long hi = handoff_get((const unsigned long long*)p + 1);
  return __builtin_bit_cast(f16x8, u32x4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi,
                                         (uint32_t)(hi >> 32)});
}

// Position of natural column c inside its 16-code block in decode order
// (inverse of perm_src).
template <int BITS>
__device__ __forceinline__ int perm_pos(int c) {
  if constexpr (BITS == 2) return c < 8 ? 2 * c : 2 * (c - 8) + 1;
  else {
    const int h = c & 8, q = c & 7;
    return h + (q < 4 ? 2 * q : 2 * (q - 4) + 1);
  }
}
__device__ __forceinline__ int perm_pos_rt(int bits, int c) {
  return bits == 2 ? perm_pos<2>(c) : perm_pos<4>(c);
}

// Per (row tile, group): packed constants -(2^e + zi) for the exponent biases
// of the decode (2-bit: 1024, 256, 64, 16, 4; 4-bit: 1024, 64), the scale, and
// the fractional part zf = z - zi of the zero-point (zi = the nearest integer).
template <int BITS>
struct PfK {
  f16x2 c[BITS == 2 ? 5 : 2];
  float s, zf;
};

template <int BITS, bool SYM>
__device__ __forceinline__ PfK<BITS> pf_consts(__half sh, __half zh, float zoff) {
  PfK<BITS> k;
  const float z = SYM ? (float)(1 << (BITS - 1)) : __half2float(zh) + zoff;
  const float zi = rintf(z);
  k.zf = z - zi;
  k.s = __half2float(sh);
  constexpr float b2[5] = {1024.f, 256.f, 64.f, 16.f, 4.f};
  constexpr float b4[2] = {1024.f, 64.f};
#pragma unroll
  for (int i = 0; i < (BITS == 2 ? 5 : 2); ++i) {
    const _Float16 v = (_Float16)(-((BITS == 2 ? b2[i] : b4[i]) + zi));  // exact integer
    k.c[i] = f16x2{v, v};
  }
  return k;
}

__device__ __forceinline__ uint32_t pf_sub(uint32_t h, f16x2 c) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, h) + c);  // exact
}

// B operand of k-step t (0..3) of a group: q - zi as fp16 (exact small integers).
template <int BITS, bool SYM>
__device__ __forceinline__ f16x8 pf_decode(const uint32_t* w, const PfK<BITS>& k, int t,
                                           const DecodeConsts& dk) {
  constexpr uint32_t xm = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  u32x4 o;
  if constexpr (BITS == 2) {
    const uint32_t wd = w[t >> 1] ^ xm;
    if ((t & 1) == 0) {
      o.x = pf_sub((wd & 0x00030003u) | dk.e25, k.c[0]);
      o.y = pf_sub((wd & 0x000C000Cu) | dk.e23, k.c[1]);
      o.z = pf_sub((wd & 0x00300030u) | dk.e21, k.c[2]);
      o.w = pf_sub((wd & 0x00C000C0u) | dk.e19, k.c[3]);
    } else {
      const uint32_t v = wd >> 10;
      o.x = pf_sub((wd & 0x03000300u) | dk.e17, k.c[4]);
      o.y = pf_sub((v & 0x00030003u) | dk.e25, k.c[0]);
      o.z = pf_sub((v & 0x000C000Cu) | dk.e23, k.c[1]);
      o.w = pf_sub((v & 0x00300030u) | dk.e21, k.c[2]);
    }
  } else {
    const uint32_t wd = w[t] ^ xm, v = wd >> 8;
    o.x = pf_sub((wd & 0x000F000Fu) | dk.e25, k.c[0]);
    o.y = pf_sub((wd & 0x00F000F0u) | dk.e21, k.c[1]);
    o.z = pf_sub((v & 0x000F000Fu) | dk.e25, k.c[0]);
    o.w = pf_sub((v & 0x00F000F0u) | dk.e21, k.c[1]);
  }
  return __builtin_bit_cast(f16x8, o);
}

// A operand of k-step t (0..3) from an LDS row holding x in NATURAL order
// (16-byte piece P at position P ^ li): the decode's order is made with
// v_perm.  2-bit step t pairs codes (j, j + 8) of word 2kb + t / 2, i.e.
// halves j of natural pieces 4kb + 2 (t / 2) and + 1 (j = 0..3 for even t,
// 4..7 for odd); 4-bit step t pairs codes (j, j + 4) of word 4kb + t, halves
// j and j + 4 of natural piece 4kb + t.
template <int BITS>
__device__ __forceinline__ f16x8 pf_nat_a(const unsigned char* row, int kb, int t, int li) {
  u32x4 o;
  if constexpr (BITS == 2) {
    const int p0 = 4 * kb + 2 * (t >> 1);
    const u32x4 lo = *(const u32x4*)(row + ((p0 ^ li) << 4));
    const u32x4 hi = *(const u32x4*)(row + (((p0 + 1) ^ li) << 4));
    const uint32_t a0 = (t & 1) ? lo.z : lo.x, a1 = (t & 1) ? lo.w : lo.y;
    const uint32_t b0 = (t & 1) ? hi.z : hi.x, b1 = (t & 1) ? hi.w : hi.y;
    o.x = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
    o.y = __builtin_amdgcn_perm(b0, a0, 0x07060302u);
    o.z = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
    o.w = __builtin_amdgcn_perm(b1, a1, 0x07060302u);
  } else {
    const u32x4 v = *(const u32x4*)(row + (((4 * kb + t) ^ li) << 4));
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  }
  return __builtin_bit_cast(f16x8, o);
}

// Weight row of row tile rt of a wave (see the file comment); may be >= N
// (clamp for loads).
template <int RT, int MODE>
__device__ __forceinline__ int pf_row(int n0, int wave, int rt, int li) {
  if constexpr (MODE == kPfGateUp) return n0 + wave * (8 * RT) + (rt % (RT / 2)) * 16 + li;
  else return n0 + wave * (16 * RT) + rt * 16 + li;
}
template <int RT, int MODE>
constexpr int pf_wg_rows() { return MODE == kPfGateUp ? 4 * 8 * RT : 4 * 16 * RT; }

// LDS slot of one group: A (TM token rows x 256 B, swizzled pieces), then per
// wave its RT row tiles' codes (16 rows x CB bytes each, padded to whole
// 1 KB load instructions), scales and zero-points (one fp16 per (row tile,
// row) at a 4-byte stride, as the 2-byte direct-to-LDS load places them).
// Ring depth D: DEEP rings take half the CU's 160 KB (two workgroups per
// CU, as many groups in flight as fit); otherwise 3 slots when two
// workgroups fit a CU, else 2.
template <int BITS, int TM, int RT, bool DEEP = false>
struct PfSlot {
  static constexpr int CB = BITS == 2 ? 32 : 64;        // code bytes per row per group
  static constexpr int CW = RT * 16 * CB;                // code bytes per wave
  static constexpr int CR = CW < 1024 ? 1024 : CW;       // LDS bytes per wave (whole loads)
  static constexpr int A = 0;
  static constexpr int C = TM * 256;
  static constexpr int S = C + 4 * CR;
  static constexpr int Z = S + 4 * 256;
  static constexpr int BYTES = Z + 4 * 256;
  static constexpr int NC = CR / 1024;                   // code load instructions per wave
  static constexpr int NI = TM / 16 + NC + 2;            // loads per lane per group (max)
  static constexpr int DMAX = 2 + 63 / NI;               // the vmcnt field is 6 bits
  static constexpr int DFIT = (80 * 1024 - 64) / BYTES;  // two workgroups per CU
  static constexpr int D = DEEP ? (DFIT < DMAX ? (DFIT < 16 ? DFIT : 16) : (DMAX < 16 ? DMAX : 16))
                                : (2 * 3 * BYTES <= 160 * 1024 ? 3 : 2);
};

template <int BITS, int TM, int RT, int MODE, bool SYM, bool ZF, bool DEEP>
__global__ __launch_bounds__(kPfThreads, 2) void pf_gemm_kernel(PfArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  using SL = PfSlot<BITS, TM, RT, DEEP>;
  constexpr int TT = TM / 16;
  constexpr int XI = TM / 16;  // A load instructions per wave per group (4 rows each)
  constexpr int WGR = pf_wg_rows<RT, MODE>();
  constexpr int NMAT = MODE == kPfGateUp ? 2 : 1;
  constexpr bool NAT = MODE == kPfDense;  // A rows in natural order (the caller's x)
  constexpr int D = SL::D;
  constexpr int NI = XI + SL::NC + 1 + (SYM ? 0 : 1);  // loads per lane per group
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  __shared__ int xflag;
  if (g.xu_rows && (int)blockIdx.y < g.xu_rows) {  // an x U job (uniform)
    const int job = blockIdx.y * gridDim.x + blockIdx.x;
    if (job < g.xu_nrb * g.xu_ns) pf_xu_job(g, job, smem, &xflag);
    return;
  }
  const int ty = blockIdx.y - g.xu_rows;
  int e = 0, p0, rows;
  if (g.tiles) {
    if (ty >= *g.ntiles) return;  // uniform over the workgroup
    e = g.tiles[3 * ty];
    p0 = g.tiles[3 * ty + 1];
    rows = g.tiles[3 * ty + 2];
  } else {
    p0 = ty * TM;
    rows = min(TM, g.M - p0);
  }
  const int tn = blockIdx.x % g.ntn, sp = blockIdx.x / g.ntn;
  const int n0 = tn * WGR;
  const int g0 = sp * g.gps, g1 = min(g0 + g.gps, g.G);

  // ---- per-lane load addresses (offsets in elements; uniform bases) ----
  // A: this lane's XI slot rows
  int aoff[XI];
#pragma unroll
  for (int q = 0; q < XI; ++q) {
    const int r = (wave * XI + q) * 4 + (lane >> 4);
    const int p = p0 + min(r, rows - 1);
    const int ar = g.arow ? g.arow[p] : p;
    aoff[q] = ar * g.K + (((lane & 15) ^ (r & 15)) << 3);
  }
  const uint32_t* cb[NMAT];
  const __half* sb[NMAT];
  const __half* zb[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    cb[m] = g.codes[m] + e * g.codes_es;
    sb[m] = g.scales[m] + e * g.sz_es;
    zb[m] = SYM ? sb[m] : g.zeros[m] + e * g.sz_es;
  }
  // codes: instruction q covers bytes q*1024 + 16*lane of the wave's region
  // (lanes past the wave's code bytes re-load its first ones into the padding)
  int coff[SL::NC], cmat[SL::NC];
#pragma unroll
  for (int q = 0; q < SL::NC; ++q) {
    const int o = (q * 1024 + 16 * lane) % SL::CW;
    const int rt = o / (16 * SL::CB), row = (o % (16 * SL::CB)) / SL::CB;
    const int piece = (o % SL::CB) / 16;
    const int n = min(pf_row<RT, MODE>(n0, wave, rt, row), g.N - 1);
    coff[q] = n * g.kw + 4 * piece;
    cmat[q] = MODE == kPfGateUp ? rt / (RT / 2) : 0;
  }
  // scales / zero-points: lane -> (row tile lane/16, row lane%16)
  int soff, smat;
  {
    const int rt = min(lane >> 4, RT - 1);
    const int n = min(pf_row<RT, MODE>(n0, wave, rt, lane & 15), g.N - 1);
    soff = n * g.G;
    smat = MODE == kPfGateUp ? rt / (RT / 2) : 0;
  }
  auto issue = [&](int grp, unsigned char* slot) {
#pragma unroll
    for (int q = 0; q < XI; ++q)
      __builtin_amdgcn_global_load_lds((const void*)(g.xp + aoff[q] + grp * 128),
                                       (lds_void*)(slot + SL::A + (wave * XI + q) * 1024), 16, 0, 0);
#pragma unroll
    for (int q = 0; q < SL::NC; ++q) {
      const uint32_t* base = NMAT == 2 && cmat[q] ? cb[NMAT - 1] : cb[0];
      __builtin_amdgcn_global_load_lds((const void*)(base + coff[q] + grp * (SL::CB / 4)),
                                       (lds_void*)(slot + SL::C + wave * SL::CR + q * 1024),
                                       16, 0, 0);
    }
    const __half* sbase = NMAT == 2 && smat ? sb[NMAT - 1] : sb[0];
    __builtin_amdgcn_global_load_lds((const void*)(sbase + soff + grp),
                                     (lds_void*)(slot + SL::S + wave * 256), 2, 0, 0);
    if constexpr (!SYM) {
      const __half* zbase = NMAT == 2 && smat ? zb[NMAT - 1] : zb[0];
      __builtin_amdgcn_global_load_lds((const void*)(zbase + soff + grp),
                                       (lds_void*)(slot + SL::Z + wave * 256), 2, 0, 0);
    }
  };

  f32x4 y[TT][RT];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) y[i][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const DecodeConsts dk = DecodeConsts::make();
  const int ng = g1 - g0;
  // every group issues the same loads (past the split's end they re-read its
  // last group into a slot never consumed), so the explicit waits count exactly
#pragma unroll
  for (int d = 0; d < D - 1; ++d) issue(g0 + min(d, ng - 1), smem + d * SL::BYTES);
  for (int it = 0; it < ng; ++it) {
    const int grp = g0 + it;
    wait_vmcnt<NI * (D - 2)>();               // this thread's loads of grp are in
    asm volatile("s_barrier" ::: "memory");   // everyone's are; the slot of grp - 1 is free
    issue(g0 + min(it + D - 1, ng - 1), smem + ((it + D - 1) % D) * SL::BYTES);
    const unsigned char* sl = smem + (it % D) * SL::BYTES;
    // this lane's codes, scale and zero-point per row tile
    uint32_t w[RT][BITS == 2 ? 2 : 4];
    PfK<BITS> kc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const unsigned char* cr = sl + SL::C + wave * SL::CR + (rt * 16 + li) * SL::CB;
      if constexpr (BITS == 2) {
        const u32x2 v = *(const u32x2*)(cr + 8 * kb);
        w[rt][0] = v.x;
        w[rt][1] = v.y;
      } else {
        const u32x4 v = *(const u32x4*)(cr + 16 * kb);
        w[rt][0] = v.x;
        w[rt][1] = v.y;
        w[rt][2] = v.z;
        w[rt][3] = v.w;
      }
      const __half sh = *(const __half*)(sl + SL::S + wave * 256 + (rt * 16 + li) * 4);
      const __half zh = SYM ? sh : *(const __half*)(sl + SL::Z + wave * 256 + (rt * 16 + li) * 4);
      kc[rt] = pf_consts<BITS, SYM>(sh, zh, g.zoff);
    }
    // the group's sum of x (q - zi), fp32
    auto a_op = [&](int i, int t) -> f16x8 {
      const unsigned char* row = sl + SL::A + (16 * i + li) * 256;
      if constexpr (NAT) return pf_nat_a<BITS>(row, kb, t, li);
      else return *(const f16x8*)(row + (((4 * kb + t) ^ li) << 4));
    };
    f32x4 acc[TT][RT];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      f16x8 bf[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) bf[rt] = pf_decode<BITS, SYM>(w[rt], kc[rt], t, dk);
#pragma unroll
      for (int i = 0; i < TT; ++i) {
        const f16x8 av = a_op(i, t);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          acc[i][rt] = mfma_16x16x32(av, bf[rt], t == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][rt]);
      }
    }
    // y += s (acc - zf c2): c2 = the group's sum of x per token, needed only
    // for non-integer zero-points (zf != 0); natural-order A forms it here
    // (an MFMA against ones, when any row of the wave has zf != 0), the
    // decode-order A of the MoE forms reads it from g.c2
    f32x4 c2v[TT];
    if constexpr (ZF && NAT) {
      bool any = false;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) any |= kc[rt].zf != 0.f;
      if (__builtin_amdgcn_ballot_w64(any) != 0) {  // uniform over the wave
        const f16x8 ones = __builtin_bit_cast(f16x8, u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u,
                                                           0x3C003C00u});
#pragma unroll
        for (int i = 0; i < TT; ++i) {
          c2v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < 4; ++t) c2v[i] = mfma_16x16x32(a_op(i, t), ones, c2v[i]);
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const float s = kc[rt].s;
      if (ZF && kc[rt].zf != 0.f) {
        const float zf = kc[rt].zf;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
          float4 c2;
          if constexpr (NAT) {
            c2 = float4{c2v[i][0], c2v[i][1], c2v[i][2], c2v[i][3]};
          } else {
            // rows past the tile's last are read (the layout has whole
            // tiles) and never stored
            c2 = *(const float4*)(g.c2 + (int64_t)grp * g.c2_ld + p0 + 16 * i + 4 * kb);
          }
          y[i][rt][0] = fmaf(s, acc[i][rt][0] - zf * c2.x, y[i][rt][0]);
          y[i][rt][1] = fmaf(s, acc[i][rt][1] - zf * c2.y, y[i][rt][1]);
          y[i][rt][2] = fmaf(s, acc[i][rt][2] - zf * c2.z, y[i][rt][2]);
          y[i][rt][3] = fmaf(s, acc[i][rt][3] - zf * c2.w, y[i][rt][3]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < TT; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) y[i][rt][j] = fmaf(s, acc[i][rt][j], y[i][rt][j]);
      }
    }
  }
  wait_vmcnt<0>();  // the tail's loads land before the workgroup's LDS goes away


  // ---- split K: partial tiles, the last split of a tile reduces ----
  if (g.ks > 1) {
    // partial tile columns: (tn, wave, rt, li), 64 RT per workgroup
    const int ncol = g.ntn * 64 * RT;
    const int cbase = tn * 64 * RT + wave * 16 * RT + li;
    float* mine = g.part + (((int64_t)sp * g.max_tiles + ty) * TM) * ncol;
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int c = cbase + rt * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          handoff_put(mine + (int64_t)(16 * i + 4 * kb + j) * ncol + c, y[i][rt][j]);
      }
    // arrival (glq_handoff.h); the last split reduces and leaves the counter
    // at zero for the next launch
    __shared__ int last;
    unsigned* cnt = g.cnt + (int64_t)ty * g.ntn + tn;
    if (!handoff_arrive(cnt, (unsigned)g.ks, &last)) return;
    if (tid == 0) handoff_reset(cnt);
#pragma unroll
    for (int i = 0; i < TT; ++i)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) y[i][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < g.ks; ++s) {
      const float* ps = g.part + (((int64_t)s * g.max_tiles + ty) * TM) * ncol;
#pragma unroll
      for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const int c = cbase + rt * 16;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            y[i][rt][j] += handoff_get(ps + (int64_t)(16 * i + 4 * kb + j) * ncol + c);
        }
    }
  }

  // ---- low-rank term: y += a SV^T (a: token rows, SV: weight rows) ----
  if (g.xu_rows && g.rank > 0) pf_xu_wait(g, p0, rows, smem, &xflag);
  if (g.a != nullptr && g.rank > 0) {
    constexpr int RM = RT / NMAT;  // row tiles per matrix
    for (int j0 = 0; j0 < g.rank; j0 += 32) {
      const int jk = j0 + 8 * kb;
      const bool jv = jk < g.rank;
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        f16x8 bv[RM];
#pragma unroll
        for (int q = 0; q < RM; ++q) {
          const int rt = m * RM + q;
          const int n = min(pf_row<RT, MODE>(n0, wave, rt, li), g.N - 1);
          bv[q] = jv ? *(const f16x8*)(g.sv[m] + e * g.sv_es + (int64_t)n * g.rank + jk)
                     : f16x8{};
        }
#pragma unroll
        for (int i = 0; i < TT; ++i) {
          const int p = p0 + min(16 * i + li, rows - 1);
          f16x8 av = f16x8{};
          if (jv) {
            const __half* ap = g.a + (int64_t)p * g.a_ld + m * g.rank + jk;
            av = g.xu_rows ? pf_load8_coh(ap) : *(const f16x8*)ap;
          }
#pragma unroll
          for (int q = 0; q < RM; ++q) y[i][m * RM + q] = mfma_16x16x32(av, bv[q], y[i][m * RM + q]);
        }
      }
    }
  }

  // ---- stores: lane holds tokens 16i + 4kb + j of weight row li ----
  if constexpr (MODE == kPfGateUp) {
    constexpr int H2 = RT / 2;
#pragma unroll
    for (int rt = 0; rt < H2; ++rt) {
      const int n = pf_row<RT, MODE>(n0, wave, rt, li);
      if (n >= g.N) continue;
      const int col = (n & ~15) + perm_pos_rt(g.out_bits, n & 15);
#pragma unroll
      for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * i + 4 * kb + j;
          if (r < rows)
            g.y[(int64_t)(p0 + r) * g.y_ld + col] = swiglu_fp16(y[i][rt][j], y[i][rt + H2][j]);
        }
    }
  } else {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = pf_row<RT, MODE>(n0, wave, rt, li);
      if (n >= g.N) continue;
      const float bn = (MODE == kPfDense && g.bias) ? __half2float(g.bias[n]) : 0.f;
#pragma unroll
      for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * i + 4 * kb + j;
          if (r >= rows) continue;
          if constexpr (MODE == kPfDense)
            g.y[(int64_t)(p0 + r) * g.y_ld + n] = __float2half(y[i][rt][j] + bn);
          else
            g.yf[(int64_t)(p0 + r) * g.yf_ld + n] = y[i][rt][j];
        }
    }
  }
  if (g.xu_rows && g.rank > 0) {  // the workgroup has read a of its rows' blocks
    __syncthreads();
    if (tid == 0)
      for (int rb = p0 / 16; rb <= (p0 + rows - 1) / 16; ++rb) {
        const unsigned old = __hip_atomic_fetch_add(g.xu_cnt + rb, 1u << 16, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        if (old + (1u << 16) == pf_xu_final(g)) handoff_reset(g.xu_cnt + rb);
      }
  }
}

// ---------------------------------------------------------------------------
// Low-rank a = x U.  A job owns 16 rows of one tile of the list (one expert)
// and K split sp; its 4 waves take the (matrix, 16-column) tiles of a.  U
// chunks of 128 k (every matrix m) are staged in LDS in their natural (k,
// rank) layout by 16-byte pieces; a lane forms its B operand (8 consecutive k
// of one rank column, in A's order: natural, or the decode order of aperm
// bits) from 8 two-byte LDS reads.  The fp32 partial sums of each split go to
// part (ks, rows, nmat * rank); the GEMM epilogue sums them in split order and
// rounds a to fp16 once.  The dense launch also runs, in its first
// workgroups, the prep of the GEMM's A: x in decode order and its per-group
// sums (one thread per (row, group)).
// ---------------------------------------------------------------------------
struct PfLowrank {
  const __half* x;         // A rows, K halves each
  const int32_t* arow;     // A row of sorted row p (null: p)
  int aperm;               // 0: A natural; 2 or 4: A in that decode order
  const __half* U[2];      // (C, K, rank) per matrix
  int64_t u_cs;            // elements between clusters
  const int32_t* cluster[2];  // (E,) cluster of expert e per matrix (null: 0)
  const int32_t* uslot[2];    // cluster -> row of U[m] (a cross-layer pool), or null
  const int32_t* tiles;    // tile list of the GEMM (null: dense)
  const int32_t* ntiles;
  int tile_rows;           // rows per tile of the list (dense: 16)
  int nmat, rows_total, K, rank, ks, kps;
  float* part;             // (ks, rows_total, nmat * rank) fp32 partial sums of a (ks > 1)
  __half* a_out;           // (rows_total, nmat * rank) a = fp16(x U) (ks == 1, or finalized)
  unsigned* zero_cnt;      // counters the following GEMM launch expects zero, or null
  int n_cnt;
};

constexpr int kLrRows = 16;  // rows per lowrank workgroup (one 16-row MFMA tile)


// One (16 rows, K split) job of a = x U: fp32 partial sums into
// part[sp][row][m * rank + j].  A rows (16 x 128 codes) and U (128 x rank of
// every matrix) reach LDS by direct global->LDS loads in a ring of two
// slots, 16-byte pieces swizzled so the operand reads spread over the banks:
// A piece p of row i at p ^ i, U piece j8 of row k at j8 ^ ((k / 8) % (rank / 8))
// (power-of-two ranks; others unswizzled).
__device__ void pf_lowrank_job(const PfLowrank& L, int job, int sp, unsigned char* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int sub = L.tile_rows / kLrRows;  // lowrank jobs per tile
  const int ti = job / sub, part = job % sub;
  int e = 0, p0, rows;
  if (L.tiles) {
    if (ti >= *L.ntiles) return;  // uniform over the workgroup
    e = L.tiles[3 * ti];
    p0 = L.tiles[3 * ti + 1] + part * kLrRows;
    rows = min(kLrRows, L.tiles[3 * ti + 2] - part * kLrRows);
  } else {
    p0 = job * kLrRows;
    rows = min(kLrRows, L.rows_total - p0);
  }
  if (rows <= 0) return;
  const int k0 = sp * L.kps, k1 = min(L.K, k0 + L.kps);
  const int r = L.rank, r8 = r / 8, nct = (r + 15) / 16;
  const int sw = (r8 & (r8 - 1)) == 0 ? r8 - 1 : 0;  // piece swizzle mask (power-of-two ranks)
  const int jobs = L.nmat * nct;  // (matrix, column tile)
  const int ub = 128 * r * 2;     // bytes of one matrix's U chunk
  const int slot_bytes = 4096 + L.nmat * ub;
  const __half* U[2];
  for (int m = 0; m < 2; ++m) {
    int c = (m < L.nmat && L.cluster[m]) ? L.cluster[m][e] : 0;
    if (m < L.nmat && L.uslot[m]) c = L.uslot[m][c];
    U[m] = m < L.nmat ? L.U[m] + (int64_t)c * L.u_cs : nullptr;
  }
  // A: wave w loads rows 4w..4w+3 (one instruction), lane -> (row, piece)
  const int arr = 4 * wave + (lane >> 4);
  const int apr = p0 + min(arr, rows - 1);
  const __half* asrc = L.x + (int64_t)(L.arow ? L.arow[apr] : apr) * L.K + 8 * ((lane & 15) ^ arr);
  const int nu = L.nmat * 128 * r8 / 64;  // U load instructions per workgroup
  auto issue = [&](int kc, unsigned char* slot) {
    __builtin_amdgcn_global_load_lds((const void*)(asrc + kc), (lds_void*)(slot + wave * 1024), 16,
                                     0, 0);
    for (int q = wave; q < nu; q += 4) {  // uniform over the wave
      const int pidx = q * 64 + lane;     // piece index over [m][k][pos]
      const int m = pidx / (128 * r8), rem = pidx - m * 128 * r8;
      const int k = rem / r8, pos = rem - k * r8;
      const int j8 = pos ^ ((k >> 3) & sw);
      const int kk = min(kc + k, L.K - 1);
      __builtin_amdgcn_global_load_lds((const void*)(U[m] + (int64_t)kk * r + 8 * j8),
                                       (lds_void*)(slot + 4096 + q * 1024), 16, 0, 0);
    }
  };
  constexpr int MJ = 8;  // jobs per wave (nmat * rank / 16 <= 32)
  f32x4 acc[MJ];
#pragma unroll
  for (int q = 0; q < MJ; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  issue(k0, smem);
  int s = 0;
  for (int kc = k0; kc < k1; kc += 128) {
    wait_vmcnt<0>();
    asm volatile("s_barrier" ::: "memory");
    if (kc + 128 < k1) issue(kc + 128, smem + (s ^ 1) * slot_bytes);
    const unsigned char* sl = smem + s * slot_bytes;
    const int kl = min(128, k1 - kc);
    for (int ks = 0; ks < kl; ks += 32) {
      const f16x8 av = *(const f16x8*)(sl + li * 256 + 16 * (((ks >> 3) + kb) ^ li));
#pragma unroll
      for (int q = 0; q < MJ; ++q) {
        const int jb = wave + 4 * q;
        if (jb >= jobs) break;  // uniform over the wave
        const int m = jb / nct, ct = jb - m * nct;
        const int j = min(ct * 16 + li, r - 1);
        const __half* um = (const __half*)(sl + 4096 + m * ub);
        f16x8 bv;
#pragma unroll
        for (int q8 = 0; q8 < 8; ++q8) {
          int k = ks + 8 * kb + q8;
          if (L.aperm) {  // position k of A holds natural index perm_src(k)
            const int p = k & 15;
            k = (k & ~15) + (L.aperm == 2 ? perm_src<2>(p) : perm_src<4>(p));
          }
          const int pos = (j >> 3) ^ ((k >> 3) & sw);
          const __half hv = um[k * r + 8 * pos + (j & 7)];
          bv[q8] = (_Float16)__half2float(hv);
        }
        acc[q] = mfma_16x16x32(av, bv, acc[q]);
      }
    }
    s ^= 1;
  }
  // acc[q][i]: row 4kb + i of the tile, rank column ct*16 + li
  const int ld = L.nmat * r;
  float* out = L.part + (int64_t)sp * L.rows_total * ld;
#pragma unroll
  for (int q = 0; q < MJ; ++q) {
    const int jb = wave + 4 * q;
    if (jb >= jobs) break;
    const int m = jb / nct, ct = jb - m * nct;
    const int j = ct * 16 + li;
    if (j >= r) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = 4 * kb + i;
      if (rr < rows) {
        const int64_t o = (int64_t)(p0 + rr) * ld + m * r + j;
        if (L.ks == 1) L.a_out[o] = __float2half(acc[q][i]);
        else out[o] = acc[q][i];
      }
    }
  }
}

// a = fp16(x U) of the dense prefill in one launch: workgroup (row block
// rb, K slice sp) forms the fp32 partial of 16 token rows over a slice of
// kLowrankRows codes (lowrank_partial<4>: v_mfma_f32_16x16x32_f16 tiles
// with U staged transposed in LDS), hands it over and counts itself in on
// the row block's counter (glq_handoff.h); the last of the block's slices
// sums them in slice order, rounds once and leaves the counter at zero.
__global__ __launch_bounds__(256) void pf_xu_kernel(const __half* __restrict__ x, int M, int K,
                                                    const __half* __restrict__ U, int rank,
                                                    int rpad, int ns, float* part,
                                                    unsigned* cnt, __half* __restrict__ a_out) {
  __shared__ float red[4 * 4 * 64];
  __shared__ __align__(16) __half xl[16 * kLowrankRows];
  __shared__ __align__(16) __half ut[64 * kLowrankUtStride];
  __shared__ int last;
  const int rb = blockIdx.x / ns, sp = blockIdx.x - rb * ns, tid = threadIdx.x;
  const int r0 = rb * 16, rows = min(16, M - r0);
  const __half* xb = x + (int64_t)r0 * K;
  auto xrow = [&](int m) { return xb + (int64_t)m * K; };
  float* slices = part + (int64_t)rb * ns * 16 * rpad;  // [slice][row][rpad]
  lowrank_partial<4, decltype(xrow), true>(xrow, rows, K, rank, rpad, U, sp,
                                           slices + (int64_t)sp * 16 * rpad, red, xl, tid, ut);
  if (!handoff_arrive(cnt + rb, (unsigned)ns, &last)) return;
  for (int i = tid; i < rows * rank; i += 256) {
    const int m = i / rank, j = i - m * rank;
    a_out[(int64_t)(r0 + m) * rank + j] =
        __float2half(sum_strided_coh(slices + m * rpad + j, 16 * rpad, ns));
  }
  if (tid == 0) handoff_reset(cnt + rb);
}

// Grid: n_jobs * ks lowrank jobs.
__global__ __launch_bounds__(kPfThreads) void pf_lowrank_kernel(PfLowrank L) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (L.zero_cnt && blockIdx.x == 0)
    for (int i = threadIdx.x; i < L.n_cnt; i += kPfThreads) L.zero_cnt[i] = 0u;
  if (L.nmat == 0) return;  // the counters were all there was to do
  const int j = blockIdx.x;
  pf_lowrank_job(L, j / L.ks, j % L.ks, smem);
}

// ---------------------------------------------------------------------------
// Host side shared by the dense GEMM and the MoE prefill
// ---------------------------------------------------------------------------

template <int BITS, int TM, int RT, int MODE, bool SYM, bool ZF, bool DEEP = false>
static int pf_launch_k(const PfArgs& g, hipStream_t s) {
  static size_t attr = 64 * 1024;
  using SL = PfSlot<BITS, TM, RT, DEEP>;
  size_t lds = (size_t)SL::D * SL::BYTES;
  if (g.xu_rows) lds = std::max(lds, kXuJobLds);  // the x U jobs and the epilogue's local form
  int rc = set_lds_limit(pf_gemm_kernel<BITS, TM, RT, MODE, SYM, ZF, DEEP>, lds, attr);
  if (rc) return rc;
  const dim3 grid((unsigned)(g.ntn * g.ks), (unsigned)(g.max_tiles + g.xu_rows));
  pf_gemm_kernel<BITS, TM, RT, MODE, SYM, ZF, DEEP><<<grid, dim3(kPfThreads), lds, s>>>(g);
  GLQ_LAUNCH_CHECK("pf_gemm_kernel");
  return GLQ_OK;
}

// Row tiles per wave for a token tile: the accumulators (2 x TM/16 x RT
// f32x4) and the codes must fit 256 VGPRs (two waves per SIMD).  The dense
// form (non-integer zero-point path compiled in) takes RT = 2 from 64
// tokens; the MoE forms RT = 4 below 128.
constexpr int pf_rt(int mode, int tm) {
  return tm == 128 ? 2 : (mode == kPfDense && tm == 64 ? 2 : 4);
}

// The dense form takes any symmetry and non-integer zero-points; the MoE
// forms asymmetric codes with integer zero-points.
template <int MODE, bool SYM, bool ZF>
static int pf_launch_shape(const PfArgs& g, int bits, int tm, hipStream_t s) {
  constexpr int R64 = pf_rt(MODE, 64);
  if (bits == 2) {
    if (tm == 128) return pf_launch_k<2, 128, 2, MODE, SYM, ZF>(g, s);
    if (tm == 64) return pf_launch_k<2, 64, R64, MODE, SYM, ZF>(g, s);
    return pf_launch_k<2, 32, 4, MODE, SYM, ZF>(g, s);
  }
  if (tm == 128) return pf_launch_k<4, 128, 2, MODE, SYM, ZF>(g, s);
  if (tm == 64) return pf_launch_k<4, 64, R64, MODE, SYM, ZF>(g, s);
  return pf_launch_k<4, 32, 4, MODE, SYM, ZF>(g, s);
}

// Tile of a dense launch: TM token rows x 64 RT weight rows, ring depth.
struct PfTile {
  int tm, rt;
  bool deep;
};

template <int BITS, bool SYM, bool ZF>
static int pf_launch_dense_bits(const PfArgs& g, PfTile t, hipStream_t s) {
  if (t.deep) {
    if (t.tm == 16) {
      if (t.rt == 1) return pf_launch_k<BITS, 16, 1, kPfDense, SYM, ZF, true>(g, s);
      return pf_launch_k<BITS, 16, 2, kPfDense, SYM, ZF, true>(g, s);
    }
    if (t.tm == 32) {
      if (t.rt == 1) return pf_launch_k<BITS, 32, 1, kPfDense, SYM, ZF, true>(g, s);
      return pf_launch_k<BITS, 32, 2, kPfDense, SYM, ZF, true>(g, s);
    }
    return pf_launch_k<BITS, 64, 2, kPfDense, SYM, ZF, true>(g, s);
  }
  if (t.tm == 128) return pf_launch_k<BITS, 128, 2, kPfDense, SYM, ZF>(g, s);
  if (t.tm == 64) return pf_launch_k<BITS, 64, 2, kPfDense, SYM, ZF>(g, s);
  return pf_launch_k<BITS, 32, 4, kPfDense, SYM, ZF>(g, s);
}

static int pf_launch_dense(const PfArgs& g, int bits, PfTile t, bool sym, hipStream_t s) {
  if (bits == 2) {
    return sym ? pf_launch_dense_bits<2, true, false>(g, t, s)
               : pf_launch_dense_bits<2, false, true>(g, t, s);
  }
  return sym ? pf_launch_dense_bits<4, true, false>(g, t, s)
             : pf_launch_dense_bits<4, false, true>(g, t, s);
}

// Weight rows per workgroup for a token tile.
static int pf_wg_rows_rt(int mode, int tm) {
  const int rt = pf_rt(mode, tm);
  return mode == kPfGateUp ? 4 * 8 * rt : 4 * 16 * rt;
}

static size_t pf_lowrank_lds(int nmat, int rank) {
  return 2 * (4096 + (size_t)nmat * 128 * rank * 2);
}

// a = fp16(sum of the K-split partials in split order): one thread per element.
__global__ __launch_bounds__(256) void pf_lowrank_finalize_kernel(const float* part, int ks,
                                                                  int64_t n, __half* a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int q = 0; q < ks; ++q) s += part[q * n + i];
  a[i] = __float2half(s);
}

// n_jobs: 16-row lowrank jobs (times L.ks splits); with none, one workgroup
// still clears L.zero_cnt.
static int pf_lowrank_launch(const PfLowrank& L, int n_jobs, hipStream_t s) {
  static size_t attr = 64 * 1024;
  const size_t lds = L.nmat > 0 ? pf_lowrank_lds(L.nmat, L.rank) : 0;
  int rc = set_lds_limit(pf_lowrank_kernel, lds, attr);
  if (rc) return rc;
  int64_t grid = L.nmat > 0 ? (int64_t)n_jobs * L.ks : 0;
  if (grid == 0 && L.zero_cnt) grid = 1;  // the job index is past the list: no job
  if (grid == 0) return GLQ_OK;
  GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
  pf_lowrank_kernel<<<dim3((unsigned)grid), dim3(kPfThreads), lds, s>>>(L);
  GLQ_LAUNCH_CHECK("pf_lowrank_kernel");
  if (L.nmat > 0 && L.ks > 1) {
    const int64_t n = (int64_t)L.rows_total * L.nmat * L.rank;
    pf_lowrank_finalize_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(
        L.part, L.ks, n, L.a_out);
    GLQ_LAUNCH_CHECK("pf_lowrank_finalize_kernel");
  }
  return GLQ_OK;
}

// K split of a = x U: splits of 512 codes (more for K > 8192: at most 16
// splits), summed by pf_lowrank_finalize_kernel.
static void pf_lowrank_split(int64_t K, int& ks, int& kps) {
  int64_t per = std::max<int64_t>(512, (K + 15) / 16);
  per = (per + 127) / 128 * 128;
  kps = (int)per;
  ks = (int)((K + per - 1) / per);
}

// ---------------------------------------------------------------------------
// Dense plan: token tile, K splits and workspace of one projection.
// ---------------------------------------------------------------------------
struct PfDensePlan {
  int tm, rt, ntn, ntm, ks, gps, lr_ks, lr_kps;
  bool deep;
  bool xu1;          // a = x U by pf_xu_kernel (one launch)
  int xu_ns;         // its K slices
  int64_t a_bytes, lp_bytes, part_bytes, cnt_bytes, total;
};

// The dense prefill workspace starts with kPfSyncBytes of counter words (the
// x U row blocks' arrivals), zero before the first call and after every
// call, so the one-launch x U takes at most kPfSyncBytes / 4 row blocks.
constexpr int64_t kPfSyncBytes = 4096;

static PfDensePlan pf_dense_plan(int64_t M, int64_t K, int64_t N, int64_t rank, int bits) {
  PfDensePlan P;
  // Big launches (a 64 x 128 tile per CU or more): 64-token tiles, shallow
  // rings, two workgroups per CU.  Smaller ones: 32-token tiles of
  // 128 rows from 256 tokens, else 16-token tiles of 64 rows, with deep rings
  // (the whole K range of a small tile nearly in flight).  No K split: the
  // tiles are sized to give the chip enough workgroups without one.
  const int64_t t64 = ((M + 63) / 64) * ((N + 127) / 128);
  if (t64 >= 256) {
    // (64-token tiles: the 128-token tile of asymmetric codes needs more
    // than 256 VGPRs and spills)
    P.tm = 64;
    P.rt = 2;
    P.deep = false;
  } else if (M >= 256) {
    P.tm = 32;
    P.rt = 2;
    P.deep = true;
  } else {
    P.tm = 16;
    P.rt = 1;
    P.deep = true;
  }
  if (const char* e = getenv("GLQ_PF_CFG")) {  // "tm,rt,deep": a supported tile
    int tm = 0, rt = 0, deep = 0;
    if (sscanf(e, "%d,%d,%d", &tm, &rt, &deep) == 3) {
      const bool ok = deep ? ((tm == 16 || tm == 32) && (rt == 1 || rt == 2)) || (tm == 64 && rt == 2)
                           : (tm == 32 && rt == 4) || ((tm == 64 || tm == 128) && rt == 2);
      if (ok) {
        P.tm = tm;
        P.rt = rt;
        P.deep = deep != 0;
      }
    }
  }
  const int wgr = 64 * P.rt;
  P.ntn = (int)((N + wgr - 1) / wgr);
  P.ntm = (int)((M + P.tm - 1) / P.tm);
  const int G = (int)(K / 128);
  int ks = 1;
  if (const char* e = getenv("GLQ_PF_KS")) ks = std::max(1, std::min(G, atoi(e)));
  P.gps = (G + ks - 1) / ks;
  P.ks = (G + P.gps - 1) / P.gps;
  pf_lowrank_split(K, P.lr_ks, P.lr_kps);
  P.a_bytes = rank > 0 ? align_up(M * rank * 2, 256) : 0;
  // a = x U in one launch (16-row blocks x K slices, last arrivers sum) when
  // the GEMM needs no split-K counters (those are cleared by the two-launch
  // form's first launch)
  const int64_t nrb = (M + 15) / 16;
  P.xu_ns = (int)((K + kLowrankRows - 1) / kLowrankRows);
  P.xu1 = rank > 0 && rank <= 128 && P.ks == 1 && nrb <= kPfSyncBytes / 4 &&
          !getenv("GLQ_PF_XU2");
  if (P.xu1) {
    const int64_t rpad = align_up(rank, 32);
    P.lp_bytes = align_up(nrb * P.xu_ns * 16 * rpad * 4, 256);
  } else {
    P.lp_bytes = rank > 0 && P.lr_ks > 1 ? align_up((int64_t)P.lr_ks * M * rank * 4, 256) : 0;
  }
  P.part_bytes = P.ks > 1 ? align_up((int64_t)P.ks * P.ntm * P.tm * P.ntn * 64 * P.rt * 4, 256)
                          : 0;
  P.cnt_bytes = P.ks > 1 ? align_up((int64_t)P.ntm * P.ntn * 4, 256) : 0;
  // the counter words come first in every workspace this path uses, so no
  // call's tables overwrite another's counters
  const int64_t body = P.a_bytes + P.lp_bytes + P.part_bytes + P.cnt_bytes;
  P.total = body ? kPfSyncBytes + body : 0;
  return P;
}

// Workspace of the prefill path of glq_gemm_lora: kPfSyncBytes of counter
// words (zero before the first call, left zero by every call), then a, its
// partials, the split-K tiles (whose arrival counters the two-launch form's
// first launch clears); none at all when the call needs no tables.
int64_t pf_gemm_prefill_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank,
                                        int bits) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (rank < 0) return -1;
  return pf_dense_plan(M, K, N, rank, bits).total;
}

// The prefill GEMM of glq_gemm_lora (called after its argument checks).
int pf_dense_gemm(const void* x, int64_t M, int64_t K, int64_t N, const int32_t* codes,
                  int bits, const void* scales, const void* zeros, int sym, const void* U,
                  const void* SV, int64_t rank, const void* xU, const void* bias, void* y,
                  void* workspace, int64_t workspace_bytes, hipStream_t s) {
  const bool lora = SV != nullptr && rank > 0;
  // a = x U needs room only when it is formed here
  const PfDensePlan P = pf_dense_plan(M, K, N, lora && xU == nullptr ? rank : 0, bits);
  GLQ_CHECK(P.total == 0 || (workspace != nullptr && workspace_bytes >= P.total),
            "workspace of %lld bytes needed (got %lld)", (long long)P.total,
            (long long)workspace_bytes);
  GLQ_CHECK(M * K < (1ll << 31), "M*K too large for the prefill path");
  unsigned* xcnt = (unsigned*)workspace;  // zero between calls
  char* w = (char*)workspace + (P.total ? kPfSyncBytes : 0);
  __half* abuf = P.a_bytes ? (__half*)w : nullptr;
  float* lpart = P.lp_bytes ? (float*)(w + P.a_bytes) : nullptr;
  char* w3 = w + P.a_bytes + P.lp_bytes;
  float* part = P.ks > 1 ? (float*)w3 : nullptr;
  unsigned* cnt = P.ks > 1 ? (unsigned*)(w3 + P.part_bytes) : nullptr;
  const bool fused = P.xu1 && xU == nullptr && !getenv("GLQ_PF_XU1");
  if (fused) {
    // a = x U in the GEMM's launch (its first grid rows)
  } else if (P.xu1 && xU == nullptr) {
    // launch 1: a = x U in one launch (its row blocks count on the
    // workspace's first words)
    const int nrb = (int)((M + 15) / 16);
    pf_xu_kernel<<<dim3((unsigned)(nrb * P.xu_ns)), dim3(256), 0, s>>>(
        (const __half*)x, (int)M, (int)K, (const __half*)U, (int)rank,
        (int)align_up(rank, 32), P.xu_ns, lpart, xcnt, abuf);
    GLQ_LAUNCH_CHECK("pf_xu_kernel");
  } else if (P.a_bytes || cnt) {
    // launch 1 (when U is given, or split-K counters need clearing): the split
    // partials of a = x U, summed by a finalize launch
    PfLowrank L = {};
    L.x = (const __half*)x;
    L.aperm = 0;
    L.nmat = P.a_bytes ? 1 : 0;
    L.U[0] = (const __half*)U;
    L.u_cs = 0;
    L.tile_rows = kLrRows;
    L.rows_total = (int)M;
    L.K = (int)K;
    L.rank = L.nmat ? (int)rank : 8;
    L.ks = P.lr_ks;
    L.kps = P.lr_kps;
    L.part = lpart;
    L.a_out = abuf;
    L.zero_cnt = cnt;  // the GEMM's split-K counters start at zero
    L.n_cnt = P.ntm * P.ntn;
    int rc = pf_lowrank_launch(L, (int)((M + kLrRows - 1) / kLrRows), s);
    if (rc) return rc;
  }
  // launch 2: the GEMM, A = x in natural order
  PfArgs g = {};
  g.xp = (const __half*)x;
  g.codes[0] = (const uint32_t*)codes;
  g.scales[0] = (const __half*)scales;
  g.zeros[0] = (const __half*)zeros;
  g.a = lora ? (xU ? (const __half*)xU : abuf) : nullptr;
  g.a_ld = (int)rank;
  g.sv[0] = lora ? (const __half*)SV : nullptr;
  g.bias = (const __half*)bias;
  g.y = (__half*)y;
  g.y_ld = N;
  g.part = part;
  g.cnt = cnt;
  g.M = (int)M;
  g.K = (int)K;
  g.N = (int)N;
  g.G = (int)(K / 128);
  g.kw = (int)(K * bits / 32);
  g.rank = lora ? (int)rank : 0;
  g.ntn = P.ntn;
  g.ks = P.ks;
  g.gps = P.gps;
  g.max_tiles = P.ntm;
  g.zoff = sym == 2 ? (float)(1 << (bits - 1)) : 0.f;
  if (fused) {
    g.xu_nrb = (int)((M + 15) / 16);
    g.xu_ns = P.xu_ns;
    g.xu_rows = (int)((g.xu_nrb * g.xu_ns + g.ntn * g.ks - 1) / (g.ntn * g.ks));
    g.xu_rpad = (int)align_up(rank, 32);
    g.xu_u = (const __half*)U;
    g.xu_part = lpart;
    g.xu_cnt = xcnt;
    // GLQ_PF_SPIN_TICKS: the epilogue's wait bound (tests set 0 to take the
    // local form)
    const char* e = getenv("GLQ_PF_SPIN_TICKS");
    g.xu_spin = e ? (uint64_t)strtoull(e, nullptr, 10) : 100000;  // 1 ms
  }
  return pf_launch_dense(g, bits, PfTile{P.tm, P.rt, P.deep}, sym == 1, s);
}
}  // namespace glq

namespace glq {

// ===========================================================================
// MoE block over many tokens (glq_moe_prefill): the reference's
// _forward_sparse (inference/moe_block.py:704-740) semantics -- route every
// token, gather each active expert's tokens, run its SwiGLU projections on
// them, weight and sum -- with the decode step's routing and combine
// arithmetic (glq_moe.hip), so a prompt and a decode step of the same tokens
// agree.
//   1. pf_moe_route_kernel     logits (MFMA, fp32 sums rounded once), softmax,
//                              top-k, weights, the shared-expert gate, and x in
//                              the decode order(s) of the GEMMs
//   2. pf_moe_dispatch_kernel  per-expert counts and positions: the pairs
//                              (token, pick) sorted by expert, and the list of
//                              TM-row tiles (expert, first row, rows)
//   3. pf_lowrank_kernel (+ finalize)  a = x U_c(e) for gate and up per pair
//   4. pf_gemm_kernel GATE/UP  inter = SwiGLU per pair (down's decode order)
//   5. pf_lowrank_kernel (+ finalize)  a = inter U_down,c(e) per pair
//   6. pf_gemm_kernel DOWN     y per pair (fp32)
//   7. shared expert (dense GATE/UP, DOWN over all tokens), when present
//   8. pf_moe_combine_kernel   out = fp16(sum_k w_k y_k + sg fp16(shared))
//                              (+ residual)
// Rows within an expert come in the order of an atomic counter, but every
// row's results depend on that row alone, so the output is the same on
// every run.
// ===========================================================================
struct PfMoe {
  int T, H, E, I, topk, norm, SI, bits, sbits, tm, max_tiles;
  const __half* h;
  const __half* router_w;  // (E, H)
  const __half* sgw;       // (H,) or null
  __half* logits_out;      // (T, E) or null
  __half* xp;              // (T, H) in the routed experts' decode order
  __half* xps;             // (T, H) in the shared expert's decode order (may alias xp)
  int32_t* sel;            // (T * topk) expert of each pick
  __half* wts;             // (T * topk)
  __half* sg;              // (T,) sigmoid(shared gate logit)
  int32_t* pos;            // (T * topk) sorted row of each pick
  int32_t* stok;           // (T * topk) token of each sorted row
  int32_t* tiles;          // (max_tiles, 3)
  int32_t* ntiles;
  const float* ybuf;       // (T * topk, H) routed outputs per sorted row
  const float* sy;         // (T, H) shared expert output, or null
  const __half* res;       // (T, H) residual or null
  __half* out;             // (T, H)
};

// One workgroup per 16 tokens: logits of every router row (MFMA tiles of 16
// rows, K split over the waves, partial tiles summed in LDS in wave order),
// then per token (one wave) softmax, top-k with ties to the lower index,
// weights, and the rows of x in decode order.
__global__ __launch_bounds__(256) void pf_moe_route_kernel(PfMoe a) {
  __shared__ float red[4][16][17];  // per wave partial logits of one 16-row tile
  __shared__ float lg[16][257];     // fp16-rounded logits (as float) of the 16 tokens
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int t0 = blockIdx.x * 16;
  const int nrow = a.E + (a.sgw ? 1 : 0), ntile = (nrow + 15) / 16;
  const int ta = min(t0 + li, a.T - 1);
  const int nks = a.H / 32;
  for (int tile = 0; tile < ntile; ++tile) {
    const int row = tile * 16 + li;
    const __half* wr = row < a.E ? a.router_w + (int64_t)row * a.H
                                 : (row == a.E && a.sgw ? a.sgw : nullptr);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int ks = wave; ks < nks; ks += 4) {
      const f16x8 av = *(const f16x8*)(a.h + (int64_t)ta * a.H + 32 * ks + 8 * kb);
      const f16x8 bv = wr ? *(const f16x8*)(wr + 32 * ks + 8 * kb) : f16x8{};
      acc = mfma_16x16x32(av, bv, acc);
    }
    // acc[i]: token 4kb + i, router row li of the tile
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * kb + i][li] = acc[i];
    __syncthreads();
    {
      const int t = tid >> 4, c = tid & 15;
      const float s = red[0][t][c] + red[1][t][c] + red[2][t][c] + red[3][t][c];
      if (tile * 16 + c < nrow) lg[t][tile * 16 + c] = __half2float(__float2half(s));
    }
    __syncthreads();
  }
  // x rows in decode order (and in the shared expert's when it differs)
  for (int idx = tid; idx < 16 * (a.H / 16); idx += 256) {
    const int t = idx / (a.H / 16), blk = idx - t * (a.H / 16);
    if (t0 + t >= a.T) continue;
    const __half* src = a.h + (int64_t)(t0 + t) * a.H + 16 * blk;
    const f16x8 a0 = *(const f16x8*)src, a1 = *(const f16x8*)(src + 8);
    _Float16 in[16];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      in[c] = a0[c];
      in[8 + c] = a1[c];
    }
    for (int which = 0; which < 2; ++which) {
      const int bits = which == 0 ? a.bits : a.sbits;
      __half* dstb = which == 0 ? a.xp : a.xps;
      if (which == 1 && (dstb == nullptr || dstb == a.xp)) break;
      f16x8 o0, o1;
#pragma unroll
      for (int pos = 0; pos < 8; ++pos) {
        o0[pos] = in[bits == 2 ? perm_src<2>(pos) : perm_src<4>(pos)];
        o1[pos] = in[bits == 2 ? perm_src<2>(pos + 8) : perm_src<4>(pos + 8)];
      }
      __half* dst = dstb + (int64_t)(t0 + t) * a.H + 16 * blk;
      *(f16x8*)dst = o0;
      *(f16x8*)(dst + 8) = o1;
    }
  }
  // routing, one wave per token
  for (int t = wave; t < 16; t += 4) {
    const int tok = t0 + t;
    if (tok >= a.T) continue;
    if (a.logits_out)
      for (int e = lane; e < a.E; e += 64)
        a.logits_out[(int64_t)tok * a.E + e] = __float2half(lg[t][e]);
    if (a.sgw && lane == 0) a.sg[tok] = __float2half(1.f / (1.f + expf(-lg[t][a.E])));
    // top-k: k rounds of the largest (logit, then lower index) not yet taken
    uint32_t taken[4] = {0u, 0u, 0u, 0u};  // experts lane + 64 q taken
    float mx = 0.f, wsel = 0.f;
    int esel = 0;
    for (int j = 0; j < a.topk; ++j) {
      float bv = -__builtin_inff();
      int be = 0x7fffffff;
      for (int q = 0; q < 4; ++q) {
        const int e = lane + 64 * q;
        if (e < a.E && !taken[q]) {
          const float v = lg[t][e];
          if (v > bv) { bv = v; be = e; }  // e ascending within a lane
        }
      }
      // wave argmax: larger value, then lower index
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oe = __shfl_xor(be, o);
        if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
      }
      if ((be & 63) == lane) taken[be >> 6] = 1u;
      if (j == 0) mx = bv;
      if (lane == j) { esel = be; wsel = bv; }
    }
    float sum = 0.f;
    for (int e = lane; e < a.E; e += 64) sum += expf(lg[t][e] - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    const float w = lane < a.topk ? expf(wsel - mx) / sum : 0.f;
    float ws = 0.f;
    if (a.norm)
      for (int j = 0; j < a.topk; ++j) ws += __shfl(w, j);
    if (lane < a.topk) {
      a.sel[(int64_t)tok * a.topk + lane] = esel;
      a.wts[(int64_t)tok * a.topk + lane] = __float2half(a.norm ? w / ws : w);
    }
  }
}

// One workgroup: per-expert counts, offsets, each pick's sorted row, the token
// of each sorted row, and the tile list.
__global__ __launch_bounds__(1024) void pf_moe_dispatch_kernel(PfMoe a) {
  __shared__ int cnt[256], off[256], cur[256], tb[257];
  const int tid = threadIdx.x, P = a.T * a.topk;
  for (int e = tid; e < a.E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += 1024) atomicAdd(&cnt[a.sel[p]], 1);
  __syncthreads();
  if (tid == 0) {
    int o = 0, tt = 0;
    for (int e = 0; e < a.E; ++e) {
      off[e] = o;
      cur[e] = o;
      tb[e] = tt;
      o += cnt[e];
      tt += (cnt[e] + a.tm - 1) / a.tm;
    }
    tb[a.E] = tt;
    *a.ntiles = tt;
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int e = a.sel[p];
    const int r = atomicAdd(&cur[e], 1);
    a.pos[p] = r;
    a.stok[r] = p / a.topk;
  }
  for (int e = tid; e < a.E; e += 1024) {
    const int n = (cnt[e] + a.tm - 1) / a.tm;
    for (int i = 0; i < n; ++i) {
      int32_t* tl = a.tiles + 3 * (tb[e] + i);
      tl[0] = e;
      tl[1] = off[e] + i * a.tm;
      tl[2] = min(a.tm, cnt[e] - i * a.tm);
    }
  }
}

// out[t][n] = fp16(sum_k w_k y[pos(t, k)][n] + sg[t] fp16(shared[t][n])),
// then fp16(residual + out): the decode step's combine (glq_moe.hip).
__global__ __launch_bounds__(256) void pf_moe_combine_kernel(PfMoe a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.T * a.H) return;
  const int t = (int)(i / a.H), n = (int)(i - (int64_t)t * a.H);
  float acc = 0.f;
  for (int k = 0; k < a.topk; ++k) {
    const int p = t * a.topk + k;
    acc = fmaf(__half2float(a.wts[p]), a.ybuf[(int64_t)a.pos[p] * a.H + n], acc);
  }
  if (a.sy) acc = fmaf(__half2float(a.sg[t]), __half2float(__float2half(a.sy[i])), acc);
  float o = __half2float(__float2half(acc));
  if (a.res) o += __half2float(a.res[i]);
  a.out[i] = __float2half(o);
}

// ---------------------------------------------------------------------------
// Host plan of glq_moe_prefill
// ---------------------------------------------------------------------------
struct PfMoePlan {
  int tm, max_tiles, ks_gu, kps_gu, ks_d, kps_d, stm;
  int64_t off_xp, off_xps, off_sel, off_wts, off_sg, off_pos, off_stok, off_tiles, off_lp,
      off_agu, off_ad, off_inter, off_y, off_sinter, off_sy, total;
};

static PfMoePlan pf_moe_plan(int64_t T, int64_t H, int64_t E, int64_t I, int64_t k,
                             int64_t rank, int64_t SI, int bits, int sbits) {
  PfMoePlan P;
  const int64_t Pn = T * k;
  const int64_t avg = Pn / std::max<int64_t>(E, 1);
  P.tm = avg >= 96 ? 128 : (avg >= 32 ? 64 : 32);
  if (const char* e = getenv("GLQ_PF_MOE_TM")) {
    const int v = atoi(e);
    P.tm = v >= 128 ? 128 : (v >= 64 ? 64 : 32);
  }
  P.max_tiles = (int)((Pn + P.tm - 1) / P.tm + E);
  pf_lowrank_split(H, P.ks_gu, P.kps_gu);
  pf_lowrank_split(I, P.ks_d, P.kps_d);
  P.stm = T >= 512 ? 128 : (T > 32 ? 64 : 32);
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  P.off_xp = take(T * H * 2);
  P.off_xps = (SI > 0 && sbits != bits) ? take(T * H * 2) : P.off_xp;
  P.off_sel = take(Pn * 4);
  P.off_wts = take(Pn * 2);
  P.off_sg = take(T * 2);
  P.off_pos = take(Pn * 4);
  P.off_stok = take(Pn * 4);
  P.off_tiles = take((int64_t)P.max_tiles * 12 + 4);
  const int64_t lp = rank > 0 ? std::max<int64_t>(P.ks_gu > 1 ? P.ks_gu * Pn * 2 * rank * 4 : 0,
                                                  P.ks_d > 1 ? P.ks_d * Pn * rank * 4 : 0)
                              : 0;
  P.off_lp = take(lp);
  P.off_agu = take(rank > 0 ? Pn * 2 * rank * 2 : 0);
  P.off_ad = take(rank > 0 ? Pn * rank * 2 : 0);
  P.off_inter = take(Pn * I * 2);
  P.off_y = take(Pn * H * 4);
  P.off_sinter = take(SI > 0 ? T * SI * 2 : 0);
  P.off_sy = take(SI > 0 ? T * H * 4 : 0);
  P.total = o;
  return P;
}

static int pf_moe_check(const glq_moe_params* p) {
  GLQ_CHECK(p != nullptr, "null params");
  const int64_t T = p->tokens, H = p->hidden, E = p->experts, I = p->inter, k = p->top_k;
  GLQ_CHECK(T >= 1 && T <= (1 << 20), "tokens=%lld must be in 1..%d", (long long)T, 1 << 20);
  GLQ_CHECK(E >= 1 && E <= 256, "experts=%lld must be in 1..256", (long long)E);
  GLQ_CHECK(k >= 1 && k <= 16 && k <= E && k <= 64, "top_k=%lld out of range", (long long)k);
  GLQ_CHECK(p->group == 128, "group must be 128 (got %d)", p->group);
  GLQ_CHECK(p->bits == 2 || p->bits == 4, "bits must be 2 or 4");
  GLQ_CHECK(H >= 128 && H % 128 == 0 && H <= (1 << 16), "hidden=%lld must be a multiple of 128",
            (long long)H);
  GLQ_CHECK(I >= 128 && I % 128 == 0 && I <= (1 << 17), "inter=%lld must be a multiple of 128",
            (long long)I);
  GLQ_CHECK(T * H < (1ll << 31) && T * k * std::max(I, H) < (1ll << 31), "tokens x width too large");
  const int64_t SI = p->shared_inter;
  GLQ_CHECK(SI >= 0 && SI % 128 == 0 && SI <= (1 << 17), "shared_inter=%lld must be a multiple of 128",
            (long long)SI);
  if (SI > 0) GLQ_CHECK(p->shared_bits == 2 || p->shared_bits == 4, "shared_bits must be 2 or 4");
  const int64_t r = p->rank;
  const bool lora = r > 0 && p->SV[0] != nullptr;
  if (lora) {
    GLQ_CHECK(r % 8 == 0 && r <= 128, "rank=%lld must be a multiple of 8, <= 128", (long long)r);
    for (int s = 0; s < 3; ++s)
      GLQ_CHECK(p->U[s] && p->cluster_of[s] && p->SV[s], "U, cluster_of and SV are needed with a rank");
  }
  GLQ_CHECK(p->h && p->router_w && p->out, "null h, router_w or out");
  for (int s = 0; s < 3; ++s) {
    GLQ_CHECK(p->codes[s] && p->scales[s] && p->zeros[s], "null routed weights (proj %d)", s);
    if (SI > 0)
      GLQ_CHECK(p->shared_codes[s] && p->shared_scales[s] && p->shared_zeros[s],
                "null shared-expert weights (proj %d)", s);
  }
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  GLQ_CHECK(al16(p->h) && al16(p->router_w) && (!p->shared_gate_w || al16(p->shared_gate_w)),
            "h, router_w and shared_gate_w must be 16-byte aligned");
  for (int s = 0; s < 3; ++s)
    GLQ_CHECK(al16(p->codes[s]) && (!lora || (al16(p->U[s]) && al16(p->SV[s]))),
              "codes, U and SV must be 16-byte aligned");
  return GLQ_OK;
}

}  // namespace glq

extern "C" int64_t glq_moe_prefill_workspace_bytes(const glq_moe_params* p) {
  using namespace glq;
  clear_error();
  if (pf_moe_check(p) != GLQ_OK) return -1;
  const bool lora = p->rank > 0 && p->SV[0] != nullptr;
  return pf_moe_plan(p->tokens, p->hidden, p->experts, p->inter, p->top_k, lora ? p->rank : 0,
                     p->shared_inter, p->bits, p->shared_bits)
      .total;
}

extern "C" int glq_moe_prefill(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  using namespace glq;
  clear_error();
  int rc = pf_moe_check(p);
  if (rc) return rc;
  const int64_t T = p->tokens, H = p->hidden, E = p->experts, I = p->inter, k = p->top_k;
  const int64_t SI = p->shared_inter, Pn = T * k;
  const bool lora = p->rank > 0 && p->SV[0] != nullptr;
  const int r = lora ? (int)p->rank : 0;
  const PfMoePlan P = pf_moe_plan(T, H, E, I, k, r, SI, p->bits, p->shared_bits);
  GLQ_CHECK(workspace != nullptr && workspace_bytes >= P.total && ((uintptr_t)workspace & 255) == 0,
            "a 256-byte aligned workspace of %lld bytes is needed (got %lld)", (long long)P.total,
            (long long)workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  char* w = (char*)workspace;
  PfMoe a = {};
  a.T = (int)T; a.H = (int)H; a.E = (int)E; a.I = (int)I; a.topk = (int)k;
  a.norm = p->norm_topk_prob ? 1 : 0;
  a.SI = (int)SI; a.bits = p->bits; a.sbits = SI > 0 ? p->shared_bits : p->bits;
  a.tm = P.tm; a.max_tiles = P.max_tiles;
  a.h = (const __half*)p->h;
  a.router_w = (const __half*)p->router_w;
  a.sgw = (const __half*)p->shared_gate_w;
  a.logits_out = (__half*)p->router_logits;
  a.xp = (__half*)(w + P.off_xp);
  a.xps = (__half*)(w + P.off_xps);
  a.sel = (int32_t*)(w + P.off_sel);
  a.wts = (__half*)(w + P.off_wts);
  a.sg = (__half*)(w + P.off_sg);
  a.pos = (int32_t*)(w + P.off_pos);
  a.stok = (int32_t*)(w + P.off_stok);
  a.tiles = (int32_t*)(w + P.off_tiles);
  a.ntiles = a.tiles + 3 * P.max_tiles;
  a.ybuf = (const float*)(w + P.off_y);
  a.sy = SI > 0 ? (const float*)(w + P.off_sy) : nullptr;
  a.res = (const __half*)p->residual;
  a.out = (__half*)p->out;
  __half* inter = (__half*)(w + P.off_inter);
  float* ybuf = (float*)(w + P.off_y);
  __half* agu = (__half*)(w + P.off_agu);
  __half* ad = (__half*)(w + P.off_ad);
  float* lp = (float*)(w + P.off_lp);

  // 1-2. routing and dispatch
  pf_moe_route_kernel<<<dim3((unsigned)((T + 15) / 16)), dim3(256), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("pf_moe_route_kernel");
  pf_moe_dispatch_kernel<<<dim3(1), dim3(1024), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("pf_moe_dispatch_kernel");

  // expert strides (elements)
  const int64_t kw_gu = H * p->bits / 32, kw_d = I * p->bits / 32;
  // 3. a = x U for gate and up per pair
  if (lora) {
    PfLowrank L = {};
    L.x = a.xp;
    L.arow = a.stok;
    L.aperm = p->bits;
    L.nmat = 2;
    for (int m = 0; m < 2; ++m) {
      L.U[m] = (const __half*)p->U[m];
      L.cluster[m] = p->cluster_of[m];
      L.uslot[m] = p->u_slot[m];
    }
    L.u_cs = H * r;
    L.tiles = a.tiles;
    L.ntiles = a.ntiles;
    L.tile_rows = P.tm;
    L.rows_total = (int)Pn;
    L.K = (int)H;
    L.rank = r;
    L.ks = P.ks_gu;
    L.kps = P.kps_gu;
    L.part = lp;
    L.a_out = agu;
    rc = pf_lowrank_launch(L, P.max_tiles * (P.tm / kLrRows), s);
    if (rc) return rc;
  }
  // 4. gate/up + SwiGLU -> inter (rows sorted by expert, down's decode order)
  {
    PfArgs g = {};
    g.xp = a.xp;
    g.arow = a.stok;
    for (int m = 0; m < 2; ++m) {
      g.codes[m] = (const uint32_t*)p->codes[m];
      g.scales[m] = (const __half*)p->scales[m];
      g.zeros[m] = (const __half*)p->zeros[m];
      g.sv[m] = lora ? (const __half*)p->SV[m] : nullptr;
    }
    g.codes_es = I * kw_gu;
    g.sz_es = I * (H / 128);
    g.a = lora ? agu : nullptr;
    g.a_ld = 2 * r;
    g.sv_es = I * r;
    g.y = inter;
    g.y_ld = I;
    g.tiles = a.tiles;
    g.ntiles = a.ntiles;
    g.M = (int)Pn; g.K = (int)H; g.N = (int)I; g.G = (int)(H / 128);
    g.kw = (int)kw_gu; g.rank = r;
    g.ntn = (int)((I + pf_wg_rows_rt(kPfGateUp, P.tm) - 1) / pf_wg_rows_rt(kPfGateUp, P.tm));
    g.ks = 1; g.gps = g.G;
    g.out_bits = p->bits;
    g.max_tiles = P.max_tiles;
    rc = pf_launch_shape<kPfGateUp, false, false>(g, p->bits, P.tm, s);
    if (rc) return rc;
  }
  // 5. a = inter U_down per pair
  if (lora) {
    PfLowrank L = {};
    L.x = inter;
    L.aperm = p->bits;
    L.nmat = 1;
    L.U[0] = (const __half*)p->U[2];
    L.cluster[0] = p->cluster_of[2];
    L.u_cs = I * r;
    L.tiles = a.tiles;
    L.ntiles = a.ntiles;
    L.tile_rows = P.tm;
    L.rows_total = (int)Pn;
    L.K = (int)I;
    L.rank = r;
    L.ks = P.ks_d;
    L.kps = P.kps_d;
    L.part = lp;
    L.a_out = ad;
    rc = pf_lowrank_launch(L, P.max_tiles * (P.tm / kLrRows), s);
    if (rc) return rc;
  }
  // 6. down -> y per sorted row (fp32)
  {
    PfArgs g = {};
    g.xp = inter;
    g.codes[0] = (const uint32_t*)p->codes[2];
    g.scales[0] = (const __half*)p->scales[2];
    g.zeros[0] = (const __half*)p->zeros[2];
    g.sv[0] = lora ? (const __half*)p->SV[2] : nullptr;
    g.codes_es = H * kw_d;
    g.sz_es = H * (I / 128);
    g.a = lora ? ad : nullptr;
    g.a_ld = r;
    g.sv_es = H * r;
    g.yf = ybuf;
    g.yf_ld = H;
    g.tiles = a.tiles;
    g.ntiles = a.ntiles;
    g.M = (int)Pn; g.K = (int)I; g.N = (int)H; g.G = (int)(I / 128);
    g.kw = (int)kw_d; g.rank = r;
    g.ntn = (int)((H + pf_wg_rows_rt(kPfDown, P.tm) - 1) / pf_wg_rows_rt(kPfDown, P.tm));
    g.ks = 1; g.gps = g.G;
    g.max_tiles = P.max_tiles;
    rc = pf_launch_shape<kPfDown, false, false>(g, p->bits, P.tm, s);
    if (rc) return rc;
  }
  // 7. shared expert over every token
  if (SI > 0) {
    const int sb = p->shared_bits;
    __half* sinter = (__half*)(w + P.off_sinter);
    const int ntm = (int)((T + P.stm - 1) / P.stm);
    PfArgs g = {};
    g.xp = a.xps;
    for (int m = 0; m < 2; ++m) {
      g.codes[m] = (const uint32_t*)p->shared_codes[m];
      g.scales[m] = (const __half*)p->shared_scales[m];
      g.zeros[m] = (const __half*)p->shared_zeros[m];
    }
    g.y = sinter;
    g.y_ld = SI;
    g.M = (int)T; g.K = (int)H; g.N = (int)SI; g.G = (int)(H / 128);
    g.kw = (int)(H * sb / 32);
    g.ntn = (int)((SI + pf_wg_rows_rt(kPfGateUp, P.stm) - 1) / pf_wg_rows_rt(kPfGateUp, P.stm));
    g.ks = 1; g.gps = g.G;
    g.out_bits = sb;
    g.max_tiles = ntm;
    rc = pf_launch_shape<kPfGateUp, false, false>(g, sb, P.stm, s);
    if (rc) return rc;
    PfArgs d = {};
    d.xp = sinter;
    d.codes[0] = (const uint32_t*)p->shared_codes[2];
    d.scales[0] = (const __half*)p->shared_scales[2];
    d.zeros[0] = (const __half*)p->shared_zeros[2];
    d.yf = (float*)(w + P.off_sy);
    d.yf_ld = H;
    d.M = (int)T; d.K = (int)SI; d.N = (int)H; d.G = (int)(SI / 128);
    d.kw = (int)(SI * sb / 32);
    d.ntn = (int)((H + pf_wg_rows_rt(kPfDown, P.stm) - 1) / pf_wg_rows_rt(kPfDown, P.stm));
    d.ks = 1; d.gps = d.G;
    d.max_tiles = ntm;
    rc = pf_launch_shape<kPfDown, false, false>(d, sb, P.stm, s);
    if (rc) return rc;
  }
  // 8. combine
  pf_moe_combine_kernel<<<dim3((unsigned)((T * H + 255) / 256)), dim3(256), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("pf_moe_combine_kernel");
  return GLQ_OK;
}
