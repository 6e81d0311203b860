// Prefill: fused dequant GEMM + low-rank correction for M > 16 tokens
// (the reference's gptq_dequant_gemm_kernel, inference/kernels/gptq_matmul.cu:
// 111-213, used for B > 4, plus the LoRA tail of GLoRCQLinear.forward,
// inference/quantized_linear.py:338-349).
//
//   y[m][n] = sum_g s[n][g] * sum_{k in g} x[m][k] (q[n][k] - z[n][g])
//             + (a SV^T)[m][n] + bias[n],     a = fp16(x U)
//
// gemm_dq_kernel: a workgroup owns a tile of 64 tokens x 64 weight rows; wave
// w computes rows 16w..16w+15 for all 64 tokens (four 16x16 MFMA tiles), so
// each decoded code feeds four MFMAs.  K advances in chunks of 256 codes (two
// groups): the x chunk of the 64 tokens is staged in LDS (double-buffered,
// permuted into the decode order, with per-group sums c1 = sum(operand
// bias * x) and c2 = sum(x)); a wave's codes, scales and zero-points go
// straight to registers, one chunk ahead.  Codes decode exactly into fp16
// 2^e + q (glq_gemv_core.h: decode2/decode4); each group's MFMA sum is
// corrected and scaled in fp32:
//   y += s_g * ((acc_g - c1_g) - z_g * c2_g).
// MFMA k-steps stay inside one group, so all 16 MFMA token rows carry tokens
// (no half-empty operands as in the GEMV's two-groups-per-step layout).
// Epilogue: y += a SV^T (MFMA), + bias, fp16 store.
//
// Split K: at prefill sizes the (N/64) x (M/64) tiles alone cannot fill 256
// CUs (44-176 workgroups at config 1) and one wave per SIMD hides no latency,
// so the K chunks are cut into `ks` splits; each (tile, split) workgroup
// writes an fp32 partial tile, extra workgroups of the same launch form the
// x U partials of each (token tile, split) with MFMA, and gemm_reduce_kernel
// sums both in a fixed order (deterministic), rounds a to fp16 once, adds
// a SV^T (MFMA) and the bias and stores fp16.  Without a workspace for the
// partials the launch is one split with the epilogue in the tile workgroups.
#include <algorithm>

#include "glq_stream.h"

namespace glq {

constexpr int kGemmBM = 64;    // tokens per workgroup tile
constexpr int kGemmBN = 64;    // weight rows per workgroup tile (16 per wave)
constexpr int kGemmKC = 256;   // codes per K chunk (two groups of 128)
constexpr int kGemmXS = kGemmKC + 8;  // halves per staged token row
constexpr int kGemmTargetWgs = 256;   // workgroups a split launch aims for (one per CU)
constexpr int kGemmXuRank = 128;      // largest rank whose x U runs inside the launch

struct GemmArgs {
  const __half* x;          // (M, K)
  const uint32_t* codes;    // (N, K*b/32)
  const __half* scales;     // (N, G)
  const __half* zeros;      // (N, G) (unused with sym)
  const __half* a;          // (M, rank) fp16 x U, or null
  const __half* sv;         // (N, rank)
  const __half* bias;       // (N,) or null
  __half* y;                // (M, N)
  const __half* u;          // (K, rank): x U inside the launch when apart != null
  float* part;              // (ks, M, N) fp32 partial tiles, or null (one split, epilogue here)
  float* apart;             // (ks, M, rpad) fp32 x U partials, or null
  int M, K, N, G, kw, rank, rpad;
  int ks, cps;              // K splits, chunks per split
  int ntn;                  // weight-row tiles along N (64 or 16 NW rows)
};

struct GemmLds {
  int xs, xc, total;  // xs: [2][BM][XS] halves; xc: [2][group 2][c1,c2][half 2][BM] floats
};
__host__ __device__ inline GemmLds gemm_lds() {
  GemmLds L;
  L.xs = 0;
  L.xc = 2 * kGemmBM * kGemmXS * 2;
  L.total = L.xc + 2 * 2 * 2 * 2 * kGemmBM * 4;
  return L;
}

// Staging assignment: thread -> (token m, group gg, half hh) of a chunk: 64
// codes = 8 f16x8 loads.
template <int BITS>
struct GemmStage {
  f16x8 v[8];
  __device__ __forceinline__ void load(const GemmArgs& g, int m0, int k0, int tid) {
    const int m = m0 + (tid >> 2), gg = (tid >> 1) & 1, hh = tid & 1;
    const int kb = k0 + 128 * gg + 64 * hh;
    const bool ok = m < g.M && kb < g.K;
    const __half* src = g.x + (int64_t)(ok ? m : 0) * g.K + (ok ? kb : 0);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ok ? *(const f16x8*)(src + 8 * u) : f16x8{};
  }
  __device__ __forceinline__ void store(__half* xs, float* xc, int tid) const {
    const int m = tid >> 2, gg = (tid >> 1) & 1, hh = tid & 1;
    float s = 0.f, sb = 0.f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {  // four 16-code blocks
      const f16x8 a = v[2 * blk], b = v[2 * blk + 1];
      f16x8 o0, o1;
      if constexpr (BITS == 2) {  // one word = 16 codes: order 0,8,1,9,..  (perm_src<2>)
        o0 = __builtin_shufflevector(a, b, 0, 8, 1, 9, 2, 10, 3, 11);
        o1 = __builtin_shufflevector(a, b, 4, 12, 5, 13, 6, 14, 7, 15);
        // operand biases (code_bias<2>): pairs (k, k+8) share 1024,256,64,16,4,1024,256,64
        const float p[8] = {(float)a[0] + (float)b[0], (float)a[1] + (float)b[1],
                            (float)a[2] + (float)b[2], (float)a[3] + (float)b[3],
                            (float)a[4] + (float)b[4], (float)a[5] + (float)b[5],
                            (float)a[6] + (float)b[6], (float)a[7] + (float)b[7]};
        sb += 1024.f * (p[0] + p[5]) + 256.f * (p[1] + p[6]) + 64.f * (p[2] + p[7]) +
              16.f * p[3] + 4.f * p[4];
#pragma unroll
        for (int c = 0; c < 8; ++c) s += p[c];
      } else {  // one word = 8 codes: order 0,4,1,5,..  per word (perm_src<4>)
        o0 = __builtin_shufflevector(a, a, 0, 4, 1, 5, 2, 6, 3, 7);
        o1 = __builtin_shufflevector(b, b, 0, 4, 1, 5, 2, 6, 3, 7);
        // operand biases (code_bias<4>): codes 0-3 of a word 1024, codes 4-7 64... per
        // decode4: positions (0,1),(4,5) -> 1024 hold codes {0,4},{2,6}; (2,3),(6,7) -> 64
        // hold codes {1,5},{3,7}
        const float e = (float)a[0] + (float)a[4] + (float)a[2] + (float)a[6] + (float)b[0] +
                        (float)b[4] + (float)b[2] + (float)b[6];
        const float o = (float)a[1] + (float)a[5] + (float)a[3] + (float)a[7] + (float)b[1] +
                        (float)b[5] + (float)b[3] + (float)b[7];
        sb += 1024.f * e + 64.f * o;
        s += e + o;
      }
      f16x8* dst = (f16x8*)(xs + m * kGemmXS + 128 * gg + 64 * hh + 16 * blk);
      dst[0] = o0;
      dst[1] = o1;
    }
    xc[((gg * 2 + 0) * 2 + hh) * kGemmBM + m] = sb;  // c1 half-sum
    xc[((gg * 2 + 1) * 2 + hh) * kGemmBM + m] = s;   // c2 half-sum
  }
};

// One wave's codes, scales and zero-points for one chunk (two groups).
template <int BITS>
struct GemmCodes {
  uint32_t w[2][BITS == 2 ? 2 : 4];
  float s[2], z[2];
  __device__ __forceinline__ void load(const GemmArgs& g, int row, int chunk, int kb, bool sym) {
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int grp = 2 * chunk + gg;
      const bool gv = grp < g.G;
      const int gc = gv ? grp : g.G - 1;
      const uint32_t* base = g.codes + (int64_t)row * g.kw;
      if constexpr (BITS == 2) {  // words 2kb, 2kb+1 of the group's 8
        const u32x2 q = *(const u32x2*)(base + 8 * gc + 2 * kb);
        w[gg][0] = q.x;
        w[gg][1] = q.y;
      } else {  // words 4kb..4kb+3 of the group's 16
        const u32x4 q = *(const u32x4*)(base + 16 * gc + 4 * kb);
        w[gg][0] = q.x;
        w[gg][1] = q.y;
        w[gg][2] = q.z;
        w[gg][3] = q.w;
      }
      const float sc = __half2float(g.scales[(int64_t)row * g.G + gc]);
      s[gg] = gv ? sc : 0.f;
      z[gg] = sym ? (float)(1 << (BITS - 1)) : __half2float(g.zeros[(int64_t)row * g.G + gc]);
    }
  }
};

// x U partial of one (token tile, K split): apart[sp][m][j] = sum over the
// split's chunks of x[m][k] U[k][j], fp32.  The x chunk (natural order) and
// the U chunk reach LDS by 16-byte loads; wave w of NW takes rank tiles w,
// w + NW, ... with v_mfma_f32_16x16x32_f16 (A = x rows, B = 8 U values of one rank
// column), accumulating over the split's chunks in registers.
template <int NW>
__device__ void gemm_xu_job(const GemmArgs& g, int m0, int sp, unsigned char* smem) {
  constexpr int NT = 64 * NW, NQ = (8 + NW - 1) / NW;  // threads; rank tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int r = g.rank, ustride = r + 8;
  __half* xl = (__half*)smem;                                       // [64][XS]
  __half* ul = (__half*)(smem + kGemmBM * kGemmXS * 2);             // [256][rank + 8]
  const int nrt = (r + 15) / 16;
  const int c0 = sp * g.cps, c1 = min(c0 + g.cps, (g.K + kGemmKC - 1) / kGemmKC);
  f32x4 acc[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[q][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int r8 = r / 8;
  for (int c = c0; c < c1; ++c) {
    const int k0 = c * kGemmKC, kl = min(kGemmKC, g.K - k0);  // a multiple of 128
    for (int idx = tid; idx < kGemmBM * (kGemmKC / 8); idx += NT) {
      const int m = idx / (kGemmKC / 8), k8 = idx - m * (kGemmKC / 8);
      f16x8 v = f16x8{};
      if (m0 + m < g.M && 8 * k8 < kl) v = *(const f16x8*)(g.x + (int64_t)(m0 + m) * g.K + k0 + 8 * k8);
      *(f16x8*)(xl + m * kGemmXS + 8 * k8) = v;
    }
    for (int idx = tid; idx < kGemmKC * r8; idx += NT) {
      const int k = idx / r8, j8 = idx - k * r8;
      f16x8 v = f16x8{};
      if (k < kl) v = *(const f16x8*)(g.u + (int64_t)(k0 + k) * r + 8 * j8);
      *(f16x8*)(ul + k * ustride + 8 * j8) = v;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int rt = wave + NW * q;
      if (rt < nrt) {  // uniform over the wave
        const int col = min(rt * 16 + li, r - 1);
        for (int u = 0; u < kGemmKC / 32; ++u) {
          const int k = 32 * u + 8 * kb;
          f16x8 bv;
#pragma unroll
          for (int e = 0; e < 8; ++e) bv[e] = (_Float16)ul[(k + e) * ustride + col];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[q][t] = mfma_16x16x32(*(const f16x8*)(xl + (16 * t + li) * kGemmXS + k), bv, acc[q][t]);
        }
      }
    }
    __syncthreads();
  }
  // acc[q][t][i]: token 16t + 4kb + i, rank column 16(wave + NW q) + li
  float* out = g.apart + (int64_t)sp * g.M * g.rpad;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int j = 16 * (wave + NW * q) + li;
    if (j >= g.rpad) continue;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * t + 4 * kb + i;
        if (m < g.M) out[(int64_t)m * g.rpad + j] = j < r ? acc[q][t][i] : 0.f;
      }
  }
}

// ---------------------------------------------------------------------------
// x prepared once per call for every weight-row tile: xp = x with each
// 16-code block permuted into the decode's operand order (perm_src), and per
// (token, 128-code group) c1 = sum code_bias(pos) xp[pos], c2 = sum x.
// One thread per 16-code block; the 8 blocks of a group are 8 consecutive
// lanes (K % 128 == 0), summed with DPP.
// ---------------------------------------------------------------------------
template <int BITS>
__global__ __launch_bounds__(256) void gemm_xprep_kernel(const __half* __restrict__ x, int M,
                                                         int K, __half* __restrict__ xp,
                                                         float* __restrict__ xc) {
  const int nb = K / 16;  // M * nb < 2^31 (host check)
  const int idx = blockIdx.x * 256 + threadIdx.x;
  const bool v = idx < M * nb;
  float s = 0.f, sb = 0.f;
  int m = 0, blk = 0;
  if (v) {
    m = idx / nb;
    blk = idx - m * nb;
    const f16x8* src = (const f16x8*)(x + (int64_t)m * K + 16 * blk);
    const f16x8 a = src[0], b = src[1];
    _Float16 in[16], o[16];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      in[c] = a[c];
      in[8 + c] = b[c];
    }
#pragma unroll
    for (int pos = 0; pos < 16; ++pos) {
      o[pos] = in[perm_src<BITS>(pos)];
      const float f = (float)o[pos];
      s += f;
      sb += code_bias<BITS>(pos) * f;
    }
    f16x8 o0, o1;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      o0[c] = o[c];
      o1[c] = o[8 + c];
    }
    f16x8* dst = (f16x8*)(xp + (int64_t)m * K + 16 * blk);
    dst[0] = o0;
    dst[1] = o1;
  }
  auto grp8 = [](float t) {  // sum over aligned groups of 8 lanes, every lane gets it
    t += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0xB1, 0xF, 0xF, false));
    t += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x4E, 0xF, 0xF, false));
    t += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x141, 0xF, 0xF, false));
    return t;
  };
  s = grp8(s);
  sb = grp8(sb);
  if (v && (blk & 7) == 0) {
    const int64_t o = ((int64_t)m * (K / 128) + blk / 8) * 2;
    xc[o] = sb;
    xc[o + 1] = s;
  }
}

// ---------------------------------------------------------------------------
// Tile kernel over the prepared x: a workgroup of NW waves owns 64 tokens x
// 16 NW weight rows and a K split, in chunks of one 128-code group.  Everything a group
// needs reaches LDS by direct global->LDS loads (no VGPRs in flight), in a
// ring of kG2Depth slots with kG2Depth - 1 groups in flight:
//   x     64 token rows x 256 B; 16-byte piece p of row r at p ^ (r % 16),
//         so the MFMA A reads of 16 rows are bank-conflict free;
//   codes per wave, its 16 weight rows' words of the group;
//   s, z  per wave, one fp16 each per row (2-byte loads; the LDS DMA puts
//         each lane's value at a 4-byte stride);
//   c     per wave, (c1, c2) of its 16 tokens of the prepared sums.
// Per group: 4 k-steps x 4 token tiles of v_mfma_f32_16x16x32_f16 (B = exact
// 2^e + q codes), y += s acc, and the operand-bias and zero-point correction
// as one v_mfma_f32_16x16x4_f32 per token tile:
//   A[tok][k] = (c1, c2, 0, 0)[k],  B[k][row] = (-s, -s z, 0, 0)[k].
// Every group issues the same loads (past the split's end they re-read its
// last group), so the explicit vmcnt wait counts exactly; a bare s_barrier
// (no fence: __syncthreads would wait for every load in flight) makes the
// other waves' pieces visible and frees the slot refilled next.
// ---------------------------------------------------------------------------
constexpr int kG2Depth = 3;
// slot layout for NW waves (16 weight rows each): x 16 KB, then per wave
// 1 KB of codes, 256 B of scales, 256 B of zero-points, 256 B of (c1, c2)
template <int NW> constexpr int g2_codes() { return kGemmBM * 256; }
template <int NW> constexpr int g2_s() { return g2_codes<NW>() + NW * 1024; }
template <int NW> constexpr int g2_z() { return g2_s<NW>() + NW * 256; }
template <int NW> constexpr int g2_c() { return g2_z<NW>() + NW * 256; }
template <int NW> constexpr int g2_slot() { return g2_c<NW>() + NW * 256; }

template <int BITS, bool SYM, int NW>
__device__ __forceinline__ void g2_issue(const GemmArgs& g, const __half* xp, const float* xc,
                                         int m0, int n0, int grp, unsigned char* slot, int wave,
                                         int lane) {
  constexpr int XI = 16 / NW;  // x instructions per wave (1 KB = 4 token rows each)
#pragma unroll
  for (int q = 0; q < XI; ++q) {
    const int r4 = 4 * (XI * wave + q);
    const int rr = r4 + (lane >> 4);
    const int p = (lane & 15) ^ (rr & 15);
    const int m = min(m0 + rr, g.M - 1);
    __builtin_amdgcn_global_load_lds((const void*)(xp + (int64_t)m * g.K + grp * 128 + 8 * p),
                                     (lds_void*)(slot + r4 * 256), 16, 0, 0);
  }
  {  // codes: 16 B a lane, the wave's 16 rows in order (2-bit: lanes 32-63 repeat)
    constexpr int LPR = BITS == 2 ? 2 : 4;  // lanes per row
    const int l = BITS == 2 ? (lane & 31) : lane;
    const int n = min(n0 + 16 * wave + l / LPR, g.N - 1);
    const uint32_t* src = g.codes + (int64_t)n * g.kw + (BITS == 2 ? 8 : 16) * grp + 4 * (l % LPR);
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (lds_void*)(slot + g2_codes<NW>() + wave * 1024), 16, 0, 0);
  }
  {  // s and z of the wave's rows: 2 B a lane (lanes 16-63 repeat row 15's)
    const int n = min(n0 + 16 * wave + min(lane, 15), g.N - 1);
    const int64_t e = (int64_t)n * g.G + grp;
    __builtin_amdgcn_global_load_lds((const void*)(g.scales + e),
                                     (lds_void*)(slot + g2_s<NW>() + wave * 256), 2, 0, 0);
    if constexpr (!SYM)
      __builtin_amdgcn_global_load_lds((const void*)(g.zeros + e),
                                       (lds_void*)(slot + g2_z<NW>() + wave * 256), 2, 0, 0);
  }
  {  // (c1, c2) of 16 tokens: 4 B a lane (lanes 32-63 repeat); wave w >= 4 repeats wave w % 4
    const int l = lane & 31;
    const int m = min(m0 + 16 * (wave & 3) + l / 2, g.M - 1);
    __builtin_amdgcn_global_load_lds((const void*)(xc + ((int64_t)m * g.G + grp) * 2 + (l & 1)),
                                     (lds_void*)(slot + g2_c<NW>() + wave * 256), 4, 0, 0);
  }
}

template <int BITS, bool SYM, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void gemm_dq2_kernel(GemmArgs g, const __half* xp,
                                                                   const float* xc) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int SLOT = g2_slot<NW>();
  const int m0 = blockIdx.y * kGemmBM;
  // the x U jobs (the longer ones) take the first workgroup ids of each token
  // tile, so they start first and overlap the weight tiles
  const int nxu = g.apart ? g.ks : 0;
  if ((int)blockIdx.x < nxu) {  // uniform over the workgroup
    gemm_xu_job<NW>(g, m0, blockIdx.x, smem);
    return;
  }
  const int job = blockIdx.x - nxu;
  const int tn = job % g.ntn, sp = job / g.ntn;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int n0 = tn * 16 * NW;
  const int g0 = sp * g.cps * 2, g1 = min(g0 + g.cps * 2, g.G);  // this split's groups
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  constexpr int NI = 16 / NW + 1 + 1 + (SYM ? 0 : 1) + 1;  // loads per group per thread
  const DecodeConsts dk = DecodeConsts::make();

  f32x4 y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = 0; d < kG2Depth - 1; ++d)
    g2_issue<BITS, SYM, NW>(g, xp, xc, m0, n0, min(g0 + d, g1 - 1), smem + d * SLOT, wave, lane);
  int slot = 0;
  for (int grp = g0; grp < g1; ++grp) {
    wait_vmcnt<NI * (kG2Depth - 2)>();  // this thread's pieces of group grp are in
    asm volatile("s_barrier" ::: "memory");  // everyone's are; the slot of grp - 1 is free
    const int sn = slot == 0 ? kG2Depth - 1 : slot - 1;
    g2_issue<BITS, SYM, NW>(g, xp, xc, m0, n0, min(grp + kG2Depth - 1, g1 - 1), smem + sn * SLOT,
                            wave, lane);
    const unsigned char* sb = smem + slot * SLOT;
    f16x8 bop[4];
    if constexpr (BITS == 2) {
      const u32x2 w = *(const u32x2*)(sb + g2_codes<NW>() + wave * 1024 + 32 * li + 8 * kb);
      decode2(w.x ^ xor_mask, bop[0], bop[1], dk);
      decode2(w.y ^ xor_mask, bop[2], bop[3], dk);
    } else {
      const u32x4 w = *(const u32x4*)(sb + g2_codes<NW>() + wave * 1024 + 64 * li + 16 * kb);
#pragma unroll
      for (int j = 0; j < 4; ++j) bop[j] = decode4(w[j] ^ xor_mask, dk);
    }
    const float sc = __half2float(*(const __half*)(sb + g2_s<NW>() + wave * 256 + 4 * li));
    float zc = (float)(1 << (BITS - 1));
    if constexpr (!SYM) zc = __half2float(*(const __half*)(sb + g2_z<NW>() + wave * 256 + 4 * li));
    const float bcor = kb == 0 ? -sc : (kb == 1 ? -sc * zc : 0.f);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const unsigned char* xr = sb + (16 * t + li) * 256;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // k-slot kb of step j: 2-bit word 2kb + j/2, half j%2; 4-bit word 4kb + j
        const int piece = BITS == 2 ? 2 * (2 * kb + (j >> 1)) + (j & 1) : 4 * kb + j;
        acc = mfma_16x16x32(*(const f16x8*)(xr + 16 * (piece ^ li)), bop[j], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) y[t][i] = fmaf(sc, acc[i], y[t][i]);
      const float cv =
          kb < 2 ? *(const float*)(sb + g2_c<NW>() + t * 256 + (2 * li + kb) * 4) : 0.f;
      y[t] = mfma_16x16x4f32(cv, bcor, y[t]);
    }
    slot = slot == kG2Depth - 1 ? 0 : slot + 1;
  }
  wait_vmcnt<0>();  // the tail's loads land before the workgroup's LDS goes away

  const int n = n0 + 16 * wave + li;
  if (g.part && n < g.N) {  // fp32 partial tile of this split
    float* pt = g.part + (int64_t)sp * g.M * g.N;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * t + 4 * kb + i;
        if (m < g.M) pt[(int64_t)m * g.N + n] = y[t][i];
      }
  }
}

template <int BITS, bool SYM>
__global__ __launch_bounds__(256, 2) void gemm_dq_kernel(GemmArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int m0 = blockIdx.y * kGemmBM;
  const int job = blockIdx.x;
  if (job >= g.ntn * g.ks) {  // uniform over the workgroup
    gemm_xu_job<4>(g, m0, job - g.ntn * g.ks, smem);
    return;
  }
  const int tn = job % g.ntn, sp = job / g.ntn;
  const GemmLds L = gemm_lds();
  __half* xs0 = (__half*)(smem + L.xs);
  float* xc0 = (float*)(smem + L.xc);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int n0 = tn * kGemmBN;
  const int row = min(n0 + 16 * wave + li, g.N - 1);
  const int nch = (g.K + kGemmKC - 1) / kGemmKC;
  const int c0 = sp * g.cps, c1 = min(c0 + g.cps, nch);
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  const DecodeConsts dk = DecodeConsts::make();

  f32x4 y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  GemmStage<BITS> st;
  GemmCodes<BITS> cur, nxt;
  st.load(g, m0, c0 * kGemmKC, tid);
  cur.load(g, row, c0, kb, SYM);
  st.store(xs0, xc0, tid);
  __syncthreads();

  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    const bool more = c + 1 < c1;
    if (more) {  // next chunk in flight while this one computes
      st.load(g, m0, (c + 1) * kGemmKC, tid);
      nxt.load(g, row, c + 1, kb, SYM);
    }
    const __half* xs = xs0 + buf * kGemmBM * kGemmXS;
    const float* xc = xc0 + buf * 2 * 2 * 2 * kGemmBM;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      f16x8 bop[4];  // B operands of the group's four MFMA k-steps
      if constexpr (BITS == 2) {
        decode2(cur.w[gg][0] ^ xor_mask, bop[0], bop[1], dk);
        decode2(cur.w[gg][1] ^ xor_mask, bop[2], bop[3], dk);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) bop[j] = decode4(cur.w[gg][j] ^ xor_mask, dk);
      }
      const float sc = cur.s[gg], zc = cur.z[gg];
      const float* c1a = xc + ((gg * 2 + 0) * 2 + 0) * kGemmBM;
      const float* c1b = xc + ((gg * 2 + 0) * 2 + 1) * kGemmBM;
      const float* c2a = xc + ((gg * 2 + 1) * 2 + 0) * kGemmBM;
      const float* c2b = xc + ((gg * 2 + 1) * 2 + 1) * kGemmBM;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const __half* xr = xs + (16 * t + li) * kGemmXS + 128 * gg;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // k-slot kb of step j: 2-bit word 2kb + j/2, half j%2; 4-bit word 4kb + j
          const int off = BITS == 2 ? 16 * (2 * kb + (j >> 1)) + 8 * (j & 1) : 8 * (4 * kb + j);
          acc = mfma_16x16x32(*(const f16x8*)(xr + off), bop[j], acc);
        }
        const int mt = 16 * t + 4 * kb;  // this lane's first token of the tile
        const f32x4 c1 = *(const f32x4*)(c1a + mt) + *(const f32x4*)(c1b + mt);
        const f32x4 c2 = *(const f32x4*)(c2a + mt) + *(const f32x4*)(c2b + mt);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[t][i] += sc * ((acc[i] - c1[i]) - zc * c2[i]);
      }
    }
    if (more) {
      st.store(xs0 + (buf ^ 1) * kGemmBM * kGemmXS, xc0 + (buf ^ 1) * 2 * 2 * 2 * kGemmBM, tid);
      cur = nxt;
    }
    __syncthreads();
  }

  const int n = n0 + 16 * wave + li;
  if (g.part) {  // fp32 partial tile of this split
    if (n < g.N) {
      float* pt = g.part + (int64_t)sp * g.M * g.N;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * t + 4 * kb + i;
          if (m < g.M) pt[(int64_t)m * g.N + n] = y[t][i];
        }
    }
    return;
  }
  // ---- one split: epilogue here, y += a SV^T, + bias, store ----
  if (g.a) {
    for (int j0 = 0; j0 < g.rank; j0 += 32) {
      const int jk = j0 + 8 * kb;
      const bool jv = jk < g.rank;
      const f16x8 bv = jv ? *(const f16x8*)(g.sv + (int64_t)row * g.rank + jk) : f16x8{};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = m0 + 16 * t + li;
        const f16x8 av = (jv && m < g.M) ? *(const f16x8*)(g.a + (int64_t)m * g.rank + jk)
                                         : f16x8{};
        y[t] = mfma_16x16x32(av, bv, y[t]);
      }
    }
  }
  if (n < g.N) {
    const float bn = g.bias ? __half2float(g.bias[n]) : 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * t + 4 * kb + i;
        if (m < g.M) g.y[(int64_t)m * g.N + n] = __float2half(y[t][i] + bn);
      }
  }
}

// y[m][n] = fp16(sum_sp part[sp][m][n] + (a SV^T)[m][n] + bias[n]), a =
// fp16(sum_sp apart[sp][m][:]) or the caller's; splits summed in order.  One
// workgroup = 16 tokens x 64 rows: wave w takes rows 16w..16w+15, lane (li,
// kb) tokens 4kb..4kb+3 of row li (the MFMA D layout), so a SV^T lands in the
// same registers.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs g) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int n = blockIdx.x * kGemmBN + 16 * wave + li, m0 = blockIdx.y * 16;
  const int nc = min(n, g.N - 1);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int64_t pstride = (int64_t)g.M * g.N;
  for (int s0 = 0; s0 < g.ks; s0 += 8) {  // 32 loads in flight, then the adds in order
    float v[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = min(m0 + 4 * kb + i, g.M - 1);
      const float* p = g.part + (int64_t)m * g.N + nc;
#pragma unroll
      for (int u = 0; u < 8; ++u) v[i][u] = s0 + u < g.ks ? p[(s0 + u) * pstride] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[i] += v[i][u];
  }
  if (g.sv && g.rank > 0) {
    const int ma = min(m0 + li, g.M - 1);  // A operand row of this lane
    for (int j0 = 0; j0 < g.rank; j0 += 32) {
      const int jk = j0 + 8 * kb;
      const bool jv = jk < g.rank;
      f16x8 av = f16x8{}, bv = f16x8{};
      if (jv) {
        bv = *(const f16x8*)(g.sv + (int64_t)nc * g.rank + jk);
        if (g.a) {
          av = *(const f16x8*)(g.a + (int64_t)ma * g.rank + jk);
        } else {
          const float* ap = g.apart + (int64_t)ma * g.rpad + jk;
          const int64_t astride = (int64_t)g.M * g.rpad;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            av[e] = (_Float16)__half2float(__float2half(sum_strided(ap + e, astride, g.ks)));
        }
      }
      acc = mfma_16x16x32(av, bv, acc);
    }
  }
  if (n < g.N) {
    const float bn = g.bias ? __half2float(g.bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 4 * kb + i;
      if (m < g.M) g.y[(int64_t)m * g.N + n] = __float2half(acc[i] + bn);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

// Split plan: ks splits of cps chunks each, enough (tile, split) workgroups
// to reach kGemmTargetWgs, no empty split.
struct GemmPlan {
  int ntn, ntm, nch, ks, cps;
  bool xu_in;  // x U partials inside the launch
  int64_t part_bytes, apart_bytes, xu_bytes, xp_bytes, xc_bytes;  // workspace pieces
};

int64_t lowrank_ws(int64_t M, int64_t K, int64_t rank) {
  const int64_t full = M / 16, tail = M % 16;
  int64_t need = glq_lowrank_workspace_bytes(full > 0 ? full : 1, 16, K, rank);
  if (tail) need = std::max(need, glq_lowrank_workspace_bytes(1, tail, K, rank));
  return align_up(need, 256) + align_up(M * rank * 2, 256);
}

constexpr int kG2Waves = 8;  // waves per workgroup of the ring kernel (128 weight rows)

GemmPlan gemm_plan(int64_t M, int64_t K, int64_t N, int64_t rank) {
  GemmPlan P;
  P.ntn = (int)((N + 16 * kG2Waves - 1) / (16 * kG2Waves));
  P.ntm = (int)((M + kGemmBM - 1) / kGemmBM);
  P.nch = (int)((K + kGemmKC - 1) / kGemmKC);
  const int64_t tiles = (int64_t)P.ntn * P.ntm;
  int ks = (int)std::min<int64_t>(P.nch, std::max<int64_t>(1, (kGemmTargetWgs + tiles - 1) / tiles));
  // (the ring kernel's 8-wave workgroups: one per CU)
  if (const char* e = getenv("GLQ_GEMM_KS")) ks = std::max(1, std::min(P.nch, atoi(e)));
  P.cps = (P.nch + ks - 1) / ks;
  P.ks = (P.nch + P.cps - 1) / P.cps;
  P.xu_in = rank > 0 && rank <= kGemmXuRank;
  P.part_bytes = align_up((int64_t)P.ks * M * N * 4, 256);
  P.apart_bytes = P.xu_in ? align_up((int64_t)P.ks * M * align_up(rank, 32) * 4, 256) : 0;
  P.xu_bytes = (rank > 0 && !P.xu_in) ? lowrank_ws(M, K, rank) : 0;
  P.xp_bytes = align_up(M * K * 2, 256);
  P.xc_bytes = align_up(M * (K / 128) * 8, 256);
  return P;
}

size_t gemm_launch_lds(const GemmArgs& g, bool ring) {
  size_t lds = ring ? (size_t)kG2Depth * g2_slot<kG2Waves>() : (size_t)gemm_lds().total;
  if (g.apart)
    lds = std::max(lds, (size_t)kGemmBM * kGemmXS * 2 + (size_t)kGemmKC * (g.rank + 8) * 2);
  return lds;
}

template <int BITS, bool SYM>
int launch_gemm(const GemmArgs& g, int ntm, __half* xp, float* xc, hipStream_t s) {
  static size_t attr = 64 * 1024, attr2 = 64 * 1024;
  const int xu_jobs = g.apart ? g.ks : 0;
  const dim3 grid((unsigned)(g.ntn * g.ks + xu_jobs), (unsigned)ntm);
  if (xp) {  // split launch over the prepared x
    const int64_t blocks = ((int64_t)g.M * (g.K / 16) + 255) / 256;
    gemm_xprep_kernel<BITS><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(g.x, g.M, g.K, xp, xc);
    GLQ_LAUNCH_CHECK("gemm_xprep_kernel");
    const size_t lds = gemm_launch_lds(g, true);
    int rc = set_lds_limit(gemm_dq2_kernel<BITS, SYM, kG2Waves>, lds, attr2);
    if (rc) return rc;
    gemm_dq2_kernel<BITS, SYM, kG2Waves><<<grid, dim3(64 * kG2Waves), lds, s>>>(g, xp, xc);
    GLQ_LAUNCH_CHECK("gemm_dq2_kernel");
  } else {
    const size_t lds = gemm_launch_lds(g, false);
    int rc = set_lds_limit(gemm_dq_kernel<BITS, SYM>, lds, attr);
    if (rc) return rc;
    gemm_dq_kernel<BITS, SYM><<<grid, dim3(256), lds, s>>>(g);
    GLQ_LAUNCH_CHECK("gemm_dq_kernel");
  }
  if (g.part) {
    const dim3 rgrid((unsigned)((g.N + kGemmBN - 1) / kGemmBN), (unsigned)((g.M + 15) / 16));
    gemm_reduce_kernel<<<rgrid, dim3(256), 0, s>>>(g);
    GLQ_LAUNCH_CHECK("gemm_reduce_kernel");
  }
  return GLQ_OK;
}

}  // namespace
}  // namespace glq

extern "C" int64_t glq_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (rank < 0) return -1;
  const glq::GemmPlan P = glq::gemm_plan(M, K, N, rank);
  return P.part_bytes + P.apart_bytes + P.xu_bytes + P.xp_bytes + P.xc_bytes;
}

extern "C" int glq_gemm_lora(const void* x, int64_t M, int64_t K, int64_t N,
                             const int32_t* codes, int bits, const void* scales,
                             const void* zeros, int64_t group, int sym, const void* U,
                             const void* SV, int64_t rank, const void* xU, const void* bias,
                             void* y, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(M >= 0 && K >= 0 && N >= 0, "negative size");
  if (M == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(bits == 2 || bits == 4, "bits must be 2 or 4 (got %d)", bits);
  GLQ_CHECK(group == 128, "the GEMM path takes group 128 (got %lld)", (long long)group);
  GLQ_CHECK(K > 0 && K % 128 == 0 && K < (1 << 24), "K=%lld must be a positive multiple of 128",
            (long long)K);
  GLQ_CHECK(N < (1ll << 30) && M < (1ll << 31) / 2 && M * (K / 16) < (1ll << 31),
            "shape too large");
  GLQ_CHECK(x && codes && scales && y && (sym || zeros), "null data pointer");
  const bool lora = SV != nullptr && rank > 0;
  if (lora) {
    GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
              (long long)rank);
    GLQ_CHECK(U != nullptr || xU != nullptr, "LoRA needs U or a precomputed xU");
  }
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x) && al16(codes) && (!lora || al16(SV)) && (!xU || al16(xU)) &&
                (!U || al16(U)),
            "x, codes, U, SV and xU must be 16-byte aligned");
  GLQ_CHECK(workspace == nullptr || ((uintptr_t)workspace & 255) == 0,
            "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const bool need_xu = lora && xU == nullptr;
  GemmPlan P = gemm_plan(M, K, N, need_xu ? rank : 0);
  const int64_t need = P.part_bytes + P.apart_bytes + P.xu_bytes + P.xp_bytes + P.xc_bytes;
  const bool split = workspace != nullptr && workspace_bytes >= need;
  GemmArgs g = {};
  g.x = (const __half*)x;
  g.codes = (const uint32_t*)codes;
  g.scales = (const __half*)scales;
  g.zeros = (const __half*)zeros;
  g.sv = lora ? (const __half*)SV : nullptr;
  g.bias = (const __half*)bias;
  g.y = (__half*)y;
  g.M = (int)M;
  g.K = (int)K;
  g.N = (int)N;
  g.G = (int)(K / 128);
  g.kw = (int)(K * bits / 32);
  g.rank = lora ? (int)rank : 0;
  g.rpad = (int)align_up(g.rank, 32);
  g.ntn = P.ntn;
  g.a = lora && xU ? (const __half*)xU : nullptr;
  __half* xp = nullptr;
  float* xc = nullptr;
  if (split) {
    char* w = (char*)workspace;
    xp = (__half*)(w + P.part_bytes + P.apart_bytes + P.xu_bytes);
    xc = (float*)((char*)xp + P.xp_bytes);
    g.part = (float*)w;
    g.ks = P.ks;
    g.cps = P.cps;
    if (need_xu && P.xu_in) {
      g.apart = (float*)(w + P.part_bytes);
      g.u = (const __half*)U;
    } else if (need_xu) {  // rank above the in-launch limit: the low-rank entry point
      char* xw = w + P.part_bytes;
      const int64_t xneed = P.xu_bytes;
      const int64_t pbytes = xneed - align_up(M * rank * 2, 256);
      __half* abuf = (__half*)(xw + pbytes);
      const int64_t full = M / 16, tail = M % 16;
      if (full > 0) {
        int rc = glq_lowrank_xu_batched(full, x, 16 * K, 16, K, U, 0, rank, abuf, 16 * rank,
                                        xw, pbytes, stream);
        if (rc) return rc;
      }
      if (tail) {
        int rc = glq_lowrank_xu_batched(1, (const __half*)x + full * 16 * K, 0, tail, K, U, 0,
                                        rank, abuf + full * 16 * rank, 0, xw, pbytes, stream);
        if (rc) return rc;
      }
      g.a = abuf;
    }
  } else {
    // no room for the partials: one split with the epilogue in the tile
    // workgroups (64-row tiles); a from xU, or (LoRA without xU) the
    // low-rank launches
    g.ks = 1;
    g.cps = P.nch;
    g.ntn = (int)((N + kGemmBN - 1) / kGemmBN);
    if (need_xu) {
      const int64_t xneed = lowrank_ws(M, K, rank);
      GLQ_CHECK(workspace != nullptr && workspace_bytes >= xneed,
                "workspace of %lld bytes needed (got %lld)", (long long)xneed,
                (long long)workspace_bytes);
      const int64_t pbytes = xneed - align_up(M * rank * 2, 256);
      __half* abuf = (__half*)((char*)workspace + pbytes);
      const int64_t full = M / 16, tail = M % 16;
      if (full > 0) {
        int rc = glq_lowrank_xu_batched(full, x, 16 * K, 16, K, U, 0, rank, abuf, 16 * rank,
                                        workspace, pbytes, stream);
        if (rc) return rc;
      }
      if (tail) {
        int rc = glq_lowrank_xu_batched(1, (const __half*)x + full * 16 * K, 0, tail, K, U, 0,
                                        rank, abuf + full * 16 * rank, 0, workspace, pbytes,
                                        stream);
        if (rc) return rc;
      }
      g.a = abuf;
    }
  }
  if (bits == 2)
    return sym ? launch_gemm<2, true>(g, P.ntm, xp, xc, s) : launch_gemm<2, false>(g, P.ntm, xp, xc, s);
  return sym ? launch_gemm<4, true>(g, P.ntm, xp, xc, s) : launch_gemm<4, false>(g, P.ntm, xp, xc, s);
}
