// Streaming fused dequant-GEMV + low-rank correction (gfx950, group 128).
//
// Same result as gemv_tile (glq_gemv_core.h) for 1 <= M <= 16, built for HBM
// bandwidth instead of simplicity:
//  * Row-split: each wave owns whole 16-row tiles (full K), so it never waits
//    on another wave after the one-time staging of x and a.
//  * Codes, scales, zero-points, SV rows and bias reach LDS by direct
//    global->LDS loads (global_load_lds_dwordx4 / _dword), so the data in
//    flight occupies no VGPRs.  Each wave keeps a ring of D chunk slots and
//    streams, per tile, its code chunks (16 rows x 128 contiguous bytes of
//    every row: 2 load instructions of 8 rows x 128 B, the pattern the MI355X
//    memory system serves fastest, plus the chunk's scales and zero-points)
//    and then its SV chunks (16 rows x 64 rank columns, + bias), which the
//    tile epilogue consumes straight from the ring.  D-1 chunks are in flight
//    while one is consumed, across tile boundaries.
//  * The 16-byte pieces of a chunk are permuted across lanes (piece ^ (row/2))
//    so the MFMA-layout reads from LDS are bank-conflict free.
//  * MFMA roles: A = x (token rows), B = codes (weight rows as columns), so
//    D[token][row] and each lane needs one scale and one zero-point per step.
//    2-bit steps (256 codes, two 128-code groups) keep their two groups apart
//    inside one MFMA: group-half h's x goes to A rows 8h..8h+7 (zeros
//    elsewhere), so D rows 0-7 / 8-15 are the two half sums; tokens 8..15 take
//    a second pass; halves merge with one cross-lane add per tile.
//  * The compiler does not order LDS reads after direct-to-LDS loads, so the
//    kernel waits explicitly: before consuming chunk c it waits until at most
//    NI*(D-1) vector-memory operations are outstanding, where NI is the number
//    of load instructions every chunk issues (padded with dummy loads where a
//    chunk needs fewer).  Loads of one wave complete in order, and any store
//    or ordinary load issued after chunk c's loads only makes that wait
//    stricter, so chunk c is in LDS when the wait returns.  Before a
//    slot is refilled, all LDS reads of the wave have completed (lgkmcnt(0)).
#pragma once

#include "glq_gemv_core.h"

namespace glq {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kStreamCodeBytes = 2048;  // 16 rows x 128 B

// Scale/zero-point bytes per slot: 2-bit with odd G moves one dword per
// (row, group) for s and for z (512 B); otherwise s and z of a chunk fit one
// instruction (256 B).
template <bool SZ2>
constexpr int stream_slot() { return kStreamCodeBytes + (SZ2 ? 512 : 256); }
// Load instructions per chunk (every chunk issues exactly this many).
template <bool SZ2>
constexpr int stream_ni() { return SZ2 ? 4 : 3; }

// Explicit waits.  Inline asm with a memory clobber, so no compiler pass moves
// an LDS access across them.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Shape/layout of a streaming launch (every item has the same K and N).
struct StreamShape {
  int K, N, G, rank, rpad, sym, kw;
  float zoff;      // added to every zero-point (signed codes stored offset by 2^(b-1))
  int nchunk;      // 128-byte code chunks per row (last one may be partial)
  int nsvc;        // SV chunks per tile (64 rank columns each; 0 = no LoRA)
  int tiles;       // 16-row tiles per item
  int xstride;     // halves per staged token row of x
  int mmax;        // largest M of any item
  int apad;        // halves per token row of staged a
  // K sub-range of a work unit (the whole row for a plain GEMV): the unit's
  // codes, scales and x start `goff` groups into the row; `gend` groups are
  // left from there to the row end; `rowlast` = bytes from the unit's first
  // code byte to the last 16-byte piece of the row.
  int goff, gend, rowlast;
};

struct StreamLds {
  // byte offsets; xc = [chunk128][16 tokens] x 2 floats; tl / pl: per-wave
  // inter tile and low-rank partials of the two-matrix form (else empty)
  int xs, xc, a, ring, tl, pl, total;
};

// x rows are staged zero-padded over every code position the row's chunks
// cover (a chunk is 128 bytes of a weight row: 512 codes at 2 bits, 256 at 4),
// so the MFMA steps of a partial last chunk read zeros, never unwritten LDS
// (0 * NaN would survive the zero scale of such a step).  Lanes without a
// token read a 512-byte zero block instead (their per-step x stride is 0);
// the per-128-code sums get matching zero padding.
__host__ __device__ inline int stream_kpad(int K, int bits) {
  const int unit = bits == 2 ? 512 : 256;
  return (K + unit - 1) / unit * unit;
}

__host__ __device__ inline StreamLds stream_lds(int D, int slot, int mmax, int K, int bits,
                                                int xstride, int apad, int nmat = 1,
                                                int postcols = 0) {
  StreamLds L;
  int o = 0;
  L.xs = o;   o += al16(mmax * xstride * 2) + 512;  // + zero block read by masked lanes
  L.xc = o;   o += al16((stream_kpad(K, bits) / 128) * 32 * 4);
  L.a = o;    o += al16(nmat * 16 * apad * 2);
  L.ring = o; o += 4 * D * slot;
  L.tl = o;   o += nmat == 2 ? 4 * 16 * 16 * 4 : 0;
  L.pl = o;   o += 4 * mmax * postcols * 4;
  L.total = o;
  return L;
}

// Pointers of one weight matrix of a work unit, already offset to the unit's
// K range (codes by goff*128 codes, scales/zero-points by goff groups).
struct StreamMat {
  const uint32_t* C;
  const __half* S;
  const __half* Z;   // == S for symmetric codes
  const __half* SV;  // nullptr: no low-rank term
  const __half* B;   // bias or nullptr
};

// Per-tile load addresses of one lane (see StreamCursor::retarget).
struct IssuePtrs {
  const char* code[2];  // this lane's row start in the codes, per instruction
  const char* sv[2];    // ... in SV
  const char* s;        // scale dword base (element row*G of this lane's row), bytes
  const char* z;        // zero-point dword base
  const char* bias;     // bias dword of this lane
};

// Issue-side cursor of one wave: which chunk of which tile goes out next.
template <int BITS, bool SZ2>
struct StreamCursor {
  int c = 0;      // chunk within the tile (codes first, then SV chunks)
  int r0 = 0;     // first row of the tile
  int slot = 0;   // ring slot the next chunk lands in
  IssuePtrs P;

  // Recomputes this lane's row pointers for the tile at row r0 (once per tile).
  __device__ __forceinline__ void retarget(const StreamMat& m, const StreamShape& sh, int lane) {
    const uint32_t* C = m.C;
    const __half *S = m.S, *Zs = m.Z, *SV = m.SV, *B = m.B;
    const int64_t rowbytes = (int64_t)sh.kw * 4;
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int n = min(r0 + 8 * I + (lane >> 3), sh.N - 1);
      P.code[I] = (const char*)C + n * rowbytes;
      P.sv[I] = SV ? (const char*)SV + (int64_t)n * sh.rank * 2 : nullptr;
    }
    if constexpr (BITS == 2 && SZ2) {
      const int n = min(r0 + (lane >> 2), sh.N - 1);
      P.s = (const char*)(S + (int64_t)n * sh.G);
      P.z = (const char*)(Zs + (int64_t)n * sh.G);
    } else {
      const int q = lane & 31;
      const int n = min(r0 + (q >> 1), sh.N - 1);
      P.s = (const char*)((lane < 32 ? S : Zs) + (int64_t)n * sh.G);
      P.z = P.s;
    }
    P.bias = B ? (const char*)(B + min(r0 + 2 * (lane & 7), sh.N - 2)) : nullptr;
  }
};

// Issues code chunk `ch` of the cursor's tile into `slot`: codes (16 rows x
// 128 B: lane q of instruction I carries row 8I + q/8, 16-byte piece
// (q%8) ^ ((row/2)%8), so MFMA-layout reads are bank-conflict free; pieces
// past the end of a row re-read the row's last piece), then the chunk's
// scales and zero-points as the aligned dwords that contain them:
//   2-bit, even G: lane q -> (q<32 ? s : z), row (q%32)/2, groups 4ch+2(q%2)+{0,1}
//   2-bit, odd G (SZ2): lane q -> row q/4, group 4ch+q%4; s then z instruction
//   4-bit: lane q -> (q<32 ? s : z), row (q%32)/2, group 2ch+q%2
// N is even (host check), so every dword lies inside its tensor.  Groups past
// the unit's K range read valid neighbours (scale forced to 0 on use).
template <int BITS, bool SZ2>
__device__ __forceinline__ void stream_issue(const IssuePtrs& P, const StreamShape& sh, int ch,
                                             unsigned char* slot, int lane, int piece0,
                                             int piece1) {
  const int rowlast = sh.rowlast;
  __builtin_amdgcn_global_load_lds((const void*)(P.code[0] + min(128 * ch + piece0, rowlast)),
                                   (lds_void*)slot, 16, 0, 0);
  __builtin_amdgcn_global_load_lds((const void*)(P.code[1] + min(128 * ch + piece1, rowlast)),
                                   (lds_void*)(slot + 1024), 16, 0, 0);
  unsigned char* szs = slot + kStreamCodeBytes;
  if constexpr (BITS == 2 && SZ2) {
    const int g = min(4 * ch + (lane & 3), sh.gend - 1);
    // element row*G + g rounded down to even: the row base parity is folded
    // in by the pointer (row*G may be odd), so round the absolute address
    const uintptr_t sa = ((uintptr_t)(P.s + 2 * g)) & ~(uintptr_t)3;
    const uintptr_t za = ((uintptr_t)(P.z + 2 * g)) & ~(uintptr_t)3;
    __builtin_amdgcn_global_load_lds((const void*)sa, (lds_void*)szs, 4, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)za, (lds_void*)(szs + 256), 4, 0, 0);
  } else if constexpr (BITS == 2) {
    const int g = min(4 * ch + 2 * (lane & 1), sh.gend - 2);  // even: G, goff even here
    __builtin_amdgcn_global_load_lds((const void*)(P.s + 2 * g), (lds_void*)szs, 4, 0, 0);
  } else {
    const int g = min(2 * ch + (lane & 1), sh.gend - 1);
    const uintptr_t sa = ((uintptr_t)(P.s + 2 * g)) & ~(uintptr_t)3;
    __builtin_amdgcn_global_load_lds((const void*)sa, (lds_void*)szs, 4, 0, 0);
  }
}

// SV chunk `c` of the cursor's tile: rank columns [64c, 64c + 64) of 16 SV
// rows (columns past the rank read the row's last piece; the matching a
// values are zero), then bias dwords (lane q -> bias[r0 + 2(q%8)], +1) or a
// dummy load, and a second dummy for NI == 4, so the chunk issues NI loads.
template <bool SZ2>
__device__ __forceinline__ void stream_issue_sv(const IssuePtrs& P, const StreamShape& sh, int c,
                                                unsigned char* slot, int piece0, int piece1,
                                                const void* dummy) {
  unsigned char* szs = slot + kStreamCodeBytes;
  if (P.sv[0]) {
    const int rowlast = sh.rank * 2 - 16;
    __builtin_amdgcn_global_load_lds((const void*)(P.sv[0] + min(128 * c + piece0, rowlast)),
                                     (lds_void*)slot, 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(P.sv[1] + min(128 * c + piece1, rowlast)),
                                     (lds_void*)(slot + 1024), 16, 0, 0);
  } else {  // bias only: two dummy loads keep the instruction count
    __builtin_amdgcn_global_load_lds(dummy, (lds_void*)slot, 4, 0, 0);
    __builtin_amdgcn_global_load_lds(dummy, (lds_void*)(slot + 1024), 4, 0, 0);
  }
  const void* src = P.bias ? (const void*)P.bias : dummy;
  __builtin_amdgcn_global_load_lds(src, (lds_void*)szs, 4, 0, 0);
  if constexpr (SZ2) __builtin_amdgcn_global_load_lds(src, (lds_void*)(szs + 256), 4, 0, 0);
}

// Per-lane constants of the consume loop (computed once per workgroup).
template <int MP>
struct StreamLane {
  int code_off[2];  // byte offset of this lane's 16 B in a slot, per step
  int xa[MP];       // half offset of this lane's x operand row (or the zero block)
  int xstep[MP];    // halves per 256-code step along that row (0 for the zero block)
  int xcb[MP];      // unused (kept for layout symmetry)
  int szb;          // byte offset of the main-path scale dword (step 0)
  int szstep;       // bytes between the scale dwords of steps 0 and 1
  int cszb;         // byte offset of the correction scale dword (group kb)
  int czoff;        // bytes from a scale dword to its zero-point dword
  int h;            // 2-bit: group-half of this lane's D rows and codes
};

// v_mfma_f32_16x16x4_f32: A 16x4, B 4x16 fp32, used for the zero-point and
// operand-bias correction over the groups of a chunk.
__device__ __forceinline__ f32x4 mfma_16x16x4f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The half selected by `sh16` (0 or 16) of an fp16 pair, as float.
__device__ __forceinline__ float half_of(uint32_t w, int sh16) {
  return __half2float(__ushort_as_half((uint16_t)(w >> sh16)));
}

// Consumes one code chunk (2 steps) of a tile from its LDS slot.
//   yacc += s_g * (MFMA sum of (2^e + q) x - c1_g) per step, the operand bias
//   c1 = sum 2^e x of each D row's (token, group) leaving before the scale
//   (so no sum of large terms runs across groups), and
//   corr -= sum_g (s_g z_g) c2_g over the chunk's groups, as one fp32 MFMA
//   (A = c2 of tokens x groups, B = s*z of groups x rows).
// D rows: 4-bit, token 4kb+i of the step's group; 2-bit, token 8p + 4(kb&1)+i
// of half kb>>1.  A group past K (2-bit tail) gets scale 0; `par*` select the
// fp16 half of each staged scale dword.
template <int BITS, int MP, bool SYM>
__device__ __forceinline__ void stream_consume(const unsigned char* slot, int ch, int par0,
                                               int par1, int cpar, const StreamShape& sh,
                                               const __half* xs, const float* xc,
                                               f32x4 (&yacc)[MP], f32x4& corr,
                                               const StreamLane<MP>& ln, const DecodeConsts& dk,
                                               int li, int kb) {
  // symmetric codes are b-bit two's complement: flipping the top bit maps
  // them to q + 2^(b-1), whose zero-point is 2^(b-1)
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  constexpr int GPC = BITS == 2 ? 4 : 2;  // groups per chunk
  const unsigned char* sz = slot + kStreamCodeBytes;
  // ---- correction for the chunk's groups (lane: row li, group kb) ----
  {
    const int g = GPC * ch + kb;
    const bool gv = kb < GPC && g * 128 < sh.K;
    const uint32_t sw_ = *(const uint32_t*)(sz + ln.cszb);
    const float sc = gv ? half_of(sw_, 16 * cpar) : 0.f;
    float zc = (float)(1 << (BITS - 1));
    if constexpr (!SYM)
      zc = half_of(*(const uint32_t*)(sz + ln.cszb + ln.czoff), 16 * cpar) + sh.zoff;
    const int gi = min(g, (stream_kpad(sh.K, BITS) >> 7) - 1);
    const float c2 = xc[gi * 32 + 16 + li];
    corr = mfma_16x16x4f32(c2, -sc * zc, corr);
  }
#pragma unroll
  for (int sp = 0; sp < 2; ++sp) {
    u32x4 w = *(const u32x4*)(slot + ln.code_off[sp]);
    if constexpr (SYM) w ^= xor_mask;
    const int st = 2 * ch + sp;
    const int c128 = BITS == 2 ? 2 * st + ln.h : st;
    const uint32_t sw_ = *(const uint32_t*)(sz + ln.szb + sp * ln.szstep);
    float s = half_of(sw_, 16 * (sp ? par1 : par0));
    s = c128 * 128 < sh.K ? s : 0.f;
    f32x4 cb[MP];  // c1 of the lane's D rows
#pragma unroll
    for (int p = 0; p < MP; ++p)
      cb[p] = *(const f32x4*)(xc + c128 * 32 + (BITS == 2 ? 8 * p + 4 * (kb & 1) : 4 * kb));
    f32x4 acc[MP];
#pragma unroll
    for (int p = 0; p < MP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (BITS == 2) {
        f16x8 b0, b1;
        decode2(w[i], b0, b1, dk);
#pragma unroll
        for (int p = 0; p < MP; ++p) {
          const __half* xr = xs + ln.xa[p] + st * ln.xstep[p] + 16 * i;
          acc[p] = mfma_16x16x32(*(const f16x8*)xr, b0, acc[p]);
          acc[p] = mfma_16x16x32(*(const f16x8*)(xr + 8), b1, acc[p]);
        }
      } else {
        const __half* xr = xs + ln.xa[0] + st * ln.xstep[0] + 8 * i;
        acc[0] = mfma_16x16x32(*(const f16x8*)xr, decode4(w[i], dk), acc[0]);
      }
    }
#pragma unroll
    for (int p = 0; p < MP; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i) yacc[p][i] = fmaf(s, acc[p][i] - cb[p][i], yacc[p][i]);
  }
}

// Post chunk of the two-matrix form: lane j accumulates, for every token m of
// the unit, sum_n inter[m][n] * Upost[n][64q + j] over the tile's 16 rows
// into the wave's partials pl[m][64q + j].  Upost rows sit in the slot like SV
// rows (row n at n*128 B, 16-byte piece p at position p ^ ((n/2) % 8)).
__device__ __forceinline__ void stream_post(const unsigned char* slot, int q, int M,
                                            const float* tl, float* pl, int pcols, int lane) {
  float u[16];
#pragma unroll
  for (int n = 0; n < 16; ++n)
    u[n] = __half2float(*(const __half*)(slot + n * 128 + ((((lane >> 3) ^ (n >> 1)) & 7) << 4) +
                                         (lane & 7) * 2));
  const int j = 64 * q + lane;
  for (int m = 0; m < M; ++m) {
    const f32x4* t4 = (const f32x4*)(tl + m * 16);
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 t = t4[v];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = fmaf(t[i], u[4 * v + i], acc);
    }
    pl[m * pcols + j] += acc;
  }
}

// Stages, for one work unit, the x rows (zero-padded, permuted into MFMA
// operand order), their per-128-code sums c1 = sum(operand bias * x) and
// c2 = sum(x), the zero block, and the low-rank inputs a of the matrices with
// a low-rank term.  x blocks and a elements share one loop, so their global
// loads go out together (one memory round trip for the whole prologue).
template <int BITS, int NMAT, class Src>
__device__ void stream_stage(const Src& src, const StreamShape& sh, int item, int M, bool lora0,
                             bool lora1, __half* xs, float* xc, __half* a_l, int tid) {
  const int kpad = stream_kpad(sh.K, BITS);
  const int nb = kpad >> 4;           // 16-code blocks per padded token row
  const int totalb = sh.mmax * nb;    // a multiple of 8: shuffle groups stay whole
  const int na0 = lora0 ? M * sh.rank : 0;
  const int na1 = NMAT == 2 && lora1 ? M * sh.rank : 0;
  const int total = totalb + na0 + na1;
  for (int base = 0; base < total; base += 256) {
    const int idx = base + tid;
    const bool v = idx < totalb;
    float s = 0.f, sb = 0.f;
    int m = 0, blk = 0;
    if (v) {
      m = idx / nb;
      blk = idx - m * nb;
      _Float16 in[16], o[16];
      if (m < M && blk * 16 < sh.K) {
        const f16x8* srcx = (const f16x8*)(src.xrow(item, m) + blk * 16);
        const f16x8 in0 = srcx[0], in1 = srcx[1];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          in[c] = in0[c];
          in[8 + c] = in1[c];
        }
      } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) in[c] = (_Float16)0.f;
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
      f16x8* dst = (f16x8*)(xs + m * sh.xstride + blk * 16);
      dst[0] = o0;
      dst[1] = o1;
    } else if (idx < total) {
      const int ai = idx - totalb;
      const int sm = ai < na0 ? 0 : 1;
      const int r = ai - (sm ? na0 : 0);
      const int am = r / sh.rank, j = r - am * sh.rank;
      a_l[(sm * 16 + am) * sh.apad + j] = src.load_a(item, sm, am, j);
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    sb += __shfl_xor(sb, 1);
    sb += __shfl_xor(sb, 2);
    sb += __shfl_xor(sb, 4);
    if (v && (idx & 7) == 0 && m < sh.mmax) {
      const int c128 = blk >> 3;
      xc[c128 * 32 + m] = sb;      // c1: sum of operand bias * x
      xc[c128 * 32 + 16 + m] = s;  // c2: sum of x
    }
  }
  for (int idx = tid; idx < 128; idx += 256)  // the zero block
    ((uint32_t*)(xs + sh.mmax * sh.xstride))[idx] = 0u;
  // tokens mmax..15 of every chunk read as zero
  const int nc = kpad >> 7, nz = 16 - sh.mmax;
  for (int idx = tid; idx < nc * nz; idx += 256) {
    const int c128 = idx / nz, m = sh.mmax + idx % nz;
    xc[c128 * 32 + m] = 0.f;
    xc[c128 * 32 + 16 + m] = 0.f;
  }
  // a: zero outside tokens < M and columns < rank (the SV chunks read
  // columns up to 64 * nsvc)
#pragma unroll
  for (int sm = 0; sm < NMAT; ++sm) {
    if (!(sm == 0 ? lora0 : lora1)) continue;
    __half* as = a_l + sm * 16 * sh.apad;
    for (int idx = tid; idx < 16 * sh.apad; idx += 256) {
      const int m = idx / sh.apad, j = idx - m * sh.apad;
      if (m >= M || j >= sh.rank) as[idx] = __float2half(0.f);
    }
  }
}

// Per-lane constants of the consume loop.
template <int BITS, int MP, bool SZ2>
__device__ __forceinline__ StreamLane<MP> stream_lane(const StreamShape& sh, int M, int li,
                                                      int kb) {
  StreamLane<MP> ln;
  const int sw = (li >> 1) & 7;
#pragma unroll
  for (int sp = 0; sp < 2; ++sp) ln.code_off[sp] = li * 128 + (((4 * sp + kb) ^ sw) << 4);
  const int zrow = sh.mmax * sh.xstride;
  if constexpr (BITS == 2) {
    ln.h = kb >> 1;
#pragma unroll
    for (int p = 0; p < MP; ++p) {
      const int m = (li & 7) + 8 * p;
      const bool act = ((li >> 3) == ln.h) && m < M;
      ln.xa[p] = act ? m * sh.xstride + 64 * kb : zrow;
      ln.xstep[p] = act ? 256 : 0;
      ln.xcb[p] = 0;
    }
    if constexpr (SZ2) {  // dword (row*4 + group%4); z 256 B after s
      ln.szb = 4 * (li * 4 + ln.h);
      ln.szstep = 8;
      ln.cszb = 4 * (li * 4 + kb);
      ln.czoff = 256;
    } else {              // dword (row*2 + group%4/2) holds groups 2j, 2j+1; z 128 B after s
      ln.szb = 8 * li;
      ln.szstep = 4;
      ln.cszb = 8 * li + 4 * (kb >> 1);
      ln.czoff = 128;
    }
  } else {
    ln.h = 0;
    ln.xa[0] = li < M ? li * sh.xstride + 32 * kb : zrow;
    ln.xstep[0] = li < M ? 128 : 0;
    ln.xcb[0] = 0;
    ln.szb = 8 * li;
    ln.szstep = 4;
    ln.cszb = 8 * li + 4 * (kb & 1);
    ln.czoff = 128;
  }
  return ln;
}

// fp16 half of each staged scale dword (main-path steps 0/1, correction) for
// the tile at row r0.
template <int BITS, bool SZ2>
__device__ __forceinline__ void stream_parities(const StreamShape& sh, int r0, int li, int kb,
                                                int h, int& par0, int& par1, int& cpar) {
  const int rowpar = (int)(((int64_t)min(r0 + li, sh.N - 1) * sh.G + sh.goff) & 1);
  if constexpr (BITS == 2 && SZ2) {
    par0 = par1 = rowpar ^ h;
    cpar = rowpar ^ (kb & 1);
  } else if constexpr (BITS == 2) {
    par0 = par1 = h;
    cpar = kb & 1;
  } else {
    par0 = rowpar;
    par1 = rowpar ^ 1;
    cpar = rowpar ^ (kb & 1);
  }
}

// The 2-bit half sums merged into the standard MFMA layout D[token 4kb+i][row li].
template <int BITS, int MP>
__device__ __forceinline__ f32x4 stream_merge(const f32x4 (&yacc)[MP], int kb) {
  if constexpr (BITS == 2) {
    f32x4 ya = yacc[0], yb = yacc[MP - 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ya[i] += __shfl_xor(ya[i], 32);
      if (MP == 2) yb[i] += __shfl_xor(yb[i], 32);
    }
    return kb < 2 ? ya : (MP == 2 ? yb : f32x4{0.f, 0.f, 0.f, 0.f});
  } else {
    return yacc[0];
  }
}

// One workgroup: tiles [t0, t1) of one work unit; wave w takes t0 + w,
// t0 + w + 4, ...  Src supplies the unit: m_rows, xrow (x row m, offset to
// the K range), mat(item, s) (StreamMat of matrix s), load_a(item, s, m, j)
// (the low-rank input a = x U of matrix s), and
//  * NMAT = 1: store(item, m, n, y) with y = Q(x) + a SV^T + bias.
//  * NMAT = 2 (gate and up of a SwiGLU MLP over the same x): each tile runs
//    matrix 0 then matrix 1; store_inter(item, m, n, inter) with
//    inter = fp16(silu(fp16 y0) * fp16 y1).  If post(item) gives the input
//    factor Upost (N x rank) of the projection that consumes inter, the
//    workgroup also forms sum_n inter[m][n] Upost[n][j] over its tiles and
//    hands it to store_post(item, m, j, partial) (one partial per workgroup).
template <int BITS, int MP, int D, bool SYM, bool SZ2, int NMAT, class Src>
__device__ void gemv_stream(const Src& src, const StreamShape& sh, int item, int t0, int t1,
                            unsigned char* smem) {
  static_assert(NMAT == 1 || NMAT == 2, "one or two matrices per tile");
  constexpr int NI = stream_ni<SZ2>();
  constexpr int SLOT = stream_slot<SZ2>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int M = src.m_rows(item);

  // Segments of a tile: matrix 0 [, matrix 1, post rows].  Scalars, not
  // arrays, so that no runtime index sends them to scratch memory.
  StreamMat mat0 = src.mat(item, 0);
  StreamMat mat1 = NMAT == 2 ? src.mat(item, 1) : mat0;
  if (sh.rank <= 0) mat0.SV = mat1.SV = nullptr;  // SV rows are read only with a rank
  if (NMAT == 2) mat0.B = mat1.B = nullptr;       // no bias in the two-matrix form
  const bool lora0 = mat0.SV != nullptr;
  const bool lora1 = NMAT == 2 && mat1.SV != nullptr;
  const __half* PU = nullptr;
  if constexpr (NMAT == 2) PU = sh.rank > 0 ? src.post(item) : nullptr;
  const int pcols = PU ? 64 * sh.nsvc : 0;
  // chunks of matrix s: codes, then SV chunks (or one bias chunk, NMAT == 1)
  const int seg0 = sh.nchunk + (lora0 ? sh.nsvc : (mat0.B ? 1 : 0));
  const int seg1 = NMAT == 2 ? sh.nchunk + (lora1 ? sh.nsvc : 0) : 0;
  const int seg2 = PU ? sh.nsvc : 0;
  const int cpt = seg0 + seg1 + seg2;  // chunks per tile
  auto seg_len = [&](int sg) { return sg == 0 ? seg0 : (sg == 1 ? seg1 : seg2); };
  auto seg_mat = [&](int sg) -> StreamMat {
    if (sg == 0) return mat0;
    if (sg == 1) return mat1;
    return StreamMat{mat0.C, mat0.S, mat0.Z, PU, nullptr};
  };
  // next segment after sg; returns true when the tile is complete
  auto next_seg = [&](int& sg) -> bool {
    if constexpr (NMAT == 1) {
      return true;
    } else {
      ++sg;
      if (sg == 2 && !PU) sg = 3;
      if (sg == 3) {
        sg = 0;
        return true;
      }
      return false;
    }
  };

  const StreamLds L = stream_lds(D, SLOT, sh.mmax, sh.K, BITS, sh.xstride, sh.apad, NMAT, pcols);
  __half* xs = (__half*)(smem + L.xs);  // mmax rows, then a 512-byte zero block
  float* xc = (float*)(smem + L.xc);    // [c128][c1 x16 | c2 x16]
  __half* a_l = (__half*)(smem + L.a);  // [matrix][16][apad]
  unsigned char* ring = smem + L.ring + wave * D * SLOT;
  float* tlw = (float*)(smem + L.tl) + wave * 256;              // [m][16] inter tile
  float* plw = (float*)(smem + L.pl) + wave * sh.mmax * pcols;  // [m][pcols]

  // This wave's work list: tiles t0 + wave + 4j, cpt chunks each.
  const int ntile_w = t1 - t0 > wave ? (t1 - t0 - wave + 3) / 4 : 0;
  const int total = ntile_w * cpt;

  // byte offsets of this lane's 16-byte pieces within a 128-byte chunk row
  const int piece0 = 16 * ((lane & 7) ^ (((lane >> 3) >> 1) & 7));
  const int piece1 = 16 * ((lane & 7) ^ (((8 + (lane >> 3)) >> 1) & 7));
  const void* dummy = (const void*)mat0.C;
  StreamCursor<BITS, SZ2> cur;
  int cur_sg = 0;
  cur.r0 = (t0 + wave) * 16;
  cur.retarget(mat0, sh, lane);
  int issued = 0;
  auto issue_next = [&]() {
    unsigned char* slot = ring + cur.slot * SLOT;
    if (cur_sg < NMAT && cur.c < sh.nchunk)
      stream_issue<BITS, SZ2>(cur.P, sh, cur.c, slot, lane, piece0, piece1);
    else
      stream_issue_sv<SZ2>(cur.P, sh, cur_sg < NMAT ? cur.c - sh.nchunk : cur.c, slot, piece0,
                           piece1, dummy);
    if (++cur.slot == D) cur.slot = 0;
    ++issued;
    if (++cur.c == seg_len(cur_sg)) {
      cur.c = 0;
      if (next_seg(cur_sg)) cur.r0 += 64;
      cur.retarget(seg_mat(cur_sg), sh, lane);
    }
  };

  // ---- prologue: D-1 chunks in flight, then stage x, its sums, and a ----
  for (int u = 0; u < D - 1 && u < total; ++u) issue_next();

  stream_stage<BITS, NMAT>(src, sh, item, M, lora0, lora1, xs, xc, a_l, tid);
  for (int idx = lane; idx < sh.mmax * pcols; idx += 64) plw[idx] = 0.f;
  __syncthreads();
  const StreamLane<MP> ln = stream_lane<BITS, MP, SZ2>(sh, M, li, kb);

  // ---- stream: consume chunk u while chunks u+1 .. u+D-1 are in flight ----
  const DecodeConsts dk = DecodeConsts::make();
  f32x4 yacc[MP];
#pragma unroll
  for (int p = 0; p < MP; ++p) yacc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 corr = {0.f, 0.f, 0.f, 0.f};
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  f32x4 y0 = {0.f, 0.f, 0.f, 0.f};  // matrix 0 result of the two-matrix form
  int c = 0, sg = 0, slot = 0;
  int r0 = (t0 + wave) * 16;
  // fp16 half of each staged scale dword: main path steps 0/1 and correction
  int par0, par1, cpar;
  auto parities = [&]() {
    const int rowpar = (int)(((int64_t)min(r0 + li, sh.N - 1) * sh.G + sh.goff) & 1);
    if constexpr (BITS == 2 && SZ2) {
      par0 = par1 = rowpar ^ ln.h;
      cpar = rowpar ^ (kb & 1);
    } else if constexpr (BITS == 2) {
      par0 = par1 = ln.h;
      cpar = kb & 1;
    } else {
      par0 = rowpar;
      par1 = rowpar ^ 1;
      cpar = rowpar ^ (kb & 1);
    }
  };
  parities();
  for (int u = 0; u < total; ++u) {
    if (issued < total) {
      wait_lgkm0();  // slot (u-1)%D: every LDS read of it has completed
      issue_next();
      wait_vmcnt<NI * (D - 1)>();
    } else {
      wait_vmcnt<0>();
    }
    const unsigned char* sl = ring + slot * SLOT;
    if (++slot == D) slot = 0;
    if (sg < NMAT && c < sh.nchunk) {
      stream_consume<BITS, MP, SYM>(sl, c, par0, par1, cpar, sh, xs, xc, yacc, corr, ln, dk, li,
                                    kb);
      if (c == sh.nchunk - 1) {
        // the tile's code sums: merge the 2-bit halves into the standard
        // MFMA layout D[token 4kb+i][row li], then add the correction
        if constexpr (BITS == 2) {
          f32x4 ya = yacc[0], yb = yacc[MP - 1];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ya[i] += __shfl_xor(ya[i], 32);
            if (MP == 2) yb[i] += __shfl_xor(yb[i], 32);
          }
          y = kb < 2 ? ya : (MP == 2 ? yb : f32x4{0.f, 0.f, 0.f, 0.f});
        } else {
          y = yacc[0];
        }
        y += corr;
        corr = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < MP; ++p) yacc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    } else if (sg < NMAT) {
      if (sg == 0 ? lora0 : lora1) {
        // SV chunk: rank columns 64(c - nchunk) .. +64 of this tile's rows
        const int j0 = 64 * (c - sh.nchunk);
        const __half* as = a_l + (NMAT == 1 ? 0 : sg) * 16 * sh.apad;
#pragma unroll
        for (int sp = 0; sp < 2; ++sp) {
          const f16x8 bv = *(const f16x8*)(sl + ln.code_off[sp]);
          const f16x8 av = *(const f16x8*)(as + li * sh.apad + j0 + 32 * sp + 8 * kb);
          y = mfma_16x16x32(av, bv, y);
        }
      }
    } else {
      stream_post(sl, c, M, tlw, plw, pcols, lane);
    }
    if (++c == seg_len(sg)) {
      const int n = r0 + li;
      if constexpr (NMAT == 1) {
        // ---- tile epilogue: bias (in the last SV chunk's slot) and store ----
        if (n < sh.N) {
          const float bn =
              mat0.B ? __half2float(((const __half*)(sl + kStreamCodeBytes))[li]) : 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * kb + i;
            if (m < M) src.store(item, m, n, y[i] + bn);
          }
        }
      } else {
        if (sg == 0) {
          y0 = y;
        } else if (sg == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * kb + i;
            const __half v = swiglu_fp16(y0[i], y[i]);
            if (m < M && n < sh.N) src.store_inter(item, m, n, v);
            tlw[m * 16 + li] = n < sh.N ? __half2float(v) : 0.f;
          }
        }
        y = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      c = 0;
      if (next_seg(sg)) {
        r0 += 64;
        parities();
      }
    }
  }
  if constexpr (NMAT == 2) {
    if (PU) {  // workgroup sum of the waves' partials
      __syncthreads();
      const float* pl0 = (const float*)(smem + L.pl);
      const int wstride = sh.mmax * pcols;
      for (int idx = tid; idx < M * sh.rank; idx += 256) {
        const int m = idx / sh.rank, j = idx - m * sh.rank;
        const int o = m * pcols + j;
        src.store_post(item, m, j, pl0[o] + pl0[wstride + o] + pl0[2 * wstride + o] +
                                       pl0[3 * wstride + o]);
      }
    }
  }
}

// LDS of the K-split form's partial tiles: two buffers x 4 waves x NMAT x 16x16 floats.
__host__ __device__ inline int stream_ks_bytes(int nmat) { return 2 * 4 * nmat * 256 * 4; }

// K-split form of gemv_stream (same Src interface and results): all four waves
// work on every tile of [t0, t1).  A tile's chunk list (matrix 0 code chunks,
// its SV chunks or bias chunk, [matrix 1 code chunks, SV chunks,] post chunks)
// is dealt round-robin, chunk c to wave c % 4, so each wave's serial chain is a
// quarter of the tile; the waves' partial tiles (codes + zero-point correction
// + low-rank term + bias) meet in LDS after one barrier per tile
// (double-buffered, summed in wave order: deterministic), every wave forms the
// whole tile, wave w stores tokens 4w..4w+3, and a wave holding a post chunk
// consumes it after the barrier from the tile's inter values.  For launches
// with few tiles per workgroup, where one wave per tile leaves each SIMD with a
// single latency-bound wave.
template <int BITS, int MP, int D, bool SYM, bool SZ2, int NMAT, class Src>
__device__ void gemv_stream_ks(const Src& src, const StreamShape& sh, int item, int t0, int t1,
                               unsigned char* smem) {
  static_assert(NMAT == 1 || NMAT == 2, "one or two matrices per tile");
  constexpr int NI = stream_ni<SZ2>();
  constexpr int SLOT = stream_slot<SZ2>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int M = src.m_rows(item);

  StreamMat mat0 = src.mat(item, 0);
  StreamMat mat1 = NMAT == 2 ? src.mat(item, 1) : mat0;
  if (sh.rank <= 0) mat0.SV = mat1.SV = nullptr;
  if (NMAT == 2) mat0.B = mat1.B = nullptr;
  const bool lora0 = mat0.SV != nullptr;
  const bool lora1 = NMAT == 2 && mat1.SV != nullptr;
  const __half* PU = nullptr;
  if constexpr (NMAT == 2) PU = sh.rank > 0 ? src.post(item) : nullptr;
  const int pcols = PU ? 64 * sh.nsvc : 0;
  const int seg0 = sh.nchunk + (lora0 ? sh.nsvc : (mat0.B ? 1 : 0));
  const int seg1 = NMAT == 2 ? sh.nchunk + (lora1 ? sh.nsvc : 0) : 0;
  const int seg2 = PU ? sh.nsvc : 0;
  const int nmain = seg0 + seg1;
  const int cpt = nmain + seg2;
  auto seg_of = [&](int c, int& lc) -> int {
    if (c < seg0) {
      lc = c;
      return 0;
    }
    if (c < nmain) {
      lc = c - seg0;
      return 1;
    }
    lc = c - nmain;
    return 2;
  };
  auto seg_mat = [&](int sg) -> StreamMat {
    if (sg == 0) return mat0;
    if (sg == 1) return mat1;
    return StreamMat{mat0.C, mat0.S, mat0.Z, PU, nullptr};
  };

  const StreamLds L = stream_lds(D, SLOT, sh.mmax, sh.K, BITS, sh.xstride, sh.apad, NMAT, pcols);
  __half* xs = (__half*)(smem + L.xs);
  float* xc = (float*)(smem + L.xc);
  __half* a_l = (__half*)(smem + L.a);
  unsigned char* ring = smem + L.ring + wave * D * SLOT;
  float* tlw = (float*)(smem + L.tl) + wave * 256;
  float* plw = (float*)(smem + L.pl) + wave * sh.mmax * pcols;
  float* red = (float*)(smem + L.total);  // [buffer][wave][matrix][256]

  const int ntile = t1 > t0 ? t1 - t0 : 0;
  const int nw = cpt > wave ? (cpt - wave + 3) / 4 : 0;  // this wave's chunks per tile
  const int total = ntile * nw;

  const int piece0 = 16 * ((lane & 7) ^ (((lane >> 3) >> 1) & 7));
  const int piece1 = 16 * ((lane & 7) ^ (((8 + (lane >> 3)) >> 1) & 7));
  const void* dummy = (const void*)mat0.C;
  StreamCursor<BITS, SZ2> cur;
  cur.r0 = -1;
  int i_t = 0, i_c = wave, i_sg = -1, issued = 0;
  auto issue_next = [&]() {
    int lc;
    const int sg = seg_of(i_c, lc);
    const int r0 = (t0 + i_t) * 16;
    if (sg != i_sg || r0 != cur.r0) {
      cur.r0 = r0;
      cur.retarget(seg_mat(sg), sh, lane);
      i_sg = sg;
    }
    unsigned char* slot = ring + cur.slot * SLOT;
    if (sg < NMAT && lc < sh.nchunk)
      stream_issue<BITS, SZ2>(cur.P, sh, lc, slot, lane, piece0, piece1);
    else
      stream_issue_sv<SZ2>(cur.P, sh, sg < NMAT ? lc - sh.nchunk : lc, slot, piece0, piece1,
                           dummy);
    if (++cur.slot == D) cur.slot = 0;
    ++issued;
    i_c += 4;
    if (i_c >= cpt) {
      i_c = wave;
      ++i_t;
    }
  };

  // ---- prologue ----
  for (int u = 0; u < D - 1 && u < total; ++u) issue_next();
  stream_stage<BITS, NMAT>(src, sh, item, M, lora0, lora1, xs, xc, a_l, tid);
  for (int idx = lane; idx < sh.mmax * pcols; idx += 64) plw[idx] = 0.f;
  __syncthreads();
  const StreamLane<MP> ln = stream_lane<BITS, MP, SZ2>(sh, M, li, kb);
  const DecodeConsts dk = DecodeConsts::make();

  int slot = 0, buf = 0;
  auto next_slot = [&]() -> const unsigned char* {
    if (issued < total) {
      wait_lgkm0();
      issue_next();
      wait_vmcnt<NI * (D - 1)>();
    } else {
      wait_vmcnt<0>();
    }
    const unsigned char* sl = ring + slot * SLOT;
    if (++slot == D) slot = 0;
    return sl;
  };

  for (int tt = 0; tt < ntile; ++tt) {
    const int r0 = (t0 + tt) * 16;
    int par0, par1, cpar;
    stream_parities<BITS, SZ2>(sh, r0, li, kb, ln.h, par0, par1, cpar);
    f32x4 yacc0[MP], yacc1[MP];
#pragma unroll
    for (int p = 0; p < MP; ++p) yacc0[p] = yacc1[p] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 corr0 = {0.f, 0.f, 0.f, 0.f}, corr1 = corr0, ysv0 = corr0, ysv1 = corr0;
    int c = wave;
    for (; c < nmain; c += 4) {
      const unsigned char* sl = next_slot();
      int lc;
      const int sg = seg_of(c, lc);
      if (lc < sh.nchunk) {
        if (sg == 0)
          stream_consume<BITS, MP, SYM>(sl, lc, par0, par1, cpar, sh, xs, xc, yacc0, corr0, ln,
                                        dk, li, kb);
        else
          stream_consume<BITS, MP, SYM>(sl, lc, par0, par1, cpar, sh, xs, xc, yacc1, corr1, ln,
                                        dk, li, kb);
      } else {
        if (sg == 0 ? lora0 : lora1) {
          const int j0 = 64 * (lc - sh.nchunk);
          const __half* as = a_l + sg * 16 * sh.apad;
          f32x4 ysv = sg == 0 ? ysv0 : ysv1;
#pragma unroll
          for (int sp = 0; sp < 2; ++sp) {
            const f16x8 bv = *(const f16x8*)(sl + ln.code_off[sp]);
            const f16x8 av = *(const f16x8*)(as + li * sh.apad + j0 + 32 * sp + 8 * kb);
            ysv = mfma_16x16x32(av, bv, ysv);
          }
          if (sg == 0)
            ysv0 = ysv;
          else
            ysv1 = ysv;
        }
        if (NMAT == 1 && mat0.B && lc == seg0 - 1) {  // bias rides in the last chunk
          const float bn = __half2float(((const __half*)(sl + kStreamCodeBytes))[li]);
#pragma unroll
          for (int i = 0; i < 4; ++i) ysv0[i] += bn;
        }
      }
    }
    // ---- partial tiles meet in LDS ----
    float* rb = red + buf * 4 * NMAT * 256;
    {
      const f32x4 p0 = stream_merge<BITS, MP>(yacc0, kb) + corr0 + ysv0;
#pragma unroll
      for (int i = 0; i < 4; ++i) rb[(wave * NMAT) * 256 + (4 * kb + i) * 16 + li] = p0[i];
      if constexpr (NMAT == 2) {
        const f32x4 p1 = stream_merge<BITS, MP>(yacc1, kb) + corr1 + ysv1;
#pragma unroll
        for (int i = 0; i < 4; ++i) rb[(wave * NMAT + 1) * 256 + (4 * kb + i) * 16 + li] = p1[i];
      }
    }
    __syncthreads();
    f32x4 y0 = {0.f, 0.f, 0.f, 0.f}, y1 = y0;
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y0[i] += rb[(w * NMAT) * 256 + (4 * kb + i) * 16 + li];
        if (NMAT == 2) y1[i] += rb[(w * NMAT + 1) * 256 + (4 * kb + i) * 16 + li];
      }
    buf ^= 1;
    const int n = r0 + li;
    if constexpr (NMAT == 1) {
      if (kb == wave && n < sh.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * kb + i < M) src.store(item, 4 * kb + i, n, y0[i]);
      }
    } else {
      const bool post = c < cpt;  // this wave holds a post chunk of the tile
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * kb + i;
        const __half v = swiglu_fp16(y0[i], y1[i]);
        if (kb == wave && m < M && n < sh.N) src.store_inter(item, m, n, v);
        if (post) tlw[m * 16 + li] = n < sh.N ? __half2float(v) : 0.f;
      }
      for (; c < cpt; c += 4) {
        const unsigned char* sl = next_slot();
        stream_post(sl, c - nmain, M, tlw, plw, pcols, lane);
      }
    }
  }
  if constexpr (NMAT == 2) {
    if (PU) {  // workgroup sum of the waves' partials
      __syncthreads();
      const float* pl0 = (const float*)(smem + L.pl);
      const int wstride = sh.mmax * pcols;
      for (int idx = tid; idx < M * sh.rank; idx += 256) {
        const int m = idx / sh.rank, j = idx - m * sh.rank;
        const int o = m * pcols + j;
        src.store_post(item, m, j, pl0[o] + pl0[wstride + o] + pl0[2 * wstride + o] +
                                       pl0[3 * wstride + o]);
      }
    }
  }
}

}  // namespace glq
