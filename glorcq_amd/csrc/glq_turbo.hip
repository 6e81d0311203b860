// TurboQuant 2-bit codebook GEMV/GEMM (the reference's own 2-bit expert format):
//
//   y[m][n] = fp16(norms[n] * sum_k C[q[n][k]] * x_rot[m][k])
//
// (inference/kernels/turbo_matmul.cu:46-137 GEMV, :150-245 GEMM, :329-415 the
// grouped form; inference/kernels/__init__.py:121-146 the fallback).  q are
// 2-bit codebook indices packed 4 per byte LSB-first, i.e. exactly this
// library's 2-bit int32 container read little-endian; C is a 4-entry fp32
// codebook; x_rot the rotated input (x Pi^T, or the randomized Hadamard
// transform of x).
//
// turbo_gemv_kernel: a workgroup covers one (item, 16-token block) and 4/wpt
// tiles of 16 rows; the wpt waves of a tile split K into contiguous parts
// (wpt = 1 for large problems, 2 or 4 when there are too few tiles to fill
// the chip) and meet in LDS at the end.  The token rows of x_rot are staged in
// LDS per K segment (the whole K unless 16 tokens of a long row would not
// fit), permuted into the decode order below.
//
// Decode is a byte permutation (v_perm_b32) into an fp16 codebook held as two
// dwords: low bytes of C0..C3 and high bytes of C0..C3.  For X = (w >> 2s) &
// 0x03030303 (codes s, s+4, s+8, s+12 of the word, one per byte) and X4 =
// X | 0x04040404, one permutation of (X4, X) gives the selector of a code pair
// (a, a+4, b, b+4) and a second one looks up (C[a], C[b]).  The codebook is
// split into fp16 hi + lo parts (C = hi + lo to ~22 bits) sharing the
// selectors, one MFMA each, so the fp32-accumulated sum keeps fp32-level
// accuracy like the reference's fp32 FMA loop; y = fp16(acc * norm) as in the
// reference.
#include <algorithm>

#include "glq_gemv_core.h"

namespace glq {

constexpr int kTurboXBudget = 64 * 1024;      // LDS bytes for one x segment (one-shot form)
constexpr int kTurboStreamTiles = 2048;       // tiles from which the streaming form is used
constexpr int kTurboStreamWgs = 1024;         // its workgroups, about 4 per CU
constexpr int kTurboStreamLds = 80 * 1024;    // its LDS limit (the whole K of 16 tokens)
constexpr int kTurboPF = 8;                   // steps of codes in flight per wave

struct TurboArgs {
  const __half* x;         // x_rot (items, M, K) fp16
  int64_t x_es;            // elements between items (0: one x for all)
  const uint32_t* codes;   // (items, N, K/16) int32 words (= (N, K/4) bytes)
  int64_t c_es;
  const float* norms;      // (items, N)
  int64_t n_es;
  const float* cent;       // (4,) fp32 codebook
  const __half* xu;        // a = fp16(x U): (items, M, rank), or nullptr
  int64_t xu_es;
  const __half* sv;        // SV (items, N, rank), or nullptr: no low-rank term
  int64_t sv_es;
  const __half* bias;      // (items, N), or nullptr
  int64_t bias_es;
  __half* y;               // (items, M, N)
  int64_t y_es;
  int M, K, N, kw;
  int rank, rpad, apad;    // low-rank width, padded to 32, LDS row stride of a
  int segsteps;            // 256-code steps per staged x segment
  int xstride;             // halves per staged token row (segment + 8)
  int wpt;                 // waves per 16-row tile: 1, 2 or 4 (K split among them)
  int rwgs, twgs;          // row groups (4/wpt tiles) and token blocks (16 tokens) per item
  // routed picks of a MoE step (glq_turbo_moe_gemv); the plain batched call
  // leaves wsel, xclus and gate null and x_div 1
  const int32_t* wsel = nullptr;  // weight set (codes, norms, SV, bias) of item i: wsel[i] (< nw)
  int nw = 0;
  int x_div = 1;                  // x row of item i: i / x_div
  const int32_t* xclus = nullptr;  // a row of item i: xclus[wsel[i]] * xu_tok + i / x_div (< xu_rows)
  int xu_tok = 0, xu_rows = 0;
  const __half* gate = nullptr;   // (items, M, N): y = fp16(fp16(silu(gate)) * y)
  // a given as fp32 partials instead of xu (M = 1 items): a of item i is
  // fp16(sum over s in order of parts[((blk * pP + s) * pM + t) * rpad + j]),
  // blk = xclus[wsel[i]] and t = i / x_div with xclus (a per (cluster,
  // token)), else blk = i and t = 0
  const float* parts = nullptr;
  int pP = 0, pM = 1, pB = 1;  // slices, token rows and blocks of parts
};

// Weight set, x row and low-rank row of an item.
__device__ __forceinline__ int turbo_w(const TurboArgs& a, int item) {
  return a.wsel ? min(max(a.wsel[item], 0), a.nw - 1) : item;
}
__device__ __forceinline__ int64_t turbo_xrow(const TurboArgs& a, int item) {
  return item / a.x_div;
}
__device__ __forceinline__ int64_t turbo_arow(const TurboArgs& a, int item) {
  if (!a.xclus) return item;
  const int64_t r = (int64_t)a.xclus[turbo_w(a, item)] * a.xu_tok + item / a.x_div;
  return min(max(r, (int64_t)0), (int64_t)a.xu_rows - 1);
}

// fp16 codebook in v_perm_b32 form: lb = low bytes of C0..C3, hb = high bytes.
struct TurboLut {
  uint32_t lb, hb;
};

__device__ __forceinline__ TurboLut turbo_lut(const float* c, bool residual) {
  uint32_t lb = 0, hb = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const __half hi = __float2half(c[i]);
    const __half v = residual ? __float2half(c[i] - __half2float(hi)) : hi;
    const uint32_t u = __half_as_ushort(v);
    lb |= (u & 0xffu) << (8 * i);
    hb |= (u >> 8) << (8 * i);
  }
  return TurboLut{lb, hb};
}

// One code word (16 codes) -> the two MFMA operand slices, for the hi and the
// lo codebook: s0 = codes 0,4,1,5,2,6,3,7 and s1 = codes 8,12,9,13,10,14,11,15.
__device__ __forceinline__ void turbo_decode(uint32_t w, const TurboLut& H, const TurboLut& L,
                                             f16x8& s0h, f16x8& s1h, f16x8& s0l, f16x8& s1l) {
  u32x4 ah, bh, al, bl;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t X = (w >> (2 * s)) & 0x03030303u;
    const uint32_t X4 = X | 0x04040404u;
    const uint32_t sa = __builtin_amdgcn_perm(X4, X, 0x05010400u);  // (q_s, q_s+4)
    const uint32_t sb = __builtin_amdgcn_perm(X4, X, 0x07030602u);  // (q_s+8, q_s+12)
    ah[s] = __builtin_amdgcn_perm(H.hb, H.lb, sa);
    bh[s] = __builtin_amdgcn_perm(H.hb, H.lb, sb);
    al[s] = __builtin_amdgcn_perm(L.hb, L.lb, sa);
    bl[s] = __builtin_amdgcn_perm(L.hb, L.lb, sb);
  }
  s0h = __builtin_bit_cast(f16x8, ah);
  s1h = __builtin_bit_cast(f16x8, bh);
  s0l = __builtin_bit_cast(f16x8, al);
  s1l = __builtin_bit_cast(f16x8, bl);
}

// norm * acc + a SV^T + bias of one 16-row tile (fp32), in acc's layout:
// acc[i] of lane (li, kb) holds token 4kb + i, row r0 + li; a_l holds the
// block's low-rank factor a (rows < mr, zero-padded to rpad columns).
// The epilogue's own loads for a lane's row -- its norm, bias and the SV
// fragments of the first kTurboPreBlocks 32-column blocks -- which need
// nothing the tile computes, so the one-shot kernel issues them at its start
// and they arrive under the K loop.
constexpr int kTurboPreBlocks = 2;
struct TurboPre {
  float nr, bb;
  f16x8 sv[kTurboPreBlocks];
};
__device__ __forceinline__ TurboPre turbo_pre(const TurboArgs& a, int item, int r0, int li,
                                              int kb) {
  TurboPre q;
  const int row = min(r0 + li, a.N - 1), w = turbo_w(a, item);
  q.nr = a.norms[(int64_t)w * a.n_es + row];
  q.bb = a.bias ? __half2float(a.bias[(int64_t)w * a.bias_es + row]) : 0.f;
  const __half* svr = a.sv ? a.sv + (int64_t)w * a.sv_es + (int64_t)row * a.rank : nullptr;
#pragma unroll
  for (int b = 0; b < kTurboPreBlocks; ++b) {
    const int j = 32 * b + 8 * kb;
    q.sv[b] = svr && j < a.rank ? *(const f16x8*)(svr + j) : f16x8{};
  }
  // a compiler memory barrier keeps the loads here instead of next to their
  // use after the K loop; it waits for nothing
  asm volatile("" ::: "memory");
  return q;
}

__device__ __forceinline__ f32x4 turbo_values(const TurboArgs& a, f32x4 acc, int item, int mr,
                                              int r0, const __half* a_l, int li, int kb,
                                              const TurboPre* pre = nullptr) {
  const int r = r0 + li, row = min(r, a.N - 1), w = turbo_w(a, item);
  const float nr = pre ? pre->nr : a.norms[(int64_t)w * a.n_es + row];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] *= nr;
  if (a.sv) {
    // A = a (token rows), B = SV rows: D[token 4kb + i][row li], acc's layout
    const __half* svr = a.sv + (int64_t)w * a.sv_es + (int64_t)row * a.rank;
    const __half* ar = a_l + min(li, mr - 1) * a.apad;
    for (int s0 = 0; s0 < a.rpad; s0 += 32) {
      const int j = s0 + 8 * kb;
      const f16x8 av = *(const f16x8*)(ar + j);
      f16x8 bv = {};
      if (pre && s0 < 32 * kTurboPreBlocks) {
#pragma unroll
        for (int b = 0; b < kTurboPreBlocks; ++b)
          if (s0 == 32 * b) bv = pre->sv[b];
      } else {
        bv = j < a.rank ? *(const f16x8*)(svr + j) : f16x8{};
      }
      acc = mfma_16x16x32(av, bv, acc);
    }
  }
  const float bb = pre ? pre->bb
                       : (a.bias ? __half2float(a.bias[(int64_t)w * a.bias_es + row]) : 0.f);
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] += bb;
  return acc;
}

// Writes one 16-row tile: y = fp16(norm * acc + a SV^T + bias), or with gate
// the SwiGLU of the gate's stored value and it.
__device__ __forceinline__ void turbo_epilogue(const TurboArgs& a, f32x4 acc, int item, int m0,
                                               int mr, int r0, const __half* a_l, int li,
                                               int kb, const TurboPre* pre = nullptr) {
  const f32x4 v = turbo_values(a, acc, item, mr, r0, a_l, li, kb, pre);
  const int r = r0 + li;
  if (r < a.N) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * kb + i;
      if (m < mr) {
        const int64_t o = (int64_t)item * a.y_es + (int64_t)(m0 + m) * a.N + r;
        a.y[o] = a.gate ? swiglu_fp16(__half2float(a.gate[o]), v[i]) : __float2half(v[i]);
      }
    }
  }
}

// The pair form's tile: y = fp16(fp16(silu(fp16(gate values))) * fp16(up
// values)) -- the bits of the gate launch's store followed by the up
// launch's SwiGLU store.
__device__ __forceinline__ void turbo_pair_epilogue(const TurboArgs& g, const TurboArgs& u,
                                                    f32x4 accg, f32x4 accu, int item, int m0,
                                                    int mr, int r0, const __half* a_lg,
                                                    const __half* a_lu, int li, int kb,
                                                    const TurboPre* preg, const TurboPre* preu) {
  const f32x4 vg = turbo_values(g, accg, item, mr, r0, a_lg, li, kb, preg);
  const f32x4 vu = turbo_values(u, accu, item, mr, r0, a_lu, li, kb, preu);
  const int r = r0 + li;
  if (r < u.N) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 4 * kb + i;
      if (m < mr) u.y[(int64_t)item * u.y_es + (int64_t)(m0 + m) * u.N + r] = swiglu_fp16(vg[i], vu[i]);
    }
  }
}

// Stages the block's token rows of x_rot for 256-code steps [sb, se) (permuted
// into the decode order; zero past K) and, when there is a low-rank term, its
// low-rank factor a.  The caller's barrier makes both visible.
__device__ __forceinline__ void turbo_stage(const TurboArgs& a, const __half* X, int item, int m0,
                                            int mr, int sb, int se, __half* xs, __half* a_l,
                                            bool with_a, int tid) {
  if (with_a && a.sv && a.parts) {  // (M = 1 items) a from the partials, in slice order
    const int64_t blk = min(max(a.xclus ? (int64_t)a.xclus[turbo_w(a, item)] : (int64_t)item,
                                (int64_t)0), (int64_t)a.pB - 1);
    const int t = a.xclus ? item / a.x_div : 0;
    const float* pp = a.parts + ((blk * a.pP) * a.pM + t) * a.rpad;
    for (int j = tid; j < a.rpad; j += 256)
      a_l[j] = j < a.rank ? __float2half(sum_strided(pp + j, (int64_t)a.pM * a.rpad, a.pP))
                          : __float2half(0.f);
  } else if (with_a && a.sv) {
    for (int idx = tid; idx < mr * a.rpad; idx += 256) {
      const int m = idx / a.rpad, j = idx - m * a.rpad;
      a_l[m * a.apad + j] = j < a.rank ? a.xu[turbo_arow(a, item) * a.xu_es +
                                              (int64_t)(m0 + m) * a.rank + j]
                                       : __float2half(0.f);
    }
  }
  const int nblk = (se - sb) * 16;  // 16-code blocks
  for (int idx = tid; idx < mr * nblk; idx += 256) {
    const int m = idx / nblk, blk = idx - m * nblk;
    const int k = sb * 256 + blk * 16;
    f16x8 o0 = f16x8{}, o1 = f16x8{};
    if (k < a.K) {
      const f16x8 v0 = *(const f16x8*)(X + (int64_t)m * a.K + k);
      const f16x8 v1 = *(const f16x8*)(X + (int64_t)m * a.K + k + 8);
      o0 = __builtin_shufflevector(v0, v1, 0, 4, 1, 5, 2, 6, 3, 7);
      o1 = __builtin_shufflevector(v0, v1, 8, 12, 9, 13, 10, 14, 11, 15);
    }
    f16x8* dst = (f16x8*)(xs + m * a.xstride + blk * 16);
    dst[0] = o0;
    dst[1] = o1;
  }
}

// Codes of one 256-code step of a row (lane kb: words 4kb..4kb+3) against the
// staged x at step offset xk: 4 words, 16 MFMAs into acc.
__device__ __forceinline__ void turbo_step(const u32x4& w, const __half* xk, const TurboLut& H,
                                           const TurboLut& L, f32x4& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x8 s0h, s1h, s0l, s1l;
    turbo_decode(w[i], H, L, s0h, s1h, s0l, s1l);
    const f16x8 x0 = *(const f16x8*)(xk + 16 * i);
    const f16x8 x1 = *(const f16x8*)(xk + 16 * i + 8);
    acc = mfma_16x16x32(x0, s0h, acc);
    acc = mfma_16x16x32(x1, s1h, acc);
    acc = mfma_16x16x32(x0, s0l, acc);
    acc = mfma_16x16x32(x1, s1l, acc);
  }
}

// turbo_stream_kernel: the streaming form for problems with many tiles and the
// whole K of the block's tokens in LDS.  A workgroup covers one (item, token
// block); its waves walk tiles gw, gw + 4R, ... (R workgroups per block) over
// the full K, keeping PF steps of codes in flight across tile boundaries
// (the slot of step s refills with step s + PF of the tile, or with step s of
// the wave's next tile), and write each tile as soon as its sum is complete.
template <int PF>
__global__ __launch_bounds__(256) void turbo_stream_kernel(TurboArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __half* a_l = (__half*)smem;        // [16][apad] low-rank factor a
  __half* xs = a_l + 16 * a.apad;     // [mr][xstride], the whole K
  const int per_item = a.rwgs * a.twgs;
  const int item = blockIdx.x / per_item;
  const int rem = blockIdx.x - item * per_item;
  const int tb = rem / a.rwgs, wl = rem - tb * a.rwgs;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), li = lane & 15, kb = lane >> 4;
  const int m0 = 16 * tb, mr = min(16, a.M - m0);
  const __half* X = a.x + turbo_xrow(a, item) * a.x_es + (int64_t)m0 * a.K;
  const uint32_t* C = a.codes + (int64_t)turbo_w(a, item) * a.c_es;
  const int T = (a.N + 15) >> 4, stride = 4 * a.rwgs, gw = wl * 4 + wave;
  const int ntw = gw < T ? (T - gw + stride - 1) / stride : 0;  // tiles of this wave
  const int nsteps = (a.K + 255) >> 8, cyc = (nsteps + PF - 1) / PF;
  const int wlast = a.kw - 4;
  const TurboLut H = turbo_lut(a.cent, false), L = turbo_lut(a.cent, true);
  auto load = [&](int t, int s) {  // step s of the wave's t-th tile
    const int row = min(16 * (gw + t * stride) + li, a.N - 1);
    return *(const u32x4*)(C + (int64_t)row * a.kw + min(16 * s + 4 * kb, wlast));
  };
  u32x4 buf[PF];
#pragma unroll
  for (int p = 0; p < PF; ++p) buf[p] = (ntw > 0 && p < nsteps) ? load(0, p) : u32x4{0, 0, 0, 0};
  turbo_stage(a, X, item, m0, mr, 0, nsteps, xs, a_l, true, tid);
  __syncthreads();
  const __half* xr = xs + min(li, mr - 1) * a.xstride + 64 * kb;
  for (int t = 0; t < ntw; ++t) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < cyc; ++c) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int s = c * PF + p;
        const u32x4 w = buf[p];
        const int nt = c + 1 < cyc ? t : t + 1, ns = c + 1 < cyc ? s + PF : p;
        if (nt < ntw && ns < nsteps) buf[p] = load(nt, ns);
        if (s < nsteps) turbo_step(w, xr + s * 256, H, L, acc);
      }
    }
    turbo_epilogue(a, acc, item, m0, mr, 16 * (gw + t * stride), a_l, li, kb);
  }
}

// PAIR: a second matrix u of the same shape (the up projection of a gate/up
// pair, its own codes, norms, codebook, low-rank term and input) is walked
// beside a, each with its own accumulator and the same order of sums as a
// launch of its own, and the tile's store is the SwiGLU of the two
// (turbo_pair_epilogue) -- one launch where gate and up took two.
template <bool PAIR>
__global__ __launch_bounds__(256) void turbo_gemv_kernel(TurboArgs a, TurboArgs u) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NM = PAIR ? 2 : 1;
  float* red = (float*)smem;                       // [NM][4 waves][4][64] partial sums
  __half* a_l = (__half*)(smem + 4096 * NM);       // [16][apad] low-rank factor a (u's after)
  __half* a_lu = a_l + 16 * a.apad;
  __half* xs = a_l + NM * 16 * a.apad;             // [mr][xstride], one K segment (u's after)
  const int per_item = a.rwgs * a.twgs;
  const int item = blockIdx.x / per_item;
  const int rem = blockIdx.x - item * per_item;
  const int tb = rem / a.rwgs, rg = rem - tb * a.rwgs;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), li = lane & 15, kb = lane >> 4;
  const int wpt = a.wpt, tpw = 4 / wpt;            // waves per tile, tiles per workgroup
  const int part = wave % wpt, r0 = (rg * tpw + wave / wpt) * 16;
  const int m0 = 16 * tb, mr = min(16, a.M - m0);  // token rows of this block
  const __half* X = a.x + turbo_xrow(a, item) * a.x_es + (int64_t)m0 * a.K;
  const __half* Xu = PAIR ? u.x + turbo_xrow(u, item) * u.x_es + (int64_t)m0 * u.K : X;
  const bool own_xu = PAIR && Xu != X;  // (uniform) u's input staged apart
  __half* xsu = own_xu ? xs + mr * a.xstride : xs;

  const TurboLut H = turbo_lut(a.cent, false), L = turbo_lut(a.cent, true);
  TurboLut Hu = H, Lu = L;
  if constexpr (PAIR) {
    Hu = turbo_lut(u.cent, false);
    Lu = turbo_lut(u.cent, true);
  }
  const int row = min(r0 + li, a.N - 1);
  const uint32_t* crow =
      a.codes + (int64_t)turbo_w(a, item) * a.c_es + (int64_t)row * a.kw;
  const uint32_t* crowu =
      PAIR ? u.codes + (int64_t)turbo_w(u, item) * u.c_es + (int64_t)row * u.kw : crow;
  const int wlast = a.kw - 4;  // last whole 16-byte piece (kw is a multiple of 4)
  const __half* xr = xs + min(li, mr - 1) * a.xstride;
  const __half* xru = xsu + min(li, mr - 1) * a.xstride;
  // the epilogue's loads (the tile's first wave of each K split writes it)
  const TurboPre pre = turbo_pre(a, item, r0, li, kb);
  TurboPre preu = pre;
  if constexpr (PAIR) preu = turbo_pre(u, item, r0, li, kb);
  const int nsteps = (a.K + 255) >> 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
  constexpr int PF = kTurboPF;  // 256-code steps of codes in flight per wave (per matrix)

  for (int sb = 0; sb < nsteps; sb += a.segsteps) {
    const int se = min(nsteps, sb + a.segsteps);
    const int q = (se - sb + wpt - 1) / wpt;
    const int j0 = sb + part * q;                 // this wave's first step
    const int jn = max(0, min(se, j0 + q) - j0);  // and its step count
    // a step of a row is 16 words; lane kb holds words 4kb..4kb+3 (clamped:
    // words past the row end meet zero x and add nothing)
    u32x4 buf[PF], bufu[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int wo = min(16 * (j0 + p) + 4 * kb, wlast);
      buf[p] = p < jn ? *(const u32x4*)(crow + wo) : u32x4{0, 0, 0, 0};
      if constexpr (PAIR) bufu[p] = p < jn ? *(const u32x4*)(crowu + wo) : u32x4{0, 0, 0, 0};
    }
    if (sb > 0) __syncthreads();  // every wave is done with the previous segment
    turbo_stage(a, X, item, m0, mr, sb, se, xs, a_l, sb == 0, tid);
    if constexpr (PAIR) {
      if (own_xu) turbo_stage(u, Xu, item, m0, mr, sb, se, xsu, a_lu, sb == 0, tid);
      else turbo_stage(u, Xu, item, m0, mr, sb, sb, xsu, a_lu, sb == 0, tid);  // a alone
    }
    __syncthreads();
    auto consume = [&](const u32x4& w, const u32x4& wu, int j) {
      turbo_step(w, xr + (j0 + j - sb) * 256 + 64 * kb, H, L, acc);
      if constexpr (PAIR) turbo_step(wu, xru + (j0 + j - sb) * 256 + 64 * kb, Hu, Lu, accu);
    };
    int jj = 0;
    for (; jj + PF <= jn; jj += PF) {  // whole rounds: refill each slot after use
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const u32x4 w = buf[p], wu = PAIR ? bufu[p] : w;
        if (jj + p + PF < jn) {
          const int wo = min(16 * (j0 + jj + p + PF) + 4 * kb, wlast);
          buf[p] = *(const u32x4*)(crow + wo);
          if constexpr (PAIR) bufu[p] = *(const u32x4*)(crowu + wo);
        }
        consume(w, wu, jj + p);
      }
    }
#pragma unroll
    for (int p = 0; p < PF; ++p)  // the last jn % PF steps
      if (jj + p < jn) consume(buf[p], PAIR ? bufu[p] : buf[p], jj + p);
  }
  // acc[i] of lane (li, kb): token 4kb + i, row li of the tile
  if (wpt > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[(wave * 4 + i) * 64 + lane] = acc[i];
      if constexpr (PAIR) red[1024 + (wave * 4 + i) * 64 + lane] = accu[i];
    }
    __syncthreads();
    if (part != 0) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = red[(wave * 4 + i) * 64 + lane];
      for (int w2 = 1; w2 < wpt; ++w2) v += red[((wave + w2) * 4 + i) * 64 + lane];
      acc[i] = v;
      if constexpr (PAIR) {
        float vu = red[1024 + (wave * 4 + i) * 64 + lane];
        for (int w2 = 1; w2 < wpt; ++w2) vu += red[1024 + ((wave + w2) * 4 + i) * 64 + lane];
        accu[i] = vu;
      }
    }
  }
  if constexpr (PAIR)
    turbo_pair_epilogue(a, u, acc, accu, item, m0, mr, r0, a_l, a_lu, li, kb, &pre, &preu);
  else
    turbo_epilogue(a, acc, item, m0, mr, r0, a_l, li, kb, &pre);
}

// ---------------------------------------------------------------------------
// Randomized Hadamard transform of rows of length d (a power of two):
//   forward: y = (1/sqrt(d)) H diag(signs) x
//   inverse: y = diag(signs) (1/sqrt(d)) H x
// (hadamard_rotation.py:52-67 rht_forward and :70-86 rht_backward; H is the
// Sylvester, natural-order Hadamard matrix that the external
// fast-hadamard-transform package applies).  The hot-path call is
// rht_forward(x.float(), signs).half() (inference/moe_block.py:351,525,649,
// 840): fp16 in, fp32 arithmetic, fp16 out.  One workgroup per row: the row in
// LDS as fp32, log2(d) butterfly passes with a barrier each.
// ---------------------------------------------------------------------------
template <class TI, class TO>
__global__ __launch_bounds__(256) void rht_kernel(const TI* __restrict__ x,
                                                  const float* __restrict__ signs,
                                                  TO* __restrict__ y, int d, int logd,
                                                  float scale, int inverse) {
  extern __shared__ float v[];
  const TI* xr = x + (int64_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) {
    const float xv = (float)xr[i];
    v[i] = inverse ? xv : xv * signs[i];
  }
  __syncthreads();
  for (int s = 0; s < logd; ++s) {
    const int h = 1 << s;
    for (int p = threadIdx.x; p < d / 2; p += 256) {
      const int i = ((p >> s) << (s + 1)) | (p & (h - 1)), j = i + h;
      const float u = v[i], w = v[j];
      v[i] = u + w;
      v[j] = u - w;
    }
    __syncthreads();
  }
  TO* yr = y + (int64_t)blockIdx.x * d;
  for (int i = threadIdx.x; i < d; i += 256) {
    const float o = v[i] * scale;
    yr[i] = (TO)(inverse ? o * signs[i] : o);
  }
}

}  // namespace glq

namespace glq {
namespace {
// Picks the form and launches; a holds every pointer, size and item field.
// With u (the pair form: a second matrix of the same shape, same items) the
// one-shot kernel runs both, with the plan a launch of a alone would take.
int turbo_run(TurboArgs& a, int64_t items, int64_t M, int64_t K, int64_t N, hipStream_t s,
              TurboArgs* u = nullptr) {
  const int mr = (int)std::min<int64_t>(16, M);
  const int nsteps = (int)((K + 255) / 256);
  const int fit = (kTurboXBudget / (2 * mr) - 8) / 256;  // steps of a segment that fit
  a.segsteps = std::max(1, std::min(nsteps, fit));
  a.xstride = a.segsteps * 256 + 8;
  a.twgs = (int)((M + 15) / 16);
  const int64_t T = (N + 15) / 16, tiles = items * a.twgs * T;
  const int64_t kpad = (int64_t)nsteps * 256;
  const size_t stream_lds = (size_t)16 * a.apad * 2 + (size_t)mr * (kpad + 8) * 2;
  if (!u && tiles >= kTurboStreamTiles && stream_lds <= (size_t)kTurboStreamLds) {
    // streaming form: the whole K staged once per workgroup, waves walk tiles
    a.segsteps = nsteps;
    a.xstride = (int)kpad + 8;
    a.wpt = 1;
    const int64_t blocks = items * a.twgs;
    a.rwgs = (int)std::max<int64_t>(1, std::min<int64_t>((kTurboStreamWgs + blocks - 1) / blocks,
                                                         (T + 3) / 4));
    static size_t attr = 64 * 1024;
    int rc = set_lds_limit(turbo_stream_kernel<kTurboPF>, stream_lds, attr);
    if (rc) return rc;
    const int64_t grid = blocks * a.rwgs;
    GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
    turbo_stream_kernel<kTurboPF><<<dim3((unsigned)grid), dim3(256), stream_lds, s>>>(a);
    GLQ_LAUNCH_CHECK("turbo_stream_kernel");
    return GLQ_OK;
  }
  // one-shot form: one wave per tile when there are enough tiles to fill the
  // chip; else the K dimension of a tile is split among 2 or 4 waves
  a.wpt = tiles >= 2048 ? 1 : tiles >= 1024 ? 2 : 4;
  const int tpw = 4 / a.wpt;
  a.rwgs = (int)((T + tpw - 1) / tpw);
  const int64_t grid = items * a.rwgs * a.twgs;
  GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
  if (u) {
    // the same plan for u (its staging and order of sums are a's)
    u->segsteps = a.segsteps;
    u->xstride = a.xstride;
    u->twgs = a.twgs;
    u->wpt = a.wpt;
    u->rwgs = a.rwgs;
    GLQ_CHECK(u->apad == a.apad && u->K == a.K && u->N == a.N && u->M == a.M &&
                  u->kw == a.kw && a.segsteps * 256 >= a.K,
              "the pair's matrices must share their shape, rank and one K segment");
    const size_t lds = 2 * 4096 + (size_t)2 * 16 * a.apad * 2 + (size_t)2 * mr * a.xstride * 2;
    static size_t attr = 64 * 1024;
    int rc = set_lds_limit(turbo_gemv_kernel<true>, lds, attr);
    if (rc) return rc;
    turbo_gemv_kernel<true><<<dim3((unsigned)grid), dim3(256), lds, s>>>(a, *u);
    GLQ_LAUNCH_CHECK("turbo_gemv_kernel");
    return GLQ_OK;
  }
  const size_t lds = 4096 + (size_t)16 * a.apad * 2 + (size_t)mr * a.xstride * 2;
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(turbo_gemv_kernel<false>, lds, attr);
  if (rc) return rc;
  turbo_gemv_kernel<false><<<dim3((unsigned)grid), dim3(256), lds, s>>>(a, a);
  GLQ_LAUNCH_CHECK("turbo_gemv_kernel");
  return GLQ_OK;
}
}  // namespace
}  // namespace glq

extern "C" int glq_turbo_gemv_batched(int64_t items, const void* x_rot, int64_t x_stride,
                                      int64_t M, int64_t K, int64_t N, const int32_t* codes,
                                      int64_t codes_stride, const float* norms,
                                      int64_t norms_stride, const float* centroids,
                                      const void* xU, int64_t xu_stride, const void* SV,
                                      int64_t sv_stride, int64_t rank, const void* bias,
                                      int64_t bias_stride, void* y, int64_t y_stride,
                                      void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(items >= 0 && M >= 0 && K >= 0 && N >= 0, "negative size");
  if (items == 0 || M == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(K > 0 && K % 64 == 0 && K < (1 << 24),
            "K=%lld must be a positive multiple of 64 (whole 16-byte code pieces per row)",
            (long long)K);
  GLQ_CHECK(M < (1ll << 24) && N < (1ll << 26), "M or N too large");
  GLQ_CHECK(x_rot && codes && norms && centroids && y, "null data pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x_rot) && al16(codes), "x_rot and codes must be 16-byte aligned");
  GLQ_CHECK(items == 1 || (x_stride % 8 == 0 && codes_stride % 4 == 0),
            "item strides must keep 16-byte alignment");
  TurboArgs a;
  a.x = (const __half*)x_rot;
  a.x_es = x_stride;
  a.codes = (const uint32_t*)codes;
  a.c_es = codes_stride;
  a.norms = norms;
  a.n_es = norms_stride;
  a.cent = centroids;
  const bool lora = SV != nullptr && rank > 0;
  GLQ_CHECK(!lora || (rank % 8 == 0 && rank <= 256),
            "rank=%lld must be a multiple of 8 up to 256", (long long)rank);
  GLQ_CHECK(!lora || xU, "SV given without the low-rank factor xU = x U");
  GLQ_CHECK(!lora || (al16(SV) && (items == 1 || sv_stride % 8 == 0)),
            "SV must be 16-byte aligned");
  a.xu = lora ? (const __half*)xU : nullptr;
  a.xu_es = xu_stride;
  a.sv = lora ? (const __half*)SV : nullptr;
  a.sv_es = sv_stride;
  a.bias = (const __half*)bias;
  a.bias_es = bias_stride;
  a.rank = lora ? (int)rank : 0;
  a.rpad = (int)align_up(a.rank, 32);
  a.apad = a.rpad + 8;
  a.y = (__half*)y;
  a.y_es = y_stride;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.kw = (int)(K / 16);
  a.wsel = nullptr;
  a.nw = (int)std::min<int64_t>(items, 1 << 30);
  a.x_div = 1;
  a.xclus = nullptr;
  a.xu_tok = a.xu_rows = 0;
  a.gate = nullptr;
  return turbo_run(a, items, M, K, N, (hipStream_t)stream);
}

extern "C" int glq_turbo_moe_gemv(int64_t picks, int64_t x_div, const void* x_rot, int64_t K,
                                  int64_t N, int64_t experts, const int32_t* sel,
                                  const int32_t* codes, const float* norms,
                                  const float* centroids, const void* xU,
                                  const int32_t* xu_cluster, int64_t xu_tokens,
                                  int64_t xu_rows, const void* SV, int64_t rank,
                                  const void* bias, const void* gate, void* y, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(picks >= 0 && K >= 0 && N >= 0 && experts >= 1 && x_div >= 1, "bad size");
  if (picks == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(K > 0 && K % 64 == 0 && K < (1 << 24),
            "K=%lld must be a positive multiple of 64 (whole 16-byte code pieces per row)",
            (long long)K);
  GLQ_CHECK(picks < (1 << 20) && N < (1ll << 26) && experts < (1 << 20), "sizes too large");
  GLQ_CHECK(x_rot && sel && codes && norms && centroids && y, "null data pointer");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x_rot) && al16(codes), "x_rot and codes must be 16-byte aligned");
  const bool lora = SV != nullptr && rank > 0;
  GLQ_CHECK(!lora || (rank % 8 == 0 && rank <= 256),
            "rank=%lld must be a multiple of 8 up to 256", (long long)rank);
  GLQ_CHECK(!lora || (xU && al16(SV)), "SV needs xU, and 16-byte alignment");
  GLQ_CHECK(!lora || !xu_cluster || (xu_tokens >= 1 && xu_rows >= 1),
            "xu_cluster needs xu_tokens and xu_rows");
  TurboArgs a;
  a.x = (const __half*)x_rot;
  a.x_es = K;
  a.codes = (const uint32_t*)codes;
  a.c_es = N * (K / 16);
  a.norms = norms;
  a.n_es = N;
  a.cent = centroids;
  a.xu = lora ? (const __half*)xU : nullptr;
  a.xu_es = lora ? rank : 0;
  a.sv = lora ? (const __half*)SV : nullptr;
  a.sv_es = N * rank;
  a.bias = (const __half*)bias;
  a.bias_es = N;
  a.rank = lora ? (int)rank : 0;
  a.rpad = (int)align_up(a.rank, 32);
  a.apad = a.rpad + 8;
  a.y = (__half*)y;
  a.y_es = N;
  a.M = 1;
  a.K = (int)K;
  a.N = (int)N;
  a.kw = (int)(K / 16);
  a.wsel = sel;
  a.nw = (int)experts;
  a.x_div = (int)x_div;
  a.xclus = lora ? xu_cluster : nullptr;
  a.xu_tok = (int)xu_tokens;
  a.xu_rows = (int)std::min<int64_t>(xu_rows, 1 << 30);
  a.gate = (const __half*)gate;
  return turbo_run(a, picks, 1, K, N, (hipStream_t)stream);
}

namespace glq {
namespace {
// TurboArgs of one projection of glq_turbo_moe_gemv2.
int turbo_mat_args(const glq_turbo_mat& m, int64_t picks, int64_t x_div, int64_t K, int64_t N,
                   int64_t experts, const int32_t* sel, int64_t rank, int64_t P, void* y,
                   TurboArgs& a) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(m.x_rot && m.codes && m.norms && m.centroids, "null projection pointer");
  GLQ_CHECK(al16(m.x_rot) && al16(m.codes), "x_rot and codes must be 16-byte aligned");
  const bool lora = m.SV != nullptr && rank > 0;
  GLQ_CHECK(!lora || (m.parts && P >= 1 && m.blocks >= 1 && al16(m.SV) &&
                      ((uintptr_t)m.parts & 3) == 0),
            "SV needs parts, P >= 1, blocks >= 1 and 16-byte alignment");
  a.x = (const __half*)m.x_rot;
  a.x_es = K;
  a.codes = (const uint32_t*)m.codes;
  a.c_es = N * (K / 16);
  a.norms = m.norms;
  a.n_es = N;
  a.cent = m.centroids;
  a.xu = nullptr;
  a.xu_es = 0;
  a.sv = lora ? (const __half*)m.SV : nullptr;
  a.sv_es = N * rank;
  a.bias = nullptr;
  a.bias_es = 0;
  a.rank = lora ? (int)rank : 0;
  a.rpad = (int)align_up(a.rank, 32);
  a.apad = a.rpad + 8;
  a.y = (__half*)y;
  a.y_es = N;
  a.M = 1;
  a.K = (int)K;
  a.N = (int)N;
  a.kw = (int)(K / 16);
  a.wsel = sel;
  a.nw = (int)experts;
  a.x_div = (int)x_div;
  a.xclus = lora ? m.cluster : nullptr;
  a.xu_tok = 0;
  a.xu_rows = 0;
  a.gate = nullptr;
  a.parts = lora ? m.parts : nullptr;
  a.pP = (int)P;
  a.pM = m.cluster ? (int)((picks + x_div - 1) / x_div) : 1;
  a.pB = (int)std::min<int64_t>(m.blocks, 1 << 30);
  return GLQ_OK;
}
}  // namespace
}  // namespace glq

extern "C" int glq_turbo_moe_gemv2(int64_t picks, int64_t x_div, int64_t K, int64_t N,
                                   int64_t experts, const int32_t* sel, const glq_turbo_mat* m,
                                   const glq_turbo_mat* up, int64_t rank, int64_t P, void* y,
                                   void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(picks >= 0 && K >= 0 && N >= 0 && experts >= 1 && x_div >= 1, "bad size");
  if (picks == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(K > 0 && K % 64 == 0 && K < (1 << 24),
            "K=%lld must be a positive multiple of 64 (whole 16-byte code pieces per row)",
            (long long)K);
  GLQ_CHECK(picks < (1 << 20) && N < (1ll << 26) && experts < (1 << 20), "sizes too large");
  GLQ_CHECK(m && sel && y, "null m, sel or y");
  GLQ_CHECK(rank >= 0 && rank <= 256 && rank % 8 == 0, "rank=%lld must be a multiple of 8 up to 256",
            (long long)rank);
  TurboArgs a, u;
  if (int rc = turbo_mat_args(*m, picks, x_div, K, N, experts, sel, rank, P, y, a)) return rc;
  if (!up) return turbo_run(a, picks, 1, K, N, (hipStream_t)stream);
  if (int rc = turbo_mat_args(*up, picks, x_div, K, N, experts, sel, rank, P, y, u)) return rc;
  GLQ_CHECK((a.sv == nullptr) == (u.sv == nullptr), "gate and up must both have SV or neither");
  return turbo_run(a, picks, 1, K, N, (hipStream_t)stream, &u);
}

extern "C" int glq_rht(const void* x, int x_fp32, int64_t rows, int64_t d, const float* signs,
                       int inverse, void* y, int y_fp32, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(rows >= 0 && d >= 0, "negative size");
  if (rows == 0) return GLQ_OK;
  GLQ_CHECK(d >= 2 && d <= 32768 && (d & (d - 1)) == 0,
            "d=%lld must be a power of two in [2, 32768]", (long long)d);
  GLQ_CHECK(rows < (1ll << 31), "too many rows");
  GLQ_CHECK(x && signs && y, "null data pointer");
  GLQ_CHECK(x != y, "y may not alias x");
  const size_t lds = (size_t)d * 4;
  int logd = 0;
  while ((1ll << logd) < d) ++logd;
  const float scale = 1.0f / sqrtf((float)d);
  const dim3 grid((unsigned)rows), block(256);
  hipStream_t s = (hipStream_t)stream;
  int rc;
#define GLQ_RHT_LAUNCH(TI, TO)                                                        \
  do {                                                                                \
    static size_t attr = 64 * 1024;                                                   \
    rc = set_lds_limit(rht_kernel<TI, TO>, lds, attr);                                \
    if (rc) return rc;                                                                \
    rht_kernel<TI, TO><<<grid, block, lds, s>>>((const TI*)x, signs, (TO*)y, (int)d, logd, \
                                               scale, inverse ? 1 : 0);               \
  } while (0)
  if (!x_fp32 && !y_fp32) GLQ_RHT_LAUNCH(__half, __half);
  else if (!x_fp32 && y_fp32) GLQ_RHT_LAUNCH(__half, float);
  else if (x_fp32 && !y_fp32) GLQ_RHT_LAUNCH(float, __half);
  else GLQ_RHT_LAUNCH(float, float);
#undef GLQ_RHT_LAUNCH
  GLQ_LAUNCH_CHECK("rht_kernel");
  return GLQ_OK;
}
