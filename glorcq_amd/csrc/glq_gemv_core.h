// Device core of the fused dequant-GEMV + low-rank correction (gfx950).
//
// One workgroup (256 threads = 4 wave64s) computes a tile of 16*T output rows
// of one "item" (an independent problem: a plain linear layer, one layer of a
// batch, or one expert of a MoE step) for up to 16 token rows:
//
//   y[m,n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) x[m,k]
//          + sum_j a[m,j] SV[n,j] + bias[n],          a = fp16(x U)
//
// Reference semantics: GLoRCQLinear.forward (inference/quantized_linear.py:
// 286-355) = GPTQ dequant-matmul (inference/kernels/__init__.py:284-346,
// kernels/gptq_matmul.cu:42-98) + LoRA `y + (x @ U) @ SV.T`.
//
// Where the item's inputs come from and where its outputs go is a policy type
// (`Src`), so the dense and the grouped (MoE) kernels share this code:
//   int  m_rows(item)                 token rows of the item (<= 16)
//   const __half* xrow(item, m)       K fp16 values of token row m
//   const uint32_t* codes(item)       packed codes, N rows of kw words
//   const __half* scales(item), zeros(item), sv(item), bias(item)
//   void load_a(item, m, j) -> __half the low-rank factor a[m][j]
//   void store(item, m, n, float)     epilogue write of y[m][n]
//
// Design (MI355X-first, not a translation of the CUDA kernel):
//  * Codes are decoded in registers straight into fp16 MFMA operands with one
//    v_and_or per two codes: code bits land in the fp16 mantissa under an
//    exponent chosen per bit position, so each operand is exactly (2^e + q).
//    The 2^e bias is removed once per 128-code chunk with a precomputed
//    sum_k 2^e(k) x[m,k]; zero-points likewise with sum_k x[m,k]; the group
//    scale multiplies the chunk's fp32 MFMA result.  No per-weight dequant.
//  * v_mfma_f32_16x16x32_f16: A = 16 weight rows x 32 codes, B = 32 codes x
//    16 token columns, fp32 accumulate.  A "step" is 16 int32 words (64 B) of
//    every row of a 16-row tile; lane group kb = lane/16 loads words 4kb..4kb+3
//    with ONE 16-byte load, so each wave load instruction covers 16 rows x
//    64 contiguous bytes (measured on MI355X: ~6.3 TB/s for this pattern vs
//    ~3.7 TB/s for 8-byte loads).  4-bit: a step is 128 codes = one group.
//    2-bit: a step is 256 codes = two 128-code halves, kb 0-1 holding the
//    first and kb 2-3 the second; the two halves (possibly two quantization
//    groups) are kept apart INSIDE one MFMA by giving the first half's x to B
//    columns 0-7 and the second half's to columns 8-15 (zeros elsewhere), so
//    D[:, m] and D[:, 8+m] are the two half sums of token m.  Tokens 8-15 take
//    a second MFMA pass.  One cross-lane add after the K loop merges halves.
//    x is staged once per workgroup in LDS in the matching permuted order.
//  * The 4 waves split K; each wave issues the loads of a batch of steps
//    (32 words per lane) before it consumes the first, and the first batch
//    is in flight while x and the scales are staged.  Partial tiles are
//    summed in LDS; the correction a SV^T is more MFMAs per tile on the same
//    accumulator.  No atomics and no cross-workgroup waits: a = x U comes
//    from an earlier launch (lowrank_partial_kernel) or from the caller.
#pragma once

#include <hip/hip_fp16.h>

#include "glq_handoff.h"
#include "glq_internal.h"

namespace glq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Problem shape shared by every item of one launch.
struct TileShape {
  int K, N, G, group, rank, sym;
  float zoff;   // added to every zero-point (signed codes stored offset by 2^(b-1))
  int kw;       // int32 words per weight row
  int rpad;     // rank rounded up to 32
  int kp;       // codes per K-phase staged in LDS (multiple of group)
  int xstride;  // halves per token row of staged x in LDS (kp + 8)
  int apad;     // halves per token row of staged a in LDS
  int mmax;     // largest token-row count of any item (<= 16)
};

// Dynamic LDS layout of a consumer workgroup (byte offsets, 16-byte aligned).
struct LdsLayout {
  int xs, xsum, xbias, s, z, red, a, total;
};

__host__ __device__ inline int al16(int v) { return (v + 15) & ~15; }

__host__ __device__ inline LdsLayout lds_layout(int M, int KP, int GP, int T, int xstride,
                                                int apad) {
  const int nch = KP >> 7;
  LdsLayout L;
  int o = 0;
  L.xs = o;    o += al16(M * xstride * 2);
  L.xsum = o;  o += al16(M * nch * 4);
  L.xbias = o; o += al16(M * nch * 4);
  L.s = o;     o += al16(GP * 16 * T * 4);
  L.z = o;     o += al16(GP * 16 * T * 4);
  L.red = o;   o += 4 * T * 64 * 16;
  L.a = o;     o += al16(M * apad * 2);
  L.total = o;
  return L;
}

// p[0] + p[stride] + ... + p[(n-1) stride] in that order, with the loads
// issued in batches of 8 so that a batch costs one memory round trip (a plain
// loop waits for each load before the next add).
__device__ __forceinline__ float sum_strided(const float* __restrict__ p, int64_t stride, int n) {
  float s = 0.f;
  for (int q0 = 0; q0 < n; q0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = q0 + u < n ? p[(int64_t)(q0 + u) * stride] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  return s;
}

__device__ __forceinline__ f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 2-bit word -> two MFMA operand slices.  Half i of the result pair p_c holds
// code c (low half) and code c+8 (high half) as 2^e + q.
//   slice0 = codes {0,8,1,9,2,10,3,11}, slice1 = {4,12,5,13,6,14,7,15}
//   biases  {1024,256,64,16} and {4,1024,256,64} per code pair.
__device__ __forceinline__ void decode2(uint32_t w, f16x8& s0, f16x8& s1) {
  const uint32_t v = w >> 10;
  u32x4 a, b;
  a.x = (w & 0x00030003u) | 0x64006400u;  // exp 25: 1024 + q
  a.y = (w & 0x000C000Cu) | 0x5C005C00u;  // exp 23:  256 + q
  a.z = (w & 0x00300030u) | 0x54005400u;  // exp 21:   64 + q
  a.w = (w & 0x00C000C0u) | 0x4C004C00u;  // exp 19:   16 + q
  b.x = (w & 0x03000300u) | 0x44004400u;  // exp 17:    4 + q
  b.y = (v & 0x00030003u) | 0x64006400u;
  b.z = (v & 0x000C000Cu) | 0x5C005C00u;
  b.w = (v & 0x00300030u) | 0x54005400u;
  s0 = __builtin_bit_cast(f16x8, a);
  s1 = __builtin_bit_cast(f16x8, b);
}

// The exponent patterns of decode2/decode4 held in VGPRs.  gfx9 VALU ops
// take at most one scalar operand and no 32-bit literal in the 3-operand
// form, so with the masks in SGPRs and these in VGPRs each code pair decodes
// in one v_and_or / v_bitop3.  The asm makes them opaque to constant folding.
struct DecodeConsts {
  uint32_t e25, e23, e21, e19, e17;
  __device__ __forceinline__ static DecodeConsts make() {
    DecodeConsts c;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(c.e25));
    asm volatile("v_mov_b32 %0, 0x5c005c00" : "=v"(c.e23));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(c.e21));
    asm volatile("v_mov_b32 %0, 0x4c004c00" : "=v"(c.e19));
    asm volatile("v_mov_b32 %0, 0x44004400" : "=v"(c.e17));
    return c;
  }
};

__device__ __forceinline__ void decode2(uint32_t w, f16x8& s0, f16x8& s1, const DecodeConsts& k) {
  const uint32_t v = w >> 10;
  u32x4 a, b;
  a.x = (w & 0x00030003u) | k.e25;
  a.y = (w & 0x000C000Cu) | k.e23;
  a.z = (w & 0x00300030u) | k.e21;
  a.w = (w & 0x00C000C0u) | k.e19;
  b.x = (w & 0x03000300u) | k.e17;
  b.y = (v & 0x00030003u) | k.e25;
  b.z = (v & 0x000C000Cu) | k.e23;
  b.w = (v & 0x00300030u) | k.e21;
  s0 = __builtin_bit_cast(f16x8, a);
  s1 = __builtin_bit_cast(f16x8, b);
}

__device__ __forceinline__ f16x8 decode4(uint32_t w, const DecodeConsts& k) {
  const uint32_t v = w >> 8;
  u32x4 a;
  a.x = (w & 0x000F000Fu) | k.e25;
  a.y = (w & 0x00F000F0u) | k.e21;
  a.z = (v & 0x000F000Fu) | k.e25;
  a.w = (v & 0x00F000F0u) | k.e21;
  return __builtin_bit_cast(f16x8, a);
}

// 4-bit word -> one slice: codes {0,4,1,5,2,6,3,7}, biases {1024,64,1024,64}.
__device__ __forceinline__ f16x8 decode4(uint32_t w) {
  const uint32_t v = w >> 8;
  u32x4 a;
  a.x = (w & 0x000F000Fu) | 0x64006400u;  // 1024 + q
  a.y = (w & 0x00F000F0u) | 0x54005400u;  //   64 + q
  a.z = (v & 0x000F000Fu) | 0x64006400u;
  a.w = (v & 0x00F000F0u) | 0x54005400u;
  return __builtin_bit_cast(f16x8, a);
}

// Operand bias of permuted position pos (0..15 within a 16-code block).
template <int BITS>
__device__ __forceinline__ float code_bias(int pos) {
  if constexpr (BITS == 2) {
    constexpr float b2[8] = {1024.f, 256.f, 64.f, 16.f, 4.f, 1024.f, 256.f, 64.f};
    return b2[pos >> 1];
  } else {
    constexpr float b4[4] = {1024.f, 64.f, 1024.f, 64.f};
    return b4[(pos & 7) >> 1];
  }
}

// Source index within a 16-code block for permuted position pos.
template <int BITS>
__device__ __forceinline__ int perm_src(int pos) {
  if constexpr (BITS == 2) return (pos >> 1) + ((pos & 1) << 3);  // 0,8,1,9,..
  else return (pos & 8) + ((pos & 7) >> 1) + ((pos & 1) << 2);     // 0,4,1,5,.. per 8
}

// Codes per step (16 words of a row): 256 for 2-bit, 128 for 4-bit.
template <int BITS>
constexpr int step_codes() { return 16 * (32 / BITS); }

// Steps per load batch: 32 words per lane in flight.
template <int T>
constexpr int batch_steps() { return T >= 8 ? 1 : 8 / T; }

// Loads steps [s, s + NB) of this lane's rows (16 B per row per step; steps
// past `se` re-read step se - 1, a valid address, and are never consumed).
// `wmax` clamps the word offset so the 2-bit tail half-step stays in bounds.
template <int T, int NB>
__device__ __forceinline__ void load_batch(u32x4 (&wv)[NB][T], const uint32_t* C,
                                           const int64_t (&roff)[T], int w0, int s, int se,
                                           int kb, int wmax) {
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int st = min(s + b, se - 1);
    const int wo = min(w0 + 16 * st + 4 * kb, wmax);
#pragma unroll
    for (int t = 0; t < T; ++t)
      wv[b][t] = __builtin_nontemporal_load((const u32x4*)(C + roff[t] + wo));
  }
}

// ---------------------------------------------------------------------------
// Low-rank partials: apart[p][m][j] = sum_{k in slice p} x[m,k] U[k,j] for
// one item and one K-slice of `ks` rows (fp32).  256 threads; thread tid owns
// columns 8*(tid&7) .. +8 of each 64-column block and rows k0 + (tid>>3) + 32i.
// ---------------------------------------------------------------------------
constexpr int kLowrankRows = 256;  // U rows per partial (K-slice)
constexpr int kLowrankUtStride = kLowrankRows + 8;  // halves per staged U column (MC == 4)

// `tid` is the thread's index in its group of 256 (a workgroup may run several
// groups side by side, each with its own LDS; every group must make the same
// calls, since the barriers are workgroup-wide).  out == nullptr: compute, but
// write nothing (a group without a job of its own).
// COH: the partials are read inside the same launch (agent-scope stores).
template <int MC, class XRow, bool COH = false>
__device__ void lowrank_partial(const XRow& xrow, int M, int K, int rank, int rpad,
                                const __half* __restrict__ U, int p,
                                float* __restrict__ out /* M x rpad */,
                                float* red /* LDS, 4*4*64 floats */,
                                __half* xl /* LDS, 16 x kLowrankRows halves */,
                                int tid, __half* ut = nullptr /* LDS, MC == 4: 64 x
                                                                  kLowrankUtStride halves */) {
  const int lane = tid & 63, wave = tid >> 6;
  const int j8 = tid & 7, kr = tid >> 3;  // kr in 0..31
  const int k0 = p * kLowrankRows;
  const int kl = min(kLowrankRows, K - k0);
  if constexpr (MC == 4) {
    // 3..16 token rows: one v_mfma_f32_16x16x32_f16 tile per 16 rank columns
    // (A = the x slice, 16 rows staged in LDS with zeros past M; B = a U
    // column, from U's 64-column block staged transposed in LDS by 16-byte
    // row loads), a wave per column tile.
    for (int idx = tid; idx < 16 * (kLowrankRows / 8); idx += 256) {
      const int m = idx / (kLowrankRows / 8), k = 8 * (idx - m * (kLowrankRows / 8));
      const __half* xs = xrow(m) + k0 + k;
      f16x8 v = {};
      if (m < M && k + 8 <= kl && ((uintptr_t)xs & 15) == 0) {
        v = *(const f16x8*)xs;
      } else {  // a row end inside the chunk, or x not 16-byte aligned
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (m < M && k + e < kl) v[e] = (_Float16)__half2float(xs[e]);
      }
      *(f16x8*)(xl + m * kLowrankRows + k) = v;
    }
    const int li = lane & 15, kb = lane >> 4;
    for (int jb = 0; jb < rpad; jb += 64) {
      for (int idx = tid; idx < kLowrankRows * 8; idx += 256) {
        const int k = idx >> 3, c = 8 * (idx & 7);
        f16x8 v = {};
        if (k < kl && jb + c < rank) v = *(const f16x8*)(U + (int64_t)(k0 + k) * rank + jb + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) ut[(c + e) * kLowrankUtStride + k] = v[e];
      }
      __syncthreads();
      const int cl = wave * 16 + li, col = jb + cl;  // 4 waves x 16 columns
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kLowrankRows / 32; ++ks) {
        const int kk = 32 * ks + 8 * kb;
        acc = mfma_16x16x32(*(const f16x8*)(xl + li * kLowrankRows + kk),
                            *(const f16x8*)(ut + cl * kLowrankUtStride + kk), acc);
      }
      // acc[i] = sum over the slice for token 4 kb + i, column col
      if (out && col < rpad) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * kb + i;
          if (m < M) {
            const float v = col < rank ? acc[i] : 0.f;
            if constexpr (COH) handoff_put(out + m * rpad + col, v);
            else out[m * rpad + col] = v;
          }
        }
      }
      __syncthreads();  // the next block's staging overwrites ut
    }
    return;
  }
  // stage the x slice (M x kl) in LDS
  for (int idx = tid; idx < M * kLowrankRows; idx += 256) {
    const int m = idx / kLowrankRows, k = idx - m * kLowrankRows;
    xl[idx] = k < kl ? xrow(m)[k0 + k] : __float2half(0.f);
  }
  __syncthreads();
  constexpr int RI = kLowrankRows / 32;  // rows per thread
  for (int jb = 0; jb < rpad; jb += 64) {
    const int j = jb + 8 * j8;
    const bool jv = j < rank;
    f16x8 u[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
      const int k = kr + 32 * i;
      u[i] = (jv && k < kl) ? *(const f16x8*)(U + (int64_t)(k0 + k) * rank + j) : f16x8{};
    }
    for (int mb = 0; mb < M; mb += MC) {
      float acc[MC][8];
#pragma unroll
      for (int mm = 0; mm < MC; ++mm)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[mm][c] = 0.f;
#pragma unroll
      for (int i = 0; i < RI; ++i) {
#pragma unroll
        for (int mm = 0; mm < MC; ++mm) {
          const int m = min(mb + mm, M - 1);
          const float xv = (float)xl[m * kLowrankRows + kr + 32 * i];
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[mm][c] = fmaf(xv, (float)u[i][c], acc[mm][c]);
        }
      }
#pragma unroll
      for (int mm = 0; mm < MC; ++mm)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          float v = acc[mm][c];
          v += __shfl_xor(v, 8);
          v += __shfl_xor(v, 16);
          v += __shfl_xor(v, 32);
          acc[mm][c] = v;
        }
      if (lane < 8) {
#pragma unroll
        for (int mm = 0; mm < MC; ++mm)
#pragma unroll
          for (int c = 0; c < 8; ++c) red[(wave * 4 + mm) * 64 + 8 * lane + c] = acc[mm][c];
      }
      __syncthreads();
      {
        const int mm = tid >> 6, jj = tid & 63;
        if (out && mm < MC && mb + mm < M && jb + jj < rpad) {
          const float s = red[(0 * 4 + mm) * 64 + jj] + red[(1 * 4 + mm) * 64 + jj] +
                          red[(2 * 4 + mm) * 64 + jj] + red[(3 * 4 + mm) * 64 + jj];
          if constexpr (COH) handoff_put(out + (mb + mm) * rpad + jb + jj, s);
          else out[(mb + mm) * rpad + jb + jj] = s;
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Consumer tile: 16*T output rows [r0, r0 + 16T) of one item.
// ---------------------------------------------------------------------------
struct PhaseLds {
  const __half* xs;
  const float* xsum;
  const float* xbias;
  const float* s_l;
  const float* z_l;
  int xstride, ncp, group, kl;
};

// Consumes steps [s, min(s + NB, se)) of a batch.  MP = token passes (2-bit:
// 1 for M <= 8, 2 for M <= 16; 4-bit: always 1).
template <int BITS, int T, int NB, int MP>
__device__ __forceinline__ void consume_batch(const u32x4 (&wv)[NB][T], int s, int se,
                                              f32x4 (&yacc)[MP][T], const PhaseLds& P, int M,
                                              int li, int kb, uint32_t xor_mask) {
  constexpr int R = 16 * T;
  constexpr int SC = step_codes<BITS>();
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int st = s + b;
    if (st >= se) break;
    if constexpr (BITS == 2) {
      // half h of this lane's D columns; hl = half held by this lane's A operand
      const int h = li >> 3, hl = kb >> 1;
      const bool hvalid = st * SC + 128 * h < P.kl;    // D-column half inside the phase
      const bool avalid = st * SC + 128 * hl < P.kl;   // A-operand half inside the phase
      const int chunk = 2 * st + h;                     // 128-code chunk of the D half
      const int g = (st * SC + 128 * h) / P.group;      // its quantization group
      f16x8 bx[MP][4][2];
      float c1[MP], c2[MP];
#pragma unroll
      for (int p = 0; p < MP; ++p) {
        const int m = (li & 7) + 8 * p;
        const bool bv = (h == hl) && avalid && m < M;
        const __half* xr = P.xs + m * P.xstride + st * SC + 64 * kb;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int q = 0; q < 2; ++q) bx[p][i][q] = bv ? *(const f16x8*)(xr + 16 * i + 8 * q) : f16x8{};
        const bool cv = hvalid && m < M;
        c1[p] = cv ? P.xbias[m * P.ncp + chunk] : 0.f;
        c2[p] = cv ? P.xsum[m * P.ncp + chunk] : 0.f;
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f32x4 acc[MP];
#pragma unroll
        for (int p = 0; p < MP; ++p) acc[p] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f16x8 a0, a1;
          decode2(wv[b][t][i] ^ xor_mask, a0, a1);
#pragma unroll
          for (int p = 0; p < MP; ++p) {
            acc[p] = mfma_16x16x32(a0, bx[p][i][0], acc[p]);
            acc[p] = mfma_16x16x32(a1, bx[p][i][1], acc[p]);
          }
        }
        if (hvalid) {
          const f32x4 sc = *(const f32x4*)(P.s_l + g * R + t * 16 + 4 * kb);
          const f32x4 zc = *(const f32x4*)(P.z_l + g * R + t * 16 + 4 * kb);
#pragma unroll
          for (int p = 0; p < MP; ++p)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              yacc[p][t][i] += sc[i] * ((acc[p][i] - c1[p]) - zc[i] * c2[p]);
        }
      }
    } else {
      const bool mv = li < M;
      const int g = (st * SC) / P.group;
      f16x8 bx[4];
      const __half* xr = P.xs + li * P.xstride + st * SC + 32 * kb;
#pragma unroll
      for (int i = 0; i < 4; ++i) bx[i] = mv ? *(const f16x8*)(xr + 8 * i) : f16x8{};
      const float c1 = mv ? P.xbias[li * P.ncp + st] : 0.f;
      const float c2 = mv ? P.xsum[li * P.ncp + st] : 0.f;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = mfma_16x16x32(decode4(wv[b][t][i] ^ xor_mask), bx[i], acc);
        const f32x4 sc = *(const f32x4*)(P.s_l + g * R + t * 16 + 4 * kb);
        const f32x4 zc = *(const f32x4*)(P.z_l + g * R + t * 16 + 4 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) yacc[0][t][i] += sc[i] * ((acc[i] - c1) - zc[i] * c2);
      }
    }
  }
}

template <int BITS, int T, int MP, class Src>
__device__ void gemv_tile(const Src& src, const TileShape& sh, int item, int tile,
                          unsigned char* smem) {
  constexpr int R = 16 * T;
  constexpr int NB = batch_steps<T>();
  constexpr int SC = step_codes<BITS>();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int M = src.m_rows(item);
  const int K = sh.K, N = sh.N, G = sh.G;
  const int KP = sh.kp;         // codes per K-phase (multiple of the group and step)
  const int ncp = KP >> 7;      // 128-code chunks per phase
  const int gp = KP / sh.group;  // groups per phase
  const int r0 = tile * R;

  const LdsLayout L = lds_layout(sh.mmax, KP, gp, T, sh.xstride, sh.apad);
  __half* xs = (__half*)(smem + L.xs);      // M x xstride, permuted x of the phase
  float* xsum = (float*)(smem + L.xsum);    // M x ncp
  float* xbias = (float*)(smem + L.xbias);  // M x ncp
  float* s_l = (float*)(smem + L.s);        // gp x R scales
  float* z_l = (float*)(smem + L.z);        // gp x R zero-points
  f32x4* red = (f32x4*)(smem + L.red);      // 4 x T x 64 partial tiles
  __half* a_l = (__half*)(smem + L.a);      // M x apad low-rank factor a

  const __half* S = src.scales(item);
  const __half* Z = src.zeros(item);
  const uint32_t* C = src.codes(item);
  const uint32_t xor_mask = sh.sym ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  int64_t roff[T];
#pragma unroll
  for (int t = 0; t < T; ++t) roff[t] = (int64_t)min(r0 + t * 16 + li, N - 1) * sh.kw;
  f32x4 yacc[MP][T];
#pragma unroll
  for (int p = 0; p < MP; ++p)
#pragma unroll
    for (int t = 0; t < T; ++t) yacc[p][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += KP) {
    const int kl = min(KP, K - k0);         // codes in this phase
    const int nst = (kl + SC - 1) / SC;     // steps in this phase
    const int sb = (wave * nst) >> 2, se = ((wave + 1) * nst) >> 2;
    const int w0 = k0 * BITS / 32;          // first word of the phase in a row
    // ---- first code batch of the phase: in flight while x and s/z stage ----
    u32x4 wv[NB][T];
    if (sb < se) load_batch<T, NB>(wv, C, roff, w0, sb, se, kb, sh.kw - 4);
    // ---- stage x (permuted to operand order) and its per-chunk sums ----
    {
      const int nb = kl >> 4;  // 16-code blocks per token row in this phase
      const int total = M * nb;
      for (int base = 0; base < total; base += 256) {
        const int idx = base + tid;
        const bool v = idx < total;
        float s = 0.f, sb2 = 0.f;
        int m = 0, blk = 0;
        if (v) {
          m = idx / nb;
          blk = idx - m * nb;
          const f16x8* srcx = (const f16x8*)(src.xrow(item, m) + k0 + blk * 16);
          f16x8 in0 = srcx[0], in1 = srcx[1];
          _Float16 in[16], o[16];
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            in[c] = in0[c];
            in[8 + c] = in1[c];
          }
#pragma unroll
          for (int pos = 0; pos < 16; ++pos) {
            o[pos] = in[perm_src<BITS>(pos)];
            const float f = (float)o[pos];
            s += f;
            sb2 += code_bias<BITS>(pos) * f;
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
        }
        // 8 consecutive blocks form one 128-code chunk (nb % 8 == 0).
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        sb2 += __shfl_xor(sb2, 1);
        sb2 += __shfl_xor(sb2, 2);
        sb2 += __shfl_xor(sb2, 4);
        if (v && (idx & 7) == 0) {
          xsum[m * ncp + (blk >> 3)] = s;
          xbias[m * ncp + (blk >> 3)] = sb2;
        }
      }
    }
    // ---- stage this phase's scales / zero-points, transposed to [g][row] ----
    {
      const int g0 = k0 / sh.group;
      const int gl = kl / sh.group;
      const float zsym = (float)(1 << (BITS - 1));
      for (int idx = tid; idx < R * gl; idx += 256) {
        const int row = idx / gl, g = idx - row * gl;
        const int n = min(r0 + row, N - 1);
        s_l[g * R + row] = __half2float(S[(int64_t)n * G + g0 + g]);
        z_l[g * R + row] = sh.sym ? zsym : __half2float(Z[(int64_t)n * G + g0 + g]) + sh.zoff;
      }
    }
    __syncthreads();

    // ---- main loop: this wave's steps, one batch in flight at a time ----
    const PhaseLds P{xs, xsum, xbias, s_l, z_l, sh.xstride, ncp, sh.group, kl};
    for (int st = sb; st < se; st += NB) {
      if (st > sb) load_batch<T, NB>(wv, C, roff, w0, st, se, kb, sh.kw - 4);
      consume_batch<BITS, T, NB, MP>(wv, st, se, yacc, P, M, li, kb, xor_mask);
    }
    __syncthreads();  // the next phase overwrites the staged x / scales
  }

  // ---- 2-bit: merge the two half sums (lanes li and li ^ 8) and move token
  //      li's result to lane li (standard MFMA layout) ----
  if constexpr (BITS == 2) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      f32x4 y0 = yacc[0][t], y1 = yacc[MP - 1][t];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        y0[i] += __shfl_xor(y0[i], 8);
        if (MP == 2) y1[i] += __shfl_xor(y1[i], 8);
      }
      yacc[0][t] = (li < 8) ? y0 : (MP == 2 ? y1 : f32x4{0.f, 0.f, 0.f, 0.f});
    }
  }

  // ---- sum the 4 waves' K-partials; low-rank factor a (M x rank) into LDS ----
#pragma unroll
  for (int t = 0; t < T; ++t) red[(wave * T + t) * 64 + lane] = yacc[0][t];
  const __half* SV = src.sv(item);
  const bool lora = sh.rank > 0 && SV != nullptr;
  if (lora) {
    for (int idx = tid; idx < M * sh.rpad; idx += 256) {
      const int m = idx / sh.rpad, j = idx - m * sh.rpad;
      a_l[m * sh.apad + j] = j < sh.rank ? src.load_a(item, m, j) : __float2half(0.f);
    }
  }
  __syncthreads();

  // ---- epilogue: wave w finishes tiles t = w, w+4, ... ----
  const bool mv = li < M;
  const __half* B = src.bias(item);
  for (int t = wave; t < T; t += 4) {
    f32x4 y = red[(0 * T + t) * 64 + lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4 o = red[(w * T + t) * 64 + lane];
      y += o;
    }
    if (lora) {
      const int rowA = min(r0 + t * 16 + li, N - 1);
      const __half* svr = SV + (int64_t)rowA * sh.rank;
      for (int s = 0; s < sh.rpad; s += 32) {
        const int j = s + 8 * kb;
        f16x8 av = {}, bv = {};
        if (j < sh.rank) av = *(const f16x8*)(svr + j);
        if (mv) bv = *(const f16x8*)(a_l + li * sh.apad + j);
        y = mfma_16x16x32(av, bv, y);
      }
    }
    if (mv) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = r0 + t * 16 + 4 * kb + i;
        if (n < N) {
          float v = y[i];
          if (B) v += __half2float(B[n]);
          src.store(item, li, n, v);
        }
      }
    }
  }
}

// inter = fp16(fp16(silu(fp16(g))) * fp16(u)): the rounding points of
// y = fp16((1/sqrt(d)) H diag(signs) x) of one row of d = 2^logd fp16 values
// (rht_forward(x.float(), signs).half(), inference/moe_block.py:351): the
// row in LDS as fp32 (v, d floats), log2(d) butterfly passes with a barrier
// each, the whole workgroup (nth threads) calling; the order of every sum is
// rht_kernel's (glq_turbo.hip).
__device__ inline void rht_row_f16(const __half* x, const float* signs, __half* y, int d, int logd,
                                   float scale, float* v, int nth) {
  for (int i = threadIdx.x; i < d; i += nth) v[i] = __half2float(x[i]) * signs[i];
  __syncthreads();
  for (int s = 0; s < logd; ++s) {
    const int h = 1 << s;
    for (int p = threadIdx.x; p < d / 2; p += nth) {
      const int i = ((p >> s) << (s + 1)) | (p & (h - 1)), j = i + h;
      const float u = v[i], w = v[j];
      v[i] = u + w;
      v[j] = u - w;
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < d; i += nth) y[i] = __float2half(v[i] * scale);
}

// act_fn(gate(x)) * up(x) on fp16 tensors; the product of two fp16 values is
// exact in fp32, so one rounding gives the correctly rounded fp16 product.
__device__ __forceinline__ __half swiglu_fp16(float g, float u) {
  const float gf = __half2float(__float2half(g));
  const float sl = __half2float(__float2half(gf / (1.f + expf(-gf))));
  return __float2half(sl * __half2float(__float2half(u)));
}

}  // namespace glq
