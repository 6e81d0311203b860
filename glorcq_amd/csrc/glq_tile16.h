// Token-tile GEMV for a few token rows against the same weight rows (the
// shared expert of a MoE step from 4 tokens, the attention projections of a
// decode step of 4..16 tokens): 4-bit group-128 codes,
//
//   y[t][n] = sum_g s[n,g] * sum_{k in g} fp16(q[n,k] - z[n,g]) x[t][k]
//
// One v_mfma_f32_16x16x32_f16 per 32 codes of a 16-row tile takes all 16
// token rows at once (A = x, tokens as rows; B = the decoded codes, weight rows
// as columns), so each code is decoded once for every token; the lane form
// (glq_lane.h) decodes it once per token.
//
//  * Workgroup (rb, s) takes rows [32 rb, 32 rb + 32) (two tiles) over K
//    slice s: groups [8 s, 8 s + 8), one group a wave (GPW groups a wave:
//    [8 GPW s, 8 GPW (s + 1)), whole rows of up to 8 GPW groups in one
//    workgroup, no slices to sum).  A wave holds the x of
//    every token over its group (16 VGPRs) and the codes of its group in both
//    tiles; per workgroup that is M x 1024 x 2 bytes of x (from L2) against
//    32 x 512 bytes of codes.  Four tiles a block halve the x reads but leave
//    the chip fewer workgroups: config 2's shared expert at 16 tokens ran
//    78.3 us a step with four, 75.5 with two.
//  * Lane (li, kb) = (row li of a tile, 32-code quarter kb of the group)
//    loads 16 bytes of codes per tile; the four 8-code dwords are the four
//    MFMA steps (both operands take the same k order, so the sums are the
//    group's).  Decode: one v_and_or per two codes gives the exact fp16
//    q - round(z) (the prefill GEMM's decode), and a packed fp16 subtract of
//    the fractional part gives fp16(q - z), the reference's fp16 dequant
//    rounding point; the group's fp32 sum is scaled once.
//  * The waves' partial blocks meet in LDS and are summed in wave order.  With
//    several K slices each workgroup writes its block to the workspace and
//    counts itself in on the row block's counter; the last one sums the slices
//    in slice order and stores.  Both orders are fixed: the same bits on every
//    run.  The blocks and the arrival go through glq_handoff.h (coherent
//    atomic stores and loads, no device-scope fence).
//  * PAIR adds a second matrix of the same shape taken in the same pass (gate
//    and up), stored together.
#pragma once

#include "glq_gemv_core.h"
#include "glq_handoff.h"

namespace glq {

constexpr int kT16Waves = 8;              // waves (K groups) a workgroup
constexpr int kT16Tiles = 2;              // 16-row tiles a row block
constexpr int kT16Rows = 16 * kT16Tiles;  // rows a row block
constexpr int kT16Elems = kT16Rows * 16;  // outputs (rows x token rows) a block and matrix
static_assert(kT16Elems % (kT16Waves * 64) == 0, "every thread takes whole outputs of a block");

// LDS bytes: every wave's partial block of each matrix.
__host__ __device__ constexpr int t16_lds_bytes(bool pair) {
  return (pair ? 2 : 1) * kT16Waves * kT16Elems * 4;
}

// The 4 B operands (8 fp16 each, decode order) of one group's 16 bytes of
// 4-bit codes: fp16(q - z).  zi = round(z), zf = z - zi (exact in fp16).
__device__ __forceinline__ void t16_decode4(const u32x4& w, float z, const DecodeConsts& dk,
                                            f16x8 (&b)[4]) {
  const float zi = rintf(z);
  const _Float16 zf = (_Float16)(z - zi);
  const _Float16 c0 = (_Float16)(-(1024.f + zi)), c1 = (_Float16)(-(64.f + zi));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 k0 = {c0, c0}, k1 = {c1, c1}, kf = {zf, zf};
  auto sub = [&](uint32_t v, h2 c) -> uint32_t {
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, v) + c) - kf);
  };
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint32_t wd = w[s], v = wd >> 8;
    u32x4 o;
    o.x = sub((wd & 0x000F000Fu) | dk.e25, k0);  // codes 0, 4
    o.y = sub((wd & 0x00F000F0u) | dk.e21, k1);  // codes 1, 5
    o.z = sub((v & 0x000F000Fu) | dk.e25, k0);   // codes 2, 6
    o.w = sub((v & 0x00F000F0u) | dk.e21, k1);   // codes 3, 7
    b[s] = __builtin_bit_cast(f16x8, o);
  }
}

// Geometry of one token-tile role: N rows of K codes (G groups of 128), M <=
// 16 token rows; RB row blocks of kT16Rows rows, ks K slices of 8 GPW groups; workgroup
// wg = rb ks + s.  With ks > 1, part holds [RB][ks][matrices][kT16Elems]
// partial blocks and cnt[RB] the arrival counters (zero between launches; the
// last workgroup of a row block leaves its counter at zero).
struct T16Geom {
  int N, K, G, kw;  // kw: int32 words per code row
  int M;
  int RB, ks;
  float* part;
  unsigned* cnt;
};

// Output element e of a block: tile j = e / 256, D index i, lane l -> token
// row 4 (l / 16) + i, weight row kT16Rows rb + 16 j + l % 16.
__device__ __forceinline__ void t16_elem(int e, int rb, int& n, int& t) {
  const int l = e & 63;
  t = 4 * (l >> 4) + ((e >> 6) & 3);
  n = kT16Rows * rb + 16 * (e >> 8) + (l & 15);
}

// Src::bind() gives a view with codes(m), scales(m), zeros(m) (m = 0, or 0
// and 1 with PAIR), xrow(t) (token t's activation row, t < M), prep(rb, s,
// ks) (called by every thread of every slice workgroup once its loads are
// issued, before its block is published; may hold barriers and use LDS past
// t16_lds_bytes; what it writes for the finishing workgroup must go out
// through handoff_put) and store(n, t, y) / PAIR store(n, t, y0, y1), called
// for every output of the row block by the workgroup that finishes it
// (reading prep's data through handoff_get); before_store() is called by
// every thread of that workgroup right before its stores (it may hold
// barriers and use all of the LDS: the block is in registers by then).  All
// 512 threads of the workgroup call t16_run (barriers inside).
template <class Src, bool PAIR, int GPW = 1>
__device__ void t16_run(const Src& srcs, const T16Geom& tg, int wg, float* lds) {
  constexpr int M2 = PAIR ? 2 : 1;
  const int rb = wg / tg.ks, sl = wg - rb * tg.ks;
  if (rb >= tg.RB) return;  // uniform over the workgroup
  const auto src = srcs.bind();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int gw0 = (sl * kT16Waves + wave) * GPW;  // this wave's groups gw0 .. + GPW
  bool gon[GPW];  // past G: x = 0, codes of group G - 1 (adds 0)
  int g[GPW];
#pragma unroll
  for (int i = 0; i < GPW; ++i) {
    gon[i] = gw0 + i < tg.G;
    g[i] = gon[i] ? gw0 + i : tg.G - 1;
  }

  // ---- loads: the codes of the tiles, then x; all in flight at once ----
  u32x4 cw[GPW][M2][kT16Tiles];
  __half sv[GPW][M2][kT16Tiles], zv[GPW][M2][kT16Tiles];
#pragma unroll
  for (int i = 0; i < GPW; ++i)
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int j = 0; j < kT16Tiles; ++j) {
        const int row = min(kT16Rows * rb + 16 * j + li, tg.N - 1);
        cw[i][m][j] = *(const u32x4*)((const uint32_t*)src.codes(m) + (int64_t)row * tg.kw +
                                      16 * g[i] + 4 * kb);
        sv[i][m][j] = src.scales(m)[(int64_t)row * tg.G + g[i]];
        zv[i][m][j] = src.zeros(m)[(int64_t)row * tg.G + g[i]];
      }
  const __half* xr0 = src.xrow(li < tg.M ? li : 0) + 32 * kb;
  f16x8 xv[GPW][4];
#pragma unroll
  for (int i = 0; i < GPW; ++i)
#pragma unroll
    for (int s = 0; s < 4; ++s) xv[i][s] = *(const f16x8*)(xr0 + (int64_t)128 * g[i] + 8 * s);
  __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the decode
  // the view's own work for the block, while the codes are in flight (its
  // first wait for its own loads covers theirs too)
  src.prep(rb, sl, tg.ks);

  // the wave's groups in order, each scaled, summed in fp32
  f32x4 yv[M2][kT16Tiles];
#pragma unroll
  for (int m = 0; m < M2; ++m)
#pragma unroll
    for (int j = 0; j < kT16Tiles; ++j) yv[m][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const DecodeConsts dk = DecodeConsts::make();
#pragma unroll
  for (int i = 0; i < GPW; ++i) {
    const bool xon = gon[i] && li < tg.M;
    f16x8 xa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // codes of a dword come decoded as 0,4,1,5,2,6,3,7
      const f16x8 sh = __builtin_shufflevector(xv[i][s], xv[i][s], 0, 4, 1, 5, 2, 6, 3, 7);
      xa[s] = xon ? sh : f16x8{};
    }
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int j = 0; j < kT16Tiles; ++j) {
        f16x8 b[4];
        t16_decode4(cw[i][m][j], __half2float(zv[i][m][j]), dk, b);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = mfma_16x16x32(xa[s], b[s], acc);
        const float sc = __half2float(sv[i][m][j]);
#pragma unroll
        for (int q = 0; q < 4; ++q) yv[m][j][q] = fmaf(sc, acc[q], yv[m][j][q]);
      }
  }
#pragma unroll
  for (int m = 0; m < M2; ++m)
#pragma unroll
    for (int j = 0; j < kT16Tiles; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        lds[((m * kT16Waves + wave) * kT16Tiles + j) * 256 + i * 64 + lane] = yv[m][j][i];
  __syncthreads();

  // ---- the block: waves summed in order; thread tid takes elements tid + 512 q ----
  constexpr int EPT = kT16Elems / (kT16Waves * 64);
  float v[M2][EPT];
#pragma unroll
  for (int m = 0; m < M2; ++m)
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int e = tid + q * kT16Waves * 64;
      float a = 0.f;
#pragma unroll
      for (int w = 0; w < kT16Waves; ++w) a += lds[(m * kT16Waves + w) * kT16Elems + e];
      v[m][q] = a;
    }

  if (tg.ks > 1) {
    float* pb = tg.part + (int64_t)(rb * tg.ks + sl) * M2 * kT16Elems;
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int q = 0; q < EPT; ++q)
        handoff_put(pb + m * kT16Elems + tid + q * kT16Waves * 64, v[m][q]);
    __shared__ int last;
    if (!handoff_arrive(tg.cnt + rb, (unsigned)tg.ks, &last)) return;
    const float* p0 = tg.part + (int64_t)rb * tg.ks * M2 * kT16Elems;
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int q = 0; q < EPT; ++q) {
        const int e = m * kT16Elems + tid + q * kT16Waves * 64;
        float a = 0.f;
        for (int s = 0; s < tg.ks; ++s) a += handoff_get(p0 + (int64_t)s * M2 * kT16Elems + e);
        v[m][q] = a;
      }
    if (tid == 0) handoff_reset(tg.cnt + rb);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // prep's stores, for the store phase
    __syncthreads();
  }
  src.before_store();
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    int n, t;
    t16_elem(tid + q * kT16Waves * 64, rb, n, t);
    if (n < tg.N && t < tg.M) {
      if constexpr (PAIR) src.store(n, t, v[0][q], v[1][q]);
      else src.store(n, t, v[0][q]);
    }
  }
}

}  // namespace glq
