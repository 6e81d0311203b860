// Streamed token-tile GEMV for the routed experts of a MoE decode step: the
// rows of one expert against the few token rows that picked it, 2-bit
// group-128 codes,
//
//   y[t][n] = sum_g s[n,g] (sum_{k in g} q[n,k] x[t][k] - z[n,g] sum_{k in g} x[t][k])
//
// which is sum_g s[n,g] sum_k (q - z) x, the dequantized row times x (the
// fp16 rounding of q - z that the reference's dequant applies when z has a
// fraction is not reproduced: the difference stays within the fp16 output
// bar).  One v_mfma_f32_16x16x32_f16 per 32 codes of a 16-row tile takes
// all 16 token rows at once (A = x, tokens as rows; B = the codes, weight rows
// as columns), so each code is decoded once for all of the expert's tokens;
// one more MFMA per group against B = 1 gives each token's sum of x.
//
//  * Workgroup (row block rb, K slice s) of W waves: wave w takes the 16 rows
//    [16 (W rb + w), + 16) of each of M2 matrices over the slice's groups, in
//    order, through a ring of R chunks of 4 groups of codes (two 16-byte
//    loads a lane, each covering 8 rows' whole 128-byte lines; the wave's LDS
//    area turns them to 8 bytes of each group for the MFMA) with their
//    rows' scales and zeros (one 8-byte load each) -- the whole row slice in
//    one wave, so no partial sums meet.
//  * x is shared by the waves through LDS: chunks of C groups of the token
//    rows, double-buffered, each staged once by the workgroup (32 bytes a
//    thread) already in the decode order below, rows padded to 272 bytes
//    (the 16 token rows of a lane group fall on different banks).
//  * Lane (li, kb) = (row li of the tile, code quarter kb of the group): each
//    dword of codes decodes to two MFMA steps (codes 0,8,1,9,2,10,3,11 then
//    4,12,5,13,6,14,7,15 of the dword): a v_and_or per pair puts two codes
//    under the exponent of 1024, 256, 64 or 16 and one packed subtract of that
//    offset leaves q exactly.
//  * Token rows past the expert's M only fill MFMA rows that are never stored
//    (a D row depends on its A row alone), so they are neither loaded nor
//    masked.
//  * LORA: slice 0 adds a SV^T (rank <= 64) after its K loop, two MFMA steps
//    per matrix (A = the view's fp16 a of each token row; B = the wave's rows
//    of SV), both loaded in one round trip (loaded with the first codes they
//    would hold 32 VGPRs through the loop: a wave fewer a SIMD).
//  * Each lane stores its outputs (token rows 4 kb .. 4 kb + 3 of row li):
//    SPLIT the slice's partial, store(s, n, t, y); PAIR store(n, t, y0, y1)
//    over the whole K (one slice).  Every sum has a fixed order: the same bits
//    on every run.
#pragma once

#include "glq_gemv_core.h"

namespace glq {

constexpr int kXsRowHalves = 136;  // halves a staged token row of a group (128 + pad)

constexpr int kXsTrRow = 36;        // dwords a row of the code transposition area (32 + pad)

// LDS bytes of the double-buffered x chunks of C groups.
__host__ __device__ constexpr int xs_lds_bytes(int C) { return 2 * C * 16 * kXsRowHalves * 2; }
// LDS bytes of the W waves' code transposition areas (16 rows of a chunk).
__host__ __device__ constexpr int xs_tr_bytes(int W) { return W * 16 * kXsTrRow * 4; }

// Row blocks of 16 W rows, K slices of kg groups (of the G groups of a row).
struct XsGeom {
  int N, K, G, kw;  // kw: int32 words a code row
  int RB, ks, kg;
};

// The 4 B operands (8 fp16 each) of one group's 8 bytes of 2-bit codes: the
// codes q themselves (exact in fp16), in the order the header states.
__device__ __forceinline__ void xs_decode2(const u32x2& w, const DecodeConsts& dk,
                                           f16x8 (&b)[4]) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 c10 = {-1024.f16, -1024.f16}, c8 = {-256.f16, -256.f16}, c6 = {-64.f16, -64.f16},
           c4 = {-16.f16, -16.f16};
  auto sub = [&](uint32_t v, h2 c) -> uint32_t {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v) + c);
  };
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t wd = w[d], v = wd >> 8;
    u32x4 o0, o1;
    o0.x = sub((wd & 0x00030003u) | dk.e25, c10);  // codes 0, 8
    o0.y = sub((wd & 0x000C000Cu) | dk.e23, c8);   // 1, 9
    o0.z = sub((wd & 0x00300030u) | dk.e21, c6);   // 2, 10
    o0.w = sub((wd & 0x00C000C0u) | dk.e19, c4);   // 3, 11
    o1.x = sub((v & 0x00030003u) | dk.e25, c10);   // 4, 12
    o1.y = sub((v & 0x000C000Cu) | dk.e23, c8);    // 5, 13
    o1.z = sub((v & 0x00300030u) | dk.e21, c6);    // 6, 14
    o1.w = sub((v & 0x00C000C0u) | dk.e19, c4);    // 7, 15
    b[2 * d] = __builtin_bit_cast(f16x8, o0);
    b[2 * d + 1] = __builtin_bit_cast(f16x8, o1);
  }
}

// View: codes(m), scales(m), zeros(m) (matrix m's rows; uniform pointers),
// issue_meta() (its loads, issued before the codes), resolve(ts) (the token
// rows M <= 16, the same in every thread, read after the first codes are
// issued; it also finds token rows ts's and li's inputs), xrow_slot() (the
// input row of token row ts, ts = (thread / 8) % 16, valid when ts < M),
// prep(rb, s) (every thread, after the first x chunk is in LDS; may hold
// barriers and use LDS past xs_lds_bytes), with LORA lora() (uniform),
// lora_issue(row, li, kb) (the term's loads, after the K loop), and
// sv_frag(m, s) and a_frag(m, li, s, kb) (the lane's row's SV and token row
// li's a, columns [32 s + 8 kb, + 8), zero past the rank), and the stores.
// Every thread of the W-wave workgroup calls xs_run; each stages 2 C / W
// pieces of 32 bytes of a chunk, of its token row ts = (thread / 8) % 16.
template <class View, bool PAIR, bool LORA, bool SPLIT, int W, int C, int R>
__device__ void xs_run(View& v, const XsGeom& g, int rb, int sl, __half* xlds, uint32_t* tlds) {
  constexpr int M2 = PAIR ? 2 : 1;
  constexpr int NP = 2 * C / W;  // 32-byte x pieces a thread stages a chunk
  static_assert(NP >= 1 && NP * W == 2 * C, "whole x pieces per thread");
  static_assert(C == 4, "a lane's 32 bytes of a chunk row are one group");
  static_assert(R == 2 || R == 3, "a ring of two or three chunks");
  constexpr int BUFH = C * 16 * kXsRowHalves;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int gb = sl * g.kg, ng = max(0, min(g.G, gb + g.kg) - gb);  // the slice's groups
  if (ng == 0) return;  // uniform
  v.issue_meta();

  const int row = min(16 * (W * rb + wave) + li, g.N - 1);
  const int soff = row * g.G;
  int rowq[2];  // code word offsets of the rows this lane loads
#pragma unroll
  for (int h = 0; h < 2; ++h) rowq[h] = min(16 * (W * rb + wave) + 8 * h + (lane >> 3), g.N - 1) * g.kw;
  const int nch = (ng + C - 1) / C;
  // a chunk's codes: two 16-byte loads a lane over the tile's 16 rows x 128
  // bytes (whole lines), passed through LDS to the MFMA order (8 bytes of
  // every group for lane (li, kb)); and the
  // rows' scales and zeros: with G and the slice in whole quads of groups,
  // one 8-byte load of each
  const bool quads = g.G % 4 == 0 && g.kg % 4 == 0;  // uniform
  struct Buf {
    u32x4 c[M2][2];
    u32x2 s[M2], z[M2];  // C fp16 scales, zeros
  };
  auto load_chunk = [&](Buf& b, int c) {  // groups past the slice: its last (unused)
    // load h takes rows 8 h + lane / 8 of the tile, 16 bytes (lane % 8) of
    // each row's 128 bytes: eight whole lines a load
    const int gq = gb + min(c * C + (lane & 7) / 2, ng - 1);
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        b.c[m][h] = *(const u32x4*)(v.codes(m) + rowq[h] + 8 * gq + 4 * (lane & 1));
#pragma unroll
    for (int m = 0; m < M2; ++m) {
      if (quads) {
        const int g0 = gb + c * C;  // + 3 < G
        b.s[m] = *(const u32x2*)(v.scales(m) + soff + g0);
        b.z[m] = *(const u32x2*)(v.zeros(m) + soff + g0);
      } else {
        uint16_t sh[4] = {0, 0, 0, 0}, zh[4] = {0, 0, 0, 0};
#pragma unroll
        for (int gc = 0; gc < C; ++gc) {
          const int gi = gb + min(c * C + gc, ng - 1);
          sh[gc] = ((const uint16_t*)v.scales(m))[soff + gi];
          zh[gc] = ((const uint16_t*)v.zeros(m))[soff + gi];
        }
        b.s[m] = u32x2{sh[0] | ((uint32_t)sh[1] << 16), sh[2] | ((uint32_t)sh[3] << 16)};
        b.z[m] = u32x2{zh[0] | ((uint32_t)zh[1] << 16), zh[2] | ((uint32_t)zh[3] << 16)};
      }
    }
  };
  Buf ring[R];
  load_chunk(ring[0], 0);
  if (nch > 1) load_chunk(ring[1], 1);
  __builtin_amdgcn_sched_barrier(0);  // the codes go out before the routing is read
  const int ts = (tid >> 3) & 15;     // the token row this thread stages
  const int M = v.resolve(ts, li);
  if (M == 0) return;  // uniform: no token picked this expert
  bool lw = false;  // the low-rank term (slice 0)
  if constexpr (LORA) lw = sl == 0 && v.lora();  // uniform

  // x staging: piece j of a chunk = (group q / 128, token row (q / 8) % 16,
  // 16-code pair q % 8), q = tid + 64 W j (token row ts for every j)
  const __half* xrow = v.xrow_slot();
  u32x4 xp[NP][2];
  auto load_x = [&](int c) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int q = tid + 64 * W * j, gi = c * C + q / 128, p = q & 7;
      if (ts < M && gi < ng) {
        const __half* src = xrow + 128 * (gb + gi) + 16 * p;
        xp[j][0] = *(const u32x4*)src;
        xp[j][1] = *(const u32x4*)(src + 8);
      }
    }
  };
  auto store_x = [&](int c) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int q = tid + 64 * W * j, gi = c * C + q / 128, p = q & 7;
      if (ts < M && gi < ng) {
        const f16x8 lo = __builtin_bit_cast(f16x8, xp[j][0]), hi = __builtin_bit_cast(f16x8, xp[j][1]);
        __half* dst = xlds + (c & 1) * BUFH + ((q / 128) * 16 + ts) * kXsRowHalves + 16 * p;
        *(f16x8*)dst = __builtin_shufflevector(lo, hi, 0, 8, 1, 9, 2, 10, 3, 11);
        *(f16x8*)(dst + 8) = __builtin_shufflevector(lo, hi, 4, 12, 5, 13, 6, 14, 7, 15);
      }
    }
  };
  load_x(0);
  store_x(0);
  __syncthreads();
  v.prep(rb, sl);

  f32x4 yv[M2];
#pragma unroll
  for (int m = 0; m < M2; ++m) yv[m] = f32x4{0.f, 0.f, 0.f, 0.f};

  const DecodeConsts dk = DecodeConsts::make();
  // the chunk's codes in MFMA order: each matrix's 16 rows x 128 bytes through
  // the wave's LDS area (its LDS operations run in order; the asm statements
  // keep the compiler from moving the reads above the writes)
  uint32_t* tl = tlds + wave * 16 * kXsTrRow;
  auto transpose = [&](const Buf& b, u32x2 (&cw)[C][M2]) {
#pragma unroll
    for (int m = 0; m < M2; ++m) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int h = 0; h < 2; ++h)
        *(u32x4*)(tl + (8 * h + (lane >> 3)) * kXsTrRow + 4 * (lane & 7)) = b.c[m][h];
      asm volatile("" ::: "memory");
#pragma unroll
      for (int gc = 0; gc < C; ++gc) cw[gc][m] = *(const u32x2*)(tl + li * kXsTrRow + 8 * gc + 2 * kb);
    }
    asm volatile("" ::: "memory");
  };
  auto compute = [&](const Buf& b, const u32x2 (&cw)[C][M2], int gc, const __half* xg) {
    f16x8 xa[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) xa[s] = *(const f16x8*)(xg + li * kXsRowHalves + 32 * kb + 8 * s);
    const f16x8 one = {1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16};
    f32x4 xs = {0.f, 0.f, 0.f, 0.f};  // each token row's sum of x over the group
#pragma unroll
    for (int s = 0; s < 4; ++s) xs = mfma_16x16x32(xa[s], one, xs);
#pragma unroll
    for (int m = 0; m < M2; ++m) {
      f16x8 bb[4];
      xs_decode2(cw[gc][m], dk, bb);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = mfma_16x16x32(xa[s], bb[s], acc);
      const uint32_t sw = b.s[m][gc >> 1], zw = b.z[m][gc >> 1];
      const float sc = __half2float(__ushort_as_half((unsigned short)((gc & 1) ? sw >> 16 : sw)));
      const float z = __half2float(__ushort_as_half((unsigned short)((gc & 1) ? zw >> 16 : zw)));
#pragma unroll
      for (int q = 0; q < 4; ++q) yv[m][q] = fmaf(sc, fmaf(-z, xs[q], acc[q]), yv[m][q]);
    }
  };
  // chunk c decodes from x buffer c & 1 and ring slot c % R; before its
  // groups it issues the next chunk's x and (R = 3) chunk c + 2's codes into
  // the slot chunk c - 1 freed (so the x store after the groups waits for the
  // x alone), or (R = 2) after its groups into its own slot; then one barrier
  for (int c0 = 0; c0 < nch; c0 += R) {
#pragma unroll
    for (int cc = 0; cc < R; ++cc) {
      const int c = c0 + cc;
      if (c < nch) {  // uniform
        if (c + 1 < nch) load_x(c + 1);
        if constexpr (R == 3)
          if (c + 2 < nch) load_chunk(ring[(cc + 2) % 3], c + 2);
        const __half* xb = xlds + (c & 1) * BUFH;
        u32x2 cw[C][M2];
        transpose(ring[cc], cw);
#pragma unroll
        for (int gc = 0; gc < C; ++gc)
          if (c * C + gc < ng) compute(ring[cc], cw, gc, xb + gc * 16 * kXsRowHalves);
        if constexpr (R == 2)
          if (c + 2 < nch) load_chunk(ring[cc], c + 2);
        if (c + 1 < nch) store_x(c + 1);
        __syncthreads();
      }
    }
  }
  if constexpr (LORA) {
    if (lw) {  // a SV^T (uniform): its loads in one round trip after the K loop
      v.lora_issue(row, li, kb);
      f32x4 acc[M2];
#pragma unroll
      for (int m = 0; m < M2; ++m) {
        acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) acc[m] = mfma_16x16x32(v.a_frag(m, li, s, kb), v.sv_frag(m, s), acc[m]);
#pragma unroll
        for (int q = 0; q < 4; ++q) yv[m][q] += acc[m][q];
      }
    }
  }
  const int n = 16 * (W * rb + wave) + li;
  if (n < g.N) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = 4 * kb + q;  // D row: token row
      if (t < M) {
        if constexpr (SPLIT) v.store(sl, n, t, yv[0][q]);
        else if constexpr (PAIR) v.store(n, t, yv[0][q], yv[1][q]);
        else v.store(n, t, yv[0][q]);
      }
    }
  }
}

}  // namespace glq
