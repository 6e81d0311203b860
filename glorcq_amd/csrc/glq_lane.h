// Lane-sliced fused dequant-GEMV + low-rank correction for one token row
// (M = 1, group 128): the decode shape of every expert and attention
// projection at batch 1.
//
//   y[n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) x[k]
//        + sum_j a[j] SV[n,j] + bias[n],          a = fp16(x U)
//
// With one token row a 16x16 MFMA tile wastes 15 of its 16 token columns,
// and the MFMA time then exceeds the decode.  Here the wave's lanes own fixed
// K slices instead:
//  * a row of codes is K*bits/8 bytes = LR 16-byte pieces (LR <= 64 NP, NP
//    pieces a lane); lanes are grouped by LRP = LR rounded up to 16, 32 or
//    64, so one wave iteration covers RPI = 64 / LRP rows, lane l holding
//    piece l % LRP (+ j LRP) of row l / LRP.  Every load instruction of codes is 64 lanes x 16 bytes of
//    consecutive rows -- contiguous when LR = LRP.
//  * lane l's x slice (the 64 or 32 codes of its piece) lives in registers
//    for the whole run of rows, already in the decode's operand order, with
//    its operand-bias sum c1 = sum 2^e(k) x[k] and c2 = sum x[k];
//  * codes decode into packed fp16 (2^e + q) with one v_and_or per two codes
//    (the same decode as the MFMA kernels) and meet x in v_dot2c_f32_f16, fp32
//    accumulate; per row the lane adds s * (dot - c1 - z c2) and its share of
//    a SV^T (one dword of SV per lane per 64 rank columns);
//  * the LRP lanes of a row reduce with DPP (strides 1, 2, 4, 8) and the
//    gfx950 permlane16/permlane32 swaps; lane l keeps the total of the row it
//    will store, so the 64 rows of a wave's unit leave in one 128-byte store.
//  * loads run PD iterations ahead of use in a register ring; nothing goes
//    through LDS.
// Semantics as gemv_tile (glq_gemv_core.h), so outputs of the two agree to
// fp32 summation order.
#pragma once

#include <type_traits>

#include "glq_gemv_core.h"

namespace glq {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Codes per lane piece (16 bytes).
template <int BITS>
constexpr int lane_piece_codes() { return 128 / BITS; }

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                false);
}

// Sum over the LRP lanes of each lane group; every lane of the group gets it.
template <int LRP>
__device__ __forceinline__ float lane_group_sum(float v) {
  auto dpp_add = [](float x, int ctrl) -> float {
    int y = 0;
    switch (ctrl) {  // the control word must be an immediate
      case 0: y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false); break;
      case 1: y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false); break;
      case 2: y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false); break;
      default: y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false); break;
    }
    return x + __int_as_float(y);
  };
  v = dpp_add(v, 0);  // quad_perm [1,0,3,2]: lane ^ 1
  v = dpp_add(v, 1);  // quad_perm [2,3,0,1]: lane ^ 2
  v = dpp_add(v, 2);  // row_half_mirror: lane i <-> 7 - i within each 8 (quads summed)
  v = dpp_add(v, 3);  // row_mirror: lane i <-> 15 - i within each 16
  if constexpr (LRP >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // rows 0+1, 2+3
  }
  if constexpr (LRP >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // halves
  }
  return v;
}

// Buffer descriptor word 3 for gfx9-family raw buffers (offset-mode range
// check against num_records), and the load's cache-policy bits: nontemporal.
constexpr int kBufferFlags = 0x00020000;
constexpr int kBufferNT = 2;

// Decoded operands of one code word as packed fp16 pairs (decode2 / decode4).
__device__ __forceinline__ void decode2_words(uint32_t w, u32x4& a, u32x4& b,
                                              const DecodeConsts& k) {
  const uint32_t v = w >> 10;
  a.x = (w & 0x00030003u) | k.e25;
  a.y = (w & 0x000C000Cu) | k.e23;
  a.z = (w & 0x00300030u) | k.e21;
  a.w = (w & 0x00C000C0u) | k.e19;
  b.x = (w & 0x03000300u) | k.e17;
  b.y = (v & 0x00030003u) | k.e25;
  b.z = (v & 0x000C000Cu) | k.e23;
  b.w = (v & 0x00300030u) | k.e21;
}
__device__ __forceinline__ void decode4_words(uint32_t w, u32x4& a, const DecodeConsts& k) {
  const uint32_t v = w >> 8;
  a.x = (w & 0x000F000Fu) | k.e25;
  a.y = (w & 0x00F000F0u) | k.e21;
  a.z = (v & 0x000F000Fu) | k.e25;
  a.w = (v & 0x00F000F0u) | k.e21;
}

// The x U phase of the lane kernel (XU): 512 threads, thread t owns column
// block b = t % NB (8 rank columns, one 16-byte load per U row) and K slot
// t / NB of KS = 512 / NB slots; slot s sums 8-row chunks s, s + KS, ...
// Its fp32 partials go to LDS (KS x rank), are summed first over slots
// s = seg (mod NSEG) by 512 threads (NSEG = 512 / rank segments per column),
// then over the segments, both in a fixed order.
struct LaneXu {
  int nb, ks, nseg;
  __host__ __device__ explicit LaneXu(int rank)
      : nb(rank / 8), ks(512 / (rank / 8)), nseg(512 / rank) {}
  // LDS bytes: slot partials, segment sums, a in fp16
  __host__ __device__ int lds_bytes(int rank) const {
    return ks * rank * 4 + nseg * rank * 4 + rank * 2;
  }
};

// sum_{k0 <= k < k0 + kn} x[k] U[k][:] (fp32, kn a multiple of 8) of one item
// by all 512 threads of the workgroup (layout in LaneXu): U rows read by
// whole-row wave loads, two 8-row chunks in flight per thread, v_dot2 over
// row pairs into fp32, the partials summed in LDS in a fixed order.  Returns
// the sums' LDS copy (rank floats); every thread of the workgroup must call
// it (it holds barriers).
// DEPTH: 8-row chunks in flight per thread (0: one row pair at a time, for
// callers short of registers; every DEPTH gives the same sums in the same
// order).
template <class View, int DEPTH = 2>
__device__ float* lane_xu_sum(const View& src, int k0, int kn, int rank, float* xu_lds) {
  const LaneXu L(rank);
  const int t = threadIdx.x;
  float* part = xu_lds;                      // (ks, rank)
  float* segs = xu_lds + L.ks * rank;        // (nseg, rank)
  const int b = t % L.nb, slot = t / L.nb;
  if (slot < L.ks) {
    const int nch = kn / 8;  // 8-row chunks
    const __half* ub = src.u() + (int64_t)k0 * rank + 8 * b;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    u32x4 u0[8], u1[8], x0, x1;
    auto load = [&](int c, u32x4 (&u)[8], u32x4& xv) {
      c = min(c, nch - 1);  // past the end: re-read the last chunk (not used)
      xv = src.x8(k0 + 8 * c);
#pragma unroll
      for (int q = 0; q < 8; ++q) u[q] = *(const u32x4*)(ub + (int64_t)(8 * c + q) * rank);
    };
    auto fma_chunk = [&](const u32x4 (&u)[8], const u32x4& xv) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // rows 2i, 2i + 1 against (x_2i, x_2i+1)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = __builtin_amdgcn_perm(u[2 * i + 1][j], u[2 * i][j], 0x05040100u);
          const uint32_t hi = __builtin_amdgcn_perm(u[2 * i + 1][j], u[2 * i][j], 0x07060302u);
          acc[2 * j] = dot2(lo, xv[i], acc[2 * j]);
          acc[2 * j + 1] = dot2(hi, xv[i], acc[2 * j + 1]);
        }
      }
    };
    // chunks slot, slot + ks, ... (two in flight); a slot at or past the
    // last chunk adds nothing
    if constexpr (DEPTH == 0) {
      for (int c = slot; c < nch; c += L.ks) {
        const u32x4 xv = src.x8(k0 + 8 * c);
#pragma unroll 1
        for (int i = 0; i < 4; ++i) {  // rows 2i, 2i + 1: fma_chunk's steps for i
          const u32x4 ua = *(const u32x4*)(ub + (int64_t)(8 * c + 2 * i) * rank);
          const u32x4 uc = *(const u32x4*)(ub + (int64_t)(8 * c + 2 * i + 1) * rank);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t lo = __builtin_amdgcn_perm(uc[j], ua[j], 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(uc[j], ua[j], 0x07060302u);
            acc[2 * j] = dot2(lo, xv[i], acc[2 * j]);
            acc[2 * j + 1] = dot2(hi, xv[i], acc[2 * j + 1]);
          }
        }
      }
    } else if constexpr (DEPTH == 1) {
      for (int c = slot; c < nch; c += L.ks) {
        load(c, u0, x0);
        fma_chunk(u0, x0);
      }
    } else {
      load(slot, u0, x0);
      for (int c = slot; c < nch; c += 2 * L.ks) {
        load(c + L.ks, u1, x1);
        fma_chunk(u0, x0);
        if (c + L.ks >= nch) break;
        load(c + 2 * L.ks, u0, x0);
        fma_chunk(u1, x1);
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) part[slot * rank + 8 * b + c] = acc[c];
  }
  __syncthreads();
  const int col = t % rank, seg = t / rank;
  if (seg < L.nseg) {  // level 1: slots seg, seg + nseg, ... in order
    float sum = 0.f;
    for (int q = seg; q < L.ks; q += L.nseg) sum += part[q * rank + col];
    segs[seg * rank + col] = sum;
  }
  __syncthreads();
  if (t < rank) {  // level 2: the segments in order, into part's first row
    float sum = 0.f;
    for (int q = 0; q < L.nseg; ++q) sum += segs[q * rank + t];
    part[t] = sum;
  }
  __syncthreads();
  return part;
}

// a = fp16(x U) over the whole row (K codes), in LDS (rank halves).
template <class View>
__device__ __half* lane_xu_phase(const View& src, int K, int rank, bool lora, float* xu_lds) {
  const LaneXu L(rank);
  __half* ah = (__half*)(xu_lds + L.ks * rank + L.nseg * rank);
  if (!lora) return ah;
  const float* sums = lane_xu_sum(src, 0, K, rank, xu_lds);
  if ((int)threadIdx.x < rank) ah[threadIdx.x] = __float2half(sums[threadIdx.x]);
  __syncthreads();
  return ah;
}

// Item types may issue the loads of a before the x slice's wait
// (a_issue(j, v) / a_issue(m, j, v) with PAIR: up to kLaneEarlyA fp32 partials
// of a[j] into v, zeros past them, and a_count() of them); lane_run then sums
// them after that wait, in sum_strided's order, so one memory round trip
// covers the rows' first loads, x and a.
constexpr int kLaneEarlyA = 4;
template <class T, class = void>
struct lane_early_a : std::false_type {};
template <class T>
struct lane_early_a<T, std::void_t<decltype(&T::a_count)>> : std::true_type {};
// Item types may also have after_issue(): work of the whole workgroup (it may
// hold barriers) run by every wave right after its rows' first loads are
// issued, so its own loads share their round trip.  Waves without rows of
// their own take part too.
template <class T, class = void>
struct lane_hook : std::false_type {};
template <class T>
struct lane_hook<T, std::void_t<decltype(&T::after_issue)>> : std::true_type {};


// sum_strided's sum of n <= kLaneEarlyA loaded partials (its zeros included)
__device__ __forceinline__ float lane_early_sum(const float (&v)[kLaneEarlyA]) {
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kLaneEarlyA; ++u) s += v[u];
#pragma unroll
  for (int u = kLaneEarlyA; u < 8; ++u) s += 0.f;
  return s;
}

// Geometry of one lane launch (or one role of a launch): every item has N
// rows of K codes; rows are cut into 64-row units of NIT = LRP iterations,
// taken in rounds of PD iterations; wave w of an item runs rounds
// w rpw .. w rpw + rpw - 1 and stores each round's rows at the round's end.
struct LaneGeom {
  int N, K, G, kw, rank;
  int group;   // codes per quantization group (a multiple of the piece's codes)
  float zoff;  // added to every zero-point (signed codes stored offset by 2^(b-1))
  int lr;      // 16-byte pieces per code row
  int rounds;  // rounds of PD iterations per item (64-row units x LRP / PD)
  int wpi;     // waves per item
  int rpw;     // rounds per wave (consecutive rounds of one item)
  int items;
};

// Item data of a lane launch.  A source type's bind(item) gives a view of one
// item with:
//   lora()                the low-rank term is present
//   codes/scales/zeros/sv/bias/u()   the item's tensors (bias may be null)
//   x8(k)                 8 halves of the item's activation row at k (k % 8 == 0)
//   load_a(j)             a[j] when a is given (not XU)
//   store(n, v)           the item's output row n
//
// Work per wave: PD iterations of loads in flight ahead of use.  Loads are
// issued unconditionally (iterations past the wave's last one re-read its
// last row), so the register ring needs no copies and the compiler's waits
// stay PD deep.  NP: 16-byte pieces per lane (a row of up to 64 NP pieces;
// lane l holds pieces l % LRP + j LRP).  NSV: SV dwords per lane (rank <= 2
// NSV LRP); HASB: a bias is added.
//
// XU: the low-rank factor a = fp16(x U) is formed in the same launch, first:
// each workgroup (8 waves, all of one item) reads the item's U with every
// wave-wide load covering whole 128-byte U rows (layout in LaneXu), two
// chunks of loads in flight per thread, v_dot2 over row pairs into fp32; the
// partials are summed in LDS in a fixed order and rounded to fp16 once.
// Then the waves take their x slices and stream their rows.  An item whose
// rows are spread over several workgroups has each of them form a.
//
// DEFER (with XU): a is formed elsewhere in the launch.  When the item's
// xu_defer() is true, each wave sums its first round without the low-rank
// term, then the workgroup calls the item's xu_wait(K, rank, xu_lds) (every
// thread; it returns a's fp16 LDS copy at lane_xu_phase's place in xu_lds),
// and the round is finished with the same operations in the same order.
template <class Src, int BITS, bool SYM, int LRP, int NP, int PD, int NSV, bool HASB, bool XU,
          bool PAIR = false, bool DEFER = false>
__device__ __forceinline__ void lane_run(const Src& srcs, const LaneGeom& lg, int wv, int wvb,
                                         float* xu_lds) {
  constexpr int C = lane_piece_codes<BITS>();  // codes per piece
  constexpr int RPI = 64 / LRP;                // rows per iteration
  constexpr int NIT = LRP;                     // row groups per 64-row unit
  constexpr int M2 = PAIR ? 2 : 1;             // matrices
  static_assert(NIT % PD == 0, "ring depth must divide the unit");
  static_assert(!PAIR || (PD % 2 == 0 && !XU && !HASB), "pairs: even depth, a given");
  static_assert(NP == 1 || LRP == 64, "several pieces per lane take whole waves per row");
  const int lane = threadIdx.x & 63;
  const int item = wv / lg.wpi;
  if (item >= lg.items) return;  // uniform over the workgroup (XU: wpi is a multiple of 8)
  // rounds rb .. rb + nr - 1 of PD iterations each, [PD R, PD R + PD)
  const int rb = (wv - item * lg.wpi) * lg.rpw;
  const int nr = min(lg.rpw, lg.rounds - rb);
  constexpr bool HOOK = lane_hook<decltype(srcs.bind(0))>::value;
  if (!XU && !HOOK && nr <= 0) return;  // (XU, HOOK: every wave takes part)
  const auto src = srcs.bind(item);
  const int rlast = min(rb + max(nr, 1), lg.rounds) - 1;  // idle waves re-read a valid round
  const int N = lg.N, G = lg.G, kw = lg.kw, rank = lg.rank;
  const int ri = lane / LRP, p = lane % LRP;
  bool act[NP];
  int pc[NP], gq[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int pj = p + j * LRP;
    act[j] = pj < lg.lr;
    pc[j] = act[j] ? pj : lg.lr - 1;  // inactive pieces read a valid one (x = 0)
    gq[j] = pc[j] * C / lg.group;     // the piece's quantization group
  }

  // ---- x slices in operand order, c1 = sum bias * x, c2 = sum x ----
  uint32_t xw[NP][C / 2];
  float c1[NP], c2[NP];
  auto load_x = [&]() {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      c1[j] = 0.f;
      c2[j] = 0.f;
#pragma unroll
      for (int blk = 0; blk < C / 16; ++blk) {
        const f16x8 in0 = __builtin_bit_cast(f16x8, src.x8(pc[j] * C + 16 * blk));
        const f16x8 in1 = __builtin_bit_cast(f16x8, src.x8(pc[j] * C + 16 * blk + 8));
        _Float16 in[16], o[16];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          in[c] = act[j] ? in0[c] : (_Float16)0.f;
          in[8 + c] = act[j] ? in1[c] : (_Float16)0.f;
        }
#pragma unroll
        for (int pos = 0; pos < 16; ++pos) {
          o[pos] = in[perm_src<BITS>(pos)];
          const float f = (float)o[pos];
          c2[j] += f;
          c1[j] += code_bias<BITS>(pos) * f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const f16x2 pr = {o[2 * q], o[2 * q + 1]};
          xw[j][8 * blk + q] = __builtin_bit_cast(uint32_t, pr);
        }
      }
      // the zero-point offset leaves with the operand bias: z + zoff per piece
      if constexpr (!SYM) c1[j] = fmaf(lg.zoff, c2[j], c1[j]);
    }
  };
  const bool lora = src.lora();
  // the item's tensors of matrix m (PAIR: 0 and 1, iterations alternating)
  auto t_codes = [&](int m) { if constexpr (PAIR) return src.codes(m); else return src.codes(); };
  auto t_scales = [&](int m) { if constexpr (PAIR) return src.scales(m); else return src.scales(); };
  auto t_zeros = [&](int m) { if constexpr (PAIR) return src.zeros(m); else return src.zeros(); };
  auto t_sv = [&](int m) { if constexpr (PAIR) return src.sv(m); else return src.sv(); };
  int svo[NSV];  // element offset of the dword within an SV row
#pragma unroll
  for (int k = 0; k < NSV; ++k) {
    const int j = p + k * LRP;  // dword j holds rank columns 2j, 2j + 1
    svo[k] = lora && 2 * j < rank ? 2 * j : 0;
  }

  // Buffer loads: one descriptor per tensor of the item (sized to it, so rows
  // past N read 0 and add 0); a lane's offset is its constant part plus the
  // iteration's first row times the row pitch.  Row of iteration i:
  // (i / NIT) * 64 + (i % NIT) * RPI + ri = RPI i + ri (PAIR: matrix i % 2,
  // row RPI (i / 2) + ri).
  const int rowbytes = kw * 4;
  decltype(__builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0)) rc[M2], rsc[M2], rz[M2], rsv[M2];
#pragma unroll
  for (int m = 0; m < M2; ++m) {
    rc[m] = __builtin_amdgcn_make_buffer_rsrc((void*)t_codes(m), 0, N * rowbytes, kBufferFlags);
    rsc[m] = __builtin_amdgcn_make_buffer_rsrc((void*)t_scales(m), 0, N * G * 2, kBufferFlags);
    rz[m] = __builtin_amdgcn_make_buffer_rsrc((void*)(SYM ? t_scales(m) : t_zeros(m)), 0,
                                              N * G * 2, kBufferFlags);
    // without a low-rank term the SV descriptor has no records: its loads read 0
    rsv[m] = __builtin_amdgcn_make_buffer_rsrc(lora ? (void*)t_sv(m) : (void*)t_codes(m), 0,
                                               lora ? N * rank * 2 : 0, kBufferFlags);
  }
  auto bias_ptr = [&]() -> void* {
    if constexpr (HASB) return (void*)src.bias();
    else return nullptr;
  };
  const auto rbi = __builtin_amdgcn_make_buffer_rsrc(bias_ptr(), 0, HASB ? N * 2 : 0,
                                                     kBufferFlags);
  const int svr = lora ? rank : 0;
  int vc[NP], vs[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    vc[j] = ri * rowbytes + pc[j] * 16;
    vs[j] = (ri * G + gq[j]) * 2;
  }
  const int vb = ri * 2;
  int vsv[NSV];
#pragma unroll
  for (int k = 0; k < NSV; ++k) vsv[k] = (ri * svr + svo[k]) * 2;
  const float bsel = p == 0 ? 1.f : 0.f;  // the first lane of a row group adds the bias

  u32x4 cw[PD][NP];
  uint32_t sw[PD][NP], zw[PD][NP], bw[PD], vw[PD][NSV];
  // loads of iteration d of the wave's round r (rounds past the last re-read it)
  auto issue = [&](int d, int r) {
    const int m = PAIR ? (d & 1) : 0;  // compile-time once unrolled
    const int it = min(rb + r, rlast) * PD + d;
    const int n0 = RPI * (PAIR ? it >> 1 : it);  // uniform
    if constexpr (HASB) bw[d] = __builtin_amdgcn_raw_buffer_load_b16(rbi, vb + n0 * 2, 0, 0);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      cw[d][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               rc[m], vc[j] + n0 * rowbytes, 0, kBufferNT));
      sw[d][j] = __builtin_amdgcn_raw_buffer_load_b16(rsc[m], vs[j] + n0 * G * 2, 0, 0);
      if constexpr (!SYM)
        zw[d][j] = __builtin_amdgcn_raw_buffer_load_b16(rz[m], vs[j] + n0 * G * 2, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < NSV; ++k)
      vw[d][k] = __builtin_amdgcn_raw_buffer_load_b32(rsv[m], vsv[k] + n0 * svr * 2, 0, 0);
  };
  // The prologue's loads go out in the loop's order (scheduling barriers on
  // both sides of every issue), so the wait the compiler places at the loop
  // head -- the tighter of the two entry states -- stays PD - 1 iterations deep.
  auto prologue = [&]() {
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      __builtin_amdgcn_sched_barrier(0);
      issue(d, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // the rows' loads go out first; x and a (below) arrive under them
  using Item = std::decay_t<decltype(src)>;
  constexpr bool EARLY = !XU && lane_early_a<Item>::value;
  float araw[EARLY ? M2 : 1][EARLY ? NSV : 1][2][kLaneEarlyA];
  bool early = false;
  if constexpr (!XU) {
    if (!HOOK || nr > 0) prologue();
    if constexpr (HOOK) {
      src.after_issue();
      if (nr <= 0) return;
    }
    if constexpr (EARLY) {
      early = src.lora() && src.a_count() <= kLaneEarlyA;
      if (early) {
#pragma unroll
        for (int m = 0; m < M2; ++m)
#pragma unroll
          for (int k = 0; k < NSV; ++k)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const int j = min(2 * (p + k * LRP) + e, rank - 1);  // past the rank: unused
              if constexpr (PAIR) src.a_issue(m, j, araw[m][k][e]);
              else src.a_issue(j, araw[m][k][e]);
            }
      }
    }
    load_x();
  }

  // ---- a pairs of this lane's SV dwords (zero past the rank) ----
  uint32_t ap[M2][NSV];
  auto set_ap = [&](const __half* ah) {
#pragma unroll
    for (int k = 0; k < NSV; ++k) {
      const int j = p + k * LRP;
      f16x2 pr = {(_Float16)0.f, (_Float16)0.f};
      if (lora && 2 * j < rank) {
        pr[0] = (_Float16)__half2float(ah[2 * j]);
        pr[1] = (_Float16)__half2float(ah[2 * j + 1]);
      }
      ap[0][k] = __builtin_bit_cast(uint32_t, pr);
    }
  };
  // DEFER: a handed over by other workgroups (the item's xu_defer()); the
  // wave's first round is summed before a is waited for (below)
  bool defer = false;
  if constexpr (XU) {
    // the rows' first loads go out before the x U phase and arrive under it
    if (nr > 0) prologue();
    if constexpr (DEFER) defer = src.xu_defer();
    if (!defer) {
      set_ap(lane_xu_phase(src, lg.K, rank, lora, xu_lds));
      if (nr <= 0) return;  // a wave with no rows of its own
    }
    if (nr > 0) load_x();
  } else {
#pragma unroll
    for (int m = 0; m < M2; ++m)
#pragma unroll
      for (int k = 0; k < NSV; ++k) {
        const int j = p + k * LRP;
        f16x2 pr = {(_Float16)0.f, (_Float16)0.f};
        if constexpr (EARLY) {
          if (early && 2 * j < rank) {
            pr[0] = (_Float16)lane_early_sum(araw[m][k][0]);
            pr[1] = (_Float16)lane_early_sum(araw[m][k][1]);
            ap[m][k] = __builtin_bit_cast(uint32_t, pr);
            continue;
          }
        }
        if (lora && 2 * j < rank) {
          if constexpr (PAIR) {
            pr[0] = (_Float16)__half2float(src.load_a(m, 2 * j));
            pr[1] = (_Float16)__half2float(src.load_a(m, 2 * j + 1));
          } else {
            pr[0] = (_Float16)__half2float(src.load_a(2 * j));
            pr[1] = (_Float16)__half2float(src.load_a(2 * j + 1));
          }
        }
        ap[m][k] = __builtin_bit_cast(uint32_t, pr);
      }
  }

  const DecodeConsts dk = DecodeConsts::make();
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  int r0 = 0;
  if constexpr (XU && DEFER) {
    if (defer) {
      // the quantized sum (and bias) of this lane's pieces of iteration d
      // (the loop's steps below)
      auto qpart = [&](int d) {
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < NP; ++j) {
          u32x4 w = cw[d][j];
          if constexpr (SYM) w ^= xor_mask;
          float acc0 = -c1[j], acc1 = 0.f;  // the operand bias leaves with c1
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            if constexpr (BITS == 2) {
              u32x4 da, db;
              decode2_words(w[k], da, db, dk);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                acc0 = dot2(da[q], xw[j][8 * k + q], acc0);
                acc1 = dot2(db[q], xw[j][8 * k + 4 + q], acc1);
              }
            } else {
              u32x4 da;
              decode4_words(w[k], da, dk);
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                if (q & 1) acc1 = dot2(da[q], xw[j][4 * k + q], acc1);
                else acc0 = dot2(da[q], xw[j][4 * k + q], acc0);
              }
            }
          }
          const float s = __half2float(__ushort_as_half((uint16_t)sw[d][j]));
          float z = (float)(1 << (BITS - 1));
          if constexpr (!SYM) z = __half2float(__ushort_as_half((uint16_t)zw[d][j]));
          part = fmaf(s, (acc0 + acc1) - z * c2[j], part);
        }
        if constexpr (HASB) part = fmaf(bsel, __half2float(__ushort_as_half((uint16_t)bw[d])), part);
        return part;
      };
      // lane l holds row (l % LRP) * RPI + l / LRP of the unit; the lanes of
      // round r's row groups store
      auto store_round = [&](int r, float yv, float yu) {
        constexpr int RG = PAIR ? PD / 2 : PD;  // row groups per round
        const int i0 = (rb + r) * PD;
        const int g0 = PAIR ? i0 >> 1 : i0;
        const int u = g0 / NIT, it0 = g0 & (NIT - 1);
        const int n = u * 64 + p * RPI + ri;
        if (p >= it0 && p < it0 + RG && n < N) {
          if constexpr (PAIR) src.store(n, yv, yu);
          else src.store(n, yv);
        }
      };
      // round 0 without the low-rank term; then a (the whole workgroup),
      // the term, the next round's loads, the sums and the stores -- the
      // same operations in the same order as the loop below
      float pt[PD];
      if (nr > 0) {
#pragma unroll
        for (int d = 0; d < PD; ++d) pt[d] = qpart(d);
      }
      set_ap(src.xu_wait(lg.K, rank, xu_lds));
      if (nr <= 0) return;  // a wave with no rows of its own
      float yv = 0.f;
#pragma unroll
      for (int d = 0; d < PD; ++d) {
        float part = pt[d];
#pragma unroll
        for (int k = 0; k < NSV; ++k) part = dot2(vw[d][k], ap[0][k], part);
        if (nr > 1) {  // (a single round reads nothing more)
          __builtin_amdgcn_sched_barrier(0);
          issue(d, 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        const float tot = lane_group_sum<LRP>(part);
        yv = p == ((rb * PD + d) & (NIT - 1)) ? tot : yv;
      }
      store_round(0, yv, 0.f);
      // x again for later rounds (its registers were free over the wait)
      if (nr > 1) load_x();
      r0 = 1;
    }
  }
  for (int r = r0; r < nr; ++r) {
    const int i0 = (rb + r) * PD;  // first iteration of the round
    float yv = 0.f, yu = 0.f;      // (PAIR: matrix 0 and matrix 1 of a row)
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      const int i = i0 + d;
      const int m = PAIR ? (d & 1) : 0;
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        u32x4 w = cw[d][j];
        if constexpr (SYM) w ^= xor_mask;
        float acc0 = -c1[j], acc1 = 0.f;  // the operand bias leaves with c1
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if constexpr (BITS == 2) {
            u32x4 da, db;
            decode2_words(w[k], da, db, dk);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              acc0 = dot2(da[q], xw[j][8 * k + q], acc0);
              acc1 = dot2(db[q], xw[j][8 * k + 4 + q], acc1);
            }
          } else {
            u32x4 da;
            decode4_words(w[k], da, dk);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (q & 1) acc1 = dot2(da[q], xw[j][4 * k + q], acc1);
              else acc0 = dot2(da[q], xw[j][4 * k + q], acc0);
            }
          }
        }
        const float s = __half2float(__ushort_as_half((uint16_t)sw[d][j]));
        float z = (float)(1 << (BITS - 1));
        if constexpr (!SYM) z = __half2float(__ushort_as_half((uint16_t)zw[d][j]));
        part = fmaf(s, (acc0 + acc1) - z * c2[j], part);
      }
      if constexpr (HASB) part = fmaf(bsel, __half2float(__ushort_as_half((uint16_t)bw[d])), part);
#pragma unroll
      for (int k = 0; k < NSV; ++k) part = dot2(vw[d][k], ap[m][k], part);
      __builtin_amdgcn_sched_barrier(0);
      issue(d, r + 1);
      __builtin_amdgcn_sched_barrier(0);
      const float tot = lane_group_sum<LRP>(part);
      if constexpr (PAIR) {
        const bool mine = p == ((i >> 1) & (NIT - 1));
        if (m == 0) yv = mine ? tot : yv;
        else yu = mine ? tot : yu;
      } else {
        yv = p == (i & (NIT - 1)) ? tot : yv;
      }
    }
    // lane l holds row (l % LRP) * RPI + l / LRP of the unit; the lanes of
    // the round's row groups store
    constexpr int RG = PAIR ? PD / 2 : PD;  // row groups per round
    const int g0 = PAIR ? i0 >> 1 : i0;
    const int u = g0 / NIT, it0 = g0 & (NIT - 1);
    const int n = u * 64 + p * RPI + ri;
    if (p >= it0 && p < it0 + RG && n < N) {
      if constexpr (PAIR) src.store(n, yv, yu);
      else src.store(n, yv);
    }
  }
}

}  // namespace glq
