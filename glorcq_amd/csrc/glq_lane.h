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
//  * a row of codes is K*bits/8 bytes = LR 16-byte pieces (LR <= 64); lanes
//    are grouped by LRP = LR rounded up to 16, 32 or 64, so one wave
//    iteration covers RPI = 64 / LRP rows, lane l holding piece l % LRP of row
//    l / LRP.  Every load instruction of codes is 64 lanes x 16 bytes of
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

// Geometry of one lane launch (or one role of a launch): every item has N
// rows of K codes; rows are cut into 64-row units of NIT = LRP iterations,
// taken in rounds of PD iterations; wave w of an item runs rounds
// w rpw .. w rpw + rpw - 1 and stores each round's rows at the round's end.
struct LaneGeom {
  int N, K, G, kw, rank;
  int lr;      // 16-byte pieces per code row
  int rounds;  // rounds of PD iterations per item (64-row units x LRP / PD)
  int wpi;     // waves per item
  int rpw;     // rounds per wave (consecutive rounds of one item)
  int items;
};

// Item data of a lane launch.  A source type provides, per item:
//   lora(item)            the low-rank term is present
//   codes/scales/zeros/sv/bias/u(item)   the item's tensors (bias may be null)
//   x8(item, k)           8 halves of the item's activation row at k (k % 8 == 0)
//   load_a(item, j)       a[j] when a is given (not XU)
//   store(item, n, v)     the item's output row n
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
template <class Src, int BITS, bool SYM, int LRP, int NP, int PD, int NSV, bool HASB, bool XU>
__device__ __forceinline__ void lane_run(const Src& src, const LaneGeom& lg, int wv, int wvb,
                                         float* xu_lds) {
  constexpr int C = lane_piece_codes<BITS>();  // codes per piece
  constexpr int RPI = 64 / LRP;                // rows per iteration
  constexpr int NIT = LRP;                     // iterations per 64-row unit
  static_assert(NIT % PD == 0, "ring depth must divide the unit");
  static_assert(NP == 1 || LRP == 64, "several pieces per lane take whole waves per row");
  const int lane = threadIdx.x & 63;
  const int item = wv / lg.wpi;
  if (item >= lg.items) return;  // uniform over the workgroup (XU: wpi is a multiple of 8)
  // rounds rb .. rb + nr - 1 of PD iterations each, [PD R, PD R + PD)
  const int rb = (wv - item * lg.wpi) * lg.rpw;
  const int nr = min(lg.rpw, lg.rounds - rb);
  if (!XU && nr <= 0) return;  // (XU: every wave takes part in forming a)
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
    gq[j] = pc[j] * C / 128;          // the piece's quantization group
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
        const f16x8 in0 = __builtin_bit_cast(f16x8, src.x8(item, pc[j] * C + 16 * blk));
        const f16x8 in1 = __builtin_bit_cast(f16x8, src.x8(item, pc[j] * C + 16 * blk + 8));
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
    }
  };
  if constexpr (!XU) load_x();
  const bool lora = src.lora(item);
  int svo[NSV];  // element offset of the dword within an SV row
#pragma unroll
  for (int k = 0; k < NSV; ++k) {
    const int j = p + k * LRP;  // dword j holds rank columns 2j, 2j + 1
    svo[k] = lora && 2 * j < rank ? 2 * j : 0;
  }

  // Buffer loads: one descriptor per tensor of the item (sized to it, so rows
  // past N read 0 and add 0); a lane's offset is its constant part plus the
  // iteration's first row times the row pitch.  Row of iteration i:
  // (i / NIT) * 64 + (i % NIT) * RPI + ri = RPI i + ri.
  const int rowbytes = kw * 4;
  const auto rc = __builtin_amdgcn_make_buffer_rsrc((void*)src.codes(item), 0, N * rowbytes,
                                                    kBufferFlags);
  const auto rsc = __builtin_amdgcn_make_buffer_rsrc((void*)src.scales(item), 0, N * G * 2,
                                                     kBufferFlags);
  const auto rz = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(SYM ? src.scales(item) : src.zeros(item)), 0, N * G * 2, kBufferFlags);
  // without a low-rank term the SV loads read the codes (finite, times a = 0)
  const auto rsv = __builtin_amdgcn_make_buffer_rsrc(
      lora ? (void*)src.sv(item) : (void*)src.codes(item), 0, lora ? N * rank * 2 : 4,
      kBufferFlags);
  const auto rbi = __builtin_amdgcn_make_buffer_rsrc(HASB ? (void*)src.bias(item) : nullptr, 0,
                                                     HASB ? N * 2 : 0, kBufferFlags);
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
    const int n0 = RPI * (min(rb + r, rlast) * PD + d);  // uniform
    if constexpr (HASB) bw[d] = __builtin_amdgcn_raw_buffer_load_b16(rbi, vb + n0 * 2, 0, 0);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      cw[d][j] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, vc[j] + n0 * rowbytes, 0, kBufferNT));
      sw[d][j] = __builtin_amdgcn_raw_buffer_load_b16(rsc, vs[j] + n0 * G * 2, 0, 0);
      if constexpr (!SYM)
        zw[d][j] = __builtin_amdgcn_raw_buffer_load_b16(rz, vs[j] + n0 * G * 2, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < NSV; ++k)
      vw[d][k] = __builtin_amdgcn_raw_buffer_load_b32(rsv, vsv[k] + n0 * svr * 2, 0, 0);
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
  if constexpr (!XU) prologue();

  // ---- a pairs of this lane's SV dwords (zero past the rank) ----
  uint32_t ap[NSV];
  if constexpr (XU) {
    // a = fp16(x U) in this workgroup (layout in LaneXu)
    const LaneXu L(rank);
    const int t = threadIdx.x;
    float* part = xu_lds;                      // (ks, rank)
    float* segs = xu_lds + L.ks * rank;        // (nseg, rank)
    __half* ah = (__half*)(segs + L.nseg * rank);
    if (lora) {
      const int b = t % L.nb, slot = t / L.nb;
      if (slot < L.ks) {
        const int nch = lg.K / 8;  // 8-row chunks
        const __half* ub = src.u(item) + 8 * b;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        u32x4 u0[8], u1[8], x0, x1;
        auto load = [&](int c, u32x4 (&u)[8], u32x4& xv) {
          c = min(c, nch - 1);  // past the end: re-read the last chunk (not used)
          xv = src.x8(item, 8 * c);
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
        // two chunks in flight: slot, slot + ks, ...; a slot at or past the
        // last chunk adds nothing
        load(slot, u0, x0);
        for (int c = slot; c < nch; c += 2 * L.ks) {
          load(c + L.ks, u1, x1);
          fma_chunk(u0, x0);
          if (c + L.ks >= nch) break;
          load(c + 2 * L.ks, u0, x0);
          fma_chunk(u1, x1);
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
      if (t < rank) {  // level 2: the segments in order
        float sum = 0.f;
        for (int q = 0; q < L.nseg; ++q) sum += segs[q * rank + t];
        ah[t] = __float2half(sum);
      }
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NSV; ++k) {
      const int j = p + k * LRP;
      f16x2 pr = {(_Float16)0.f, (_Float16)0.f};
      if (lora && 2 * j < rank) {
        pr[0] = (_Float16)__half2float(ah[2 * j]);
        pr[1] = (_Float16)__half2float(ah[2 * j + 1]);
      }
      ap[k] = __builtin_bit_cast(uint32_t, pr);
    }
    if (nr <= 0) return;  // a wave with no rows of its own
    load_x();
    prologue();
  } else {
#pragma unroll
    for (int k = 0; k < NSV; ++k) {
      const int j = p + k * LRP;
      f16x2 pr = {(_Float16)0.f, (_Float16)0.f};
      if (lora && 2 * j < rank) {
        pr[0] = (_Float16)__half2float(src.load_a(item, 2 * j));
        pr[1] = (_Float16)__half2float(src.load_a(item, 2 * j + 1));
      }
      ap[k] = __builtin_bit_cast(uint32_t, pr);
    }
  }

  const DecodeConsts dk = DecodeConsts::make();
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  for (int r = 0; r < nr; ++r) {
    const int i0 = (rb + r) * PD;  // first iteration of the round
    float yv = 0.f;
#pragma unroll
    for (int d = 0; d < PD; ++d) {
      const int i = i0 + d;
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
      for (int k = 0; k < NSV; ++k) part = dot2(vw[d][k], ap[k], part);
      __builtin_amdgcn_sched_barrier(0);
      issue(d, r + 1);
      __builtin_amdgcn_sched_barrier(0);
      const float tot = lane_group_sum<LRP>(part);
      yv = p == (i & (NIT - 1)) ? tot : yv;
    }
    // lane l holds row (l % LRP) * RPI + l / LRP of the unit; the lanes of
    // the round's PD iterations store
    const int u = i0 / NIT, it0 = i0 & (NIT - 1);
    const int n = u * 64 + p * RPI + ri;
    if (p >= it0 && p < it0 + PD && n < N) src.store(item, n, yv);
  }
}

// Dense items (glq_gemv.hip): item i at base + i * stride, one token row.
struct DenseLaneSrc {
  const DenseArgs& a;
  __device__ bool lora(int) const { return a.sv != nullptr && a.sh.rank > 0; }
  __device__ const uint32_t* codes(int item) const { return a.codes + (int64_t)item * a.codes_es; }
  __device__ const __half* scales(int item) const { return a.scales + (int64_t)item * a.sz_es; }
  __device__ const __half* zeros(int item) const { return a.zeros + (int64_t)item * a.sz_es; }
  __device__ const __half* sv(int item) const { return a.sv + (int64_t)item * a.sv_es; }
  __device__ const __half* bias(int item) const { return a.bias + (int64_t)item * a.bias_es; }
  __device__ const __half* u(int item) const { return a.u + (int64_t)item * a.u_es; }
  __device__ u32x4 x8(int item, int k) const {
    return *(const u32x4*)(a.x + (int64_t)item * a.x_es + k);
  }
  __device__ __half load_a(int item, int j) const {
    if (a.xu) return a.xu[(int64_t)item * a.xu_es + j];
    const float* pp = a.apart + (int64_t)item * a.P * a.M * a.sh.rpad + j;
    return __float2half(sum_strided(pp, (int64_t)a.M * a.sh.rpad, a.P));
  }
  __device__ void store(int item, int n, float v) const {
    a.y[(int64_t)item * a.y_es + n] = __float2half(v);
  }
};

struct LaneArgs {
  DenseArgs a;
  LaneGeom g;
};

template <int BITS, bool SYM, int LRP, int PD, int NSV, bool HASB, bool XU>
__global__ __launch_bounds__(XU ? 512 : 256) void gemv_lane_kernel(LaneArgs la) {
  extern __shared__ float xu_lds[];
  constexpr int WPB = XU ? 8 : 4;  // waves per workgroup
  const DenseLaneSrc src{la.a};
  const int wvb = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  lane_run<DenseLaneSrc, BITS, SYM, LRP, 1, PD, NSV, HASB, XU>(src, la.g, blockIdx.x * WPB + wvb,
                                                               wvb, xu_lds);
}

}  // namespace glq
