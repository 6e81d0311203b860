// MoE block decode step for a few tokens (glq_moe_decode with tokens <=
// kMoeLaneMaxB): GraphCompatibleMoeBlock.forward (inference/moe_block.py:
// 381-436) on the lane-sliced GEMV of glq_lane.h, one token row per work item.
// The only cross-workgroup handshakes are last-arriver handoffs (glq_handoff.h:
// coherent stores and loads, no fence): a token's router rows over several
// workgroups, and the K slices of the token-tile form.
//
//  1. moe_lane_route_kernel  workgroups per token: router logits (fp32 dot
//                            products rounded to fp16 once), softmax, top-k
//                            (ties to the lower index), optional
//                            renormalisation (moe_block.py:386-392), the
//                            shared-expert gate sigmoid(fp16 logit); the other
//                            workgroups run the shared expert's gate and up
//                            rows in pairs and write its inter = fp16(fp16(
//                            silu(g)) * u) (moe_block.py:465-468); from 4
//                            tokens in the token-tile form (glq_tile16.h)
//  2. moe_lane_xu_kernel     (with LoRA) one workgroup per (pick, gate/up):
//                            a = fp16(x U_c) of the pick's cluster (the
//                            cluster-shared precompute, moe_block.py:290-322)
//  3. moe_lane_gu_kernel     routed gate and up rows of every pick in pairs
//                            (both matrices' row n in one lane group), with
//                            their a SV^T terms, writing the pick's inter
//  4. moe_lane_down_kernel   routed down rows of every pick without the
//                            low-rank term (fp32); rows of more than 64
//                            pieces in K parts of at most 64 (one a lane),
//                            summed in part order at the combine; with LoRA,
//                            workgroups past them form each pick's a_down =
//                            fp16(inter U_down)
//  5. moe_lane_sdown_kernel  the shared expert's down rows, each row's store
//                            combining out = fp16(sum_k w_k (y_k + a_down,k
//                            SV_k^T) + gate * fp16(shared)) (+ the caller's
//                            residual); from 4 tokens
//                            moe_lane_sdown_t16_kernel (token-tile form);
//                            without a shared expert moe_lane_combine_kernel
//                            does the sum alone
//
// The end of the file holds the pieces of a step whose routed experts are
// TurboQuant layers (composed by glorcq_amd/moe_block.py): glq_moe_route (the
// router alone), glq_moe_combine, glq_swiglu.
//
// Only the picked experts' weights are read, a pick's U once.  Every sum has
// a fixed order, so the step gives the same bits on every run; routing and the
// combine's order of terms follow the many-token launches (glq_moe.hip).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "glq_handoff.h"
#include "glq_internal.h"
#include "glq_lane.h"
#include "glq_moe_route.h"
#include "glq_stream.h"
#include "glq_tile16.h"
#include "glq_xstream.h"

namespace glq {

constexpr int kMoeLaneThreads = 512;  // 8 waves (the lane x U form)
constexpr int kMoeLaneWaves = 2048;   // target waves per lane role
constexpr int64_t kMoeLaneXuAllBytes = 12ll << 20;  // all clusters' x U in the router launch
constexpr int64_t kMoeLaneXuAllPairs = 32;          // ... for at most this many (cluster, token)

struct MoeLaneArgs {
  int B, H, E, I, SI, topk, norm, C, rank;
  int urows[3];
  const __half* h;
  const __half* rw;
  const __half* sgw;
  const uint32_t* codes[3];
  const __half* scales[3];
  const __half* zeros[3];
  int64_t c_es[3], s_es[3], sv_es[3];
  const __half* U[3];
  const int32_t* clus[3];
  const int32_t* uslot[2];
  const __half* SV[3];
  const uint32_t* scodes[3];
  const __half* sscales[3];
  const __half* szeros[3];
  // workspace
  int32_t* sel;     // [P] expert of pick p = t * topk + k
  __half* wts;      // [P] routing weights
  __half* sg;       // [B] shared-expert gate
  float* agu;       // fp32 partial sums of a over K slices of kXuSlice codes:
                    // [2][P][S][rank] for each pick's gate and up, or (xuall)
                    // [2][C][B][S][rank] for every cluster's gate and up
  int xuall;        // a for every cluster in the router's launch: 1 by (matrix,
                    // cluster, token, slice) jobs, 2 by (matrix, cluster, slice)
                    // jobs over every token at once (moe_lane_xu_tile); 0: after
                    // routing, per pick
  int su;           // K slices of gate/up (H), and of down (I)
  int sd;
  int kd, kdp;      // routed down: K parts of a row (one lane piece each), codes per part
  __half* inter;    // [P][I] each pick's inter
  float* yb;        // [kd][P][H] routed down outputs per K part, without the low-rank term
  float* ad;        // [P][sd][rank] fp32 partial sums of each pick's a_down
  __half* sinter;   // [B][SI] the shared expert's inter
  int nrw;          // router workgroups per token (each a slice of the router rows)
  __half* lgw;      // [B][E + 1] logits of the sliced router
  unsigned* rcnt;   // [B] router arrival counters (zero between steps)
  // outputs
  __half* out;
  const __half* res;
  __half* logits;
  LaneGeom gSGU, gRGU, gRD, gSD;
  T16Geom gS16, gSD16;  // the shared gate/up and down in the tile form (t16s, t16d)
  int t16s, t16d;
  float* rtd;           // [B][H] routed part of the outputs (t16d)
  int nrd;          // workgroups of the routed down rows
  int rows_wg;      // output rows per shared-down workgroup (its combine)
  // Combine in the routed down launch (fuse): the shared down runs in the
  // gate/up launch (sy = fp16 of its rows), and the last of a (token, row
  // block)'s down workgroups and a_down jobs to arrive on ccnt combines the
  // block's rows.
  int fuse;
  __half* sy;       // [B][H] shared expert outputs
  unsigned* ccnt;   // [B][nrb] arrival counters (zero between steps)
  unsigned* adcnt;  // [B] the token's a_down jobs done (low half) and their readers (high)
  uint64_t spin;    // bound of the combine's wait, ticks of the 100 MHz real-time counter
  int nrb;          // row blocks of an output row (routed down workgroups per item)
  int rows_blk;     // output rows per row block
  int ngu;          // workgroups of the routed gate/up role (fuse: the shared down's follow)
  // Routed experts in the streamed token-tile form (xt, glq_xstream.h): one
  // workgroup set per expert whose token rows are the expert's picks, each
  // code decoded once for all of them; gate/up (pairs, whole K, the low-rank
  // term by MFMA) and down (K slices stored apart in yb, kd = the slices).
  int xt;
  XsGeom gXgu, gXd;
  // (xuall = 2 with xt) a = fp16 of the slices' sums of every (matrix,
  // cluster, token), [2][C][B][rank], formed by the last of a (matrix,
  // cluster)'s tile jobs to arrive on xucnt[m C + c] (zero between steps)
  __half* a16;
  unsigned* xucnt;
};

constexpr int kXuSlice = 512;  // codes per x U job
constexpr int kXuTileStride = 68;  // halves per staged U row (moe_lane_xu_tile): 34 words,
                                   // so the 4 row groups of a column read hit 4 bank groups
constexpr int kXuTileMaxB = 16;    // tokens of a tile job (the MFMA's 16 rows)
constexpr int kXuTileMaxRank = 64;

// Workgroups of the router launch's x U jobs.
__host__ __device__ inline int64_t moe_lane_nxu(int xuall, int C, int B, int su) {
  return xuall == 1 ? 2ll * C * B * su : xuall == 2 ? 2ll * C * su : 0;
}

// Iterations of row loads in flight per wave: gate/up pairs; single rows of
// np pieces a lane (fewer for several pieces, whose x slices hold registers).
#ifndef GLQ_MOE_PAIR_PD
#define GLQ_MOE_PAIR_PD 4
#endif
#ifndef GLQ_MOE_ROW_PD
#define GLQ_MOE_ROW_PD 4
#endif
constexpr int kMoePairPD = GLQ_MOE_PAIR_PD;
constexpr int moe_lane_pd(int np) { return np >= 3 ? 2 : np == 2 ? 4 : GLQ_MOE_ROW_PD; }

__device__ __forceinline__ int moe_lane_clamp(int v, int n) { return min(max(v, 0), n - 1); }

// U row of matrix m (gate 0, up 1, down 2) for expert e.
__device__ __forceinline__ const __half* moe_lane_u(const MoeLaneArgs& a, int m, int e) {
  const int K = m == 2 ? a.I : a.H;
  int row;
  if (m == 2) {
    row = moe_lane_clamp(a.clus[2][e], a.urows[2]);  // the pool row itself
  } else {
    const int c = moe_lane_clamp(a.clus[m][e], a.C);
    row = moe_lane_clamp(a.uslot[m] ? a.uslot[m][c] : c, a.urows[m]);
  }
  return a.U[m] + (int64_t)row * K * a.rank;
}

// ---- item views (glq_lane.h source types) ----
// Routed gate and up of pick p, in pairs; stores the pick's inter.
struct RguItem {
  const MoeLaneArgs& a;
  int p, e;
  const __half* x;
  __device__ bool lora() const { return a.rank > 0 && a.SV[0] != nullptr; }
  __device__ const uint32_t* codes(int m) const { return a.codes[m] + (int64_t)e * a.c_es[m]; }
  __device__ const __half* scales(int m) const { return a.scales[m] + (int64_t)e * a.s_es[m]; }
  __device__ const __half* zeros(int m) const { return a.zeros[m] + (int64_t)e * a.s_es[m]; }
  __device__ const __half* sv(int m) const { return a.SV[m] + (int64_t)e * a.sv_es[m]; }
  __device__ u32x4 x8(int k) const { return *(const u32x4*)(x + k); }
  // a = fp16(sum of the slices' partials, in slice order)
  __device__ const float* a_parts(int m, int j) const {
    const int64_t job = a.xuall ? ((int64_t)m * a.C + moe_lane_clamp(a.clus[m][e], a.C)) * a.B +
                                      p / a.topk
                                : (int64_t)m * a.B * a.topk + p;
    return a.agu + job * a.su * a.rank + j;
  }
  __device__ __half load_a(int m, int j) const {
    return __float2half(sum_strided(a_parts(m, j), a.rank, a.su));
  }
  // the slices' partials, issued before the x slice's wait (glq_lane.h)
  __device__ int a_count() const { return a.su; }
  __device__ void a_issue(int m, int j, float (&v)[kLaneEarlyA]) const {
    const float* pp = a_parts(m, j);
#pragma unroll
    for (int q = 0; q < kLaneEarlyA; ++q) v[q] = q < a.su ? pp[(int64_t)q * a.rank] : 0.f;
  }
  __device__ void store(int n, float g, float u) const {
    a.inter[(int64_t)p * a.I + n] = swiglu_fp16(g, u);
  }
};
struct RguSrc {
  const MoeLaneArgs& a;
  __device__ RguItem bind(int p) const {
    return RguItem{a, p, a.sel[p], a.h + (int64_t)(p / a.topk) * a.H};
  }
};

// Routed down rows of pick p over K part q (codes q kdp .. + kdp of each
// row) without the low-rank term (added at the combine, with the parts).
template <int BITS>
struct RdItem {
  const MoeLaneArgs& a;
  int p, e, q;
  __device__ bool lora() const { return false; }
  __device__ const uint32_t* codes() const {
    return a.codes[2] + (int64_t)e * a.c_es[2] + q * (a.kdp * BITS / 32);
  }
  __device__ const __half* scales() const {
    return a.scales[2] + (int64_t)e * a.s_es[2] + q * (a.kdp / 128);
  }
  __device__ const __half* zeros() const {
    return a.zeros[2] + (int64_t)e * a.s_es[2] + q * (a.kdp / 128);
  }
  __device__ const __half* sv() const { return nullptr; }
  __device__ const __half* bias() const { return nullptr; }
  __device__ const __half* u() const { return nullptr; }
  __device__ u32x4 x8(int k) const {
    return *(const u32x4*)(a.inter + (int64_t)p * a.I + q * a.kdp + k);
  }
  __device__ __half load_a(int) const { return __float2half(0.f); }
  __device__ void store(int n, float v) const {
    float* d = a.yb + ((int64_t)q * a.B * a.topk + p) * a.H + n;
    if (a.fuse) handoff_put(d, v);  // read by this launch's combine
    else *d = v;
  }
};
template <int BITS>
struct RdSrc {
  const MoeLaneArgs& a;
  // item = p kd + q
  __device__ RdItem<BITS> bind(int item) const {
    const int p = item / a.kd;
    return RdItem<BITS>{a, p, a.sel[p], item - p * a.kd};
  }
};

// x U jobs: the input row and U of one (pick, matrix).
struct XuJob {
  const __half* x;
  const __half* uu;
  __device__ const __half* u() const { return uu; }
  __device__ u32x4 x8(int k) const { return *(const u32x4*)(x + k); }
};

// Shared gate and up of token t, in pairs; stores the shared inter.
struct SguItem {
  const MoeLaneArgs& a;
  int t;
  __device__ bool lora() const { return false; }
  __device__ const uint32_t* codes(int m) const { return a.scodes[m]; }
  __device__ const __half* scales(int m) const { return a.sscales[m]; }
  __device__ const __half* zeros(int m) const { return a.szeros[m]; }
  __device__ const __half* sv(int) const { return nullptr; }
  __device__ u32x4 x8(int k) const { return *(const u32x4*)(a.h + (int64_t)t * a.H + k); }
  __device__ __half load_a(int, int) const { return __float2half(0.f); }
  __device__ void store(int n, float g, float u) const {
    a.sinter[(int64_t)t * a.SI + n] = swiglu_fp16(g, u);
  }
};
struct SguSrc {
  const MoeLaneArgs& a;
  __device__ SguItem bind(int t) const { return SguItem{a, t}; }
};

// Shared gate and up of every token at once (glq_tile16.h: one decode of each
// code for all token rows), storing the shared inter.
struct SguTileView {
  const MoeLaneArgs& a;
  __device__ const uint32_t* codes(int m) const { return a.scodes[m]; }
  __device__ const __half* scales(int m) const { return a.sscales[m]; }
  __device__ const __half* zeros(int m) const { return a.szeros[m]; }
  __device__ const __half* xrow(int t) const { return a.h + (int64_t)t * a.H; }
  __device__ void prep(int, int, int) const {}
  __device__ void before_store() const {}
  __device__ void store(int n, int t, float g, float u) const {
    a.sinter[(int64_t)t * a.SI + n] = swiglu_fp16(g, u);
  }
};
struct SguTileSrc {
  const MoeLaneArgs& a;
  __device__ SguTileView bind() const { return SguTileView{a}; }
};
constexpr int kMoeT16MinB = 4;  // tokens from which the shared expert takes the tile form

// ---- routed experts in the streamed token-tile form (glq_xstream.h) ----
// The picks of expert e in pick order, which is token order (a token picks an
// expert once), as the token rows of the tile: lane l loads sel[l] and
// sel[64 + l] (P <= 128) before the expert's codes go out; after them the
// two ballots give every wave the same list.
struct XtPicks {
  int s0, s1;
  int mine;  // pick of the token row this thread stages (row 0's past M)
  int mli;   // pick of token row li (the lane's MFMA A row; row 0's past M)
  int M;
  __device__ void issue(const MoeLaneArgs& a) {
    const int l = threadIdx.x & 63, P = a.B * a.topk;
    s0 = l < P ? a.sel[l] : -1;
    s1 = l + 64 < P ? a.sel[l + 64] : -1;
  }
  // xl[t] = the pick of token row t (LDS; read after a barrier)
  __device__ int resolve(int e, int ts, int li, int* xl) {
    const uint64_t m0 = __builtin_amdgcn_ballot_w64(s0 == e);
    const uint64_t m1 = __builtin_amdgcn_ballot_w64(s1 == e);
    int slot = 0, first = 0, own = -1, ownl = -1;
    for (uint64_t m = m0; m; m &= m - 1, ++slot) {
      const int p = __builtin_ctzll(m);
      if (slot == 0) first = p;
      if (slot == ts) own = p;
      if (slot == li) ownl = p;
    }
    for (uint64_t m = m1; m; m &= m - 1, ++slot) {
      const int p = 64 + __builtin_ctzll(m);
      if (slot == 0) first = p;
      if (slot == ts) own = p;
      if (slot == li) ownl = p;
    }
    M = min(slot, 16);
    mine = own >= 0 ? own : first;
    mli = ownl >= 0 ? ownl : first;
    if ((threadIdx.x & 7) == 0 && threadIdx.x < 128 && ts < M) xl[ts] = mine;
    return M;
  }
};

// Gate and up rows of expert e for its picks, in pairs, each pick's low-rank
// term a SV^T by MFMA (a = fp16 of the sum of its slices' partials, the lane
// form's load_a), storing the picks' inter.  kXguWaves waves, whole rows.
constexpr int kXguWaves = 4;
struct XguView {
  const MoeLaneArgs& a;
  int e;
  __half* al;  // LDS [2][16][rank]: a of each token row
  int* xl;     // LDS [16]
  XtPicks pk;
  __device__ const uint32_t* codes(int m) const { return a.codes[m] + (int64_t)e * a.c_es[m]; }
  __device__ const __half* scales(int m) const { return a.scales[m] + (int64_t)e * a.s_es[m]; }
  __device__ const __half* zeros(int m) const { return a.zeros[m] + (int64_t)e * a.s_es[m]; }
  u32x4 svf[2][2], af[2][2];  // the lane's SV and (a16) a fragments, matrix x MFMA step
  __device__ void issue_meta() { pk.issue(a); }
  __device__ int resolve(int ts, int li) { return pk.resolve(e, ts, li, xl); }
  __device__ const __half* xrow_slot() const { return a.h + (int64_t)(pk.mine / a.topk) * a.H; }
  __device__ bool lora() const { return a.rank > 0 && a.SV[0] != nullptr; }
  // the low-rank term's loads, issued with the first codes: SV of the lane's
  // row (B) and, with a16, a of its token row li (A)
  __device__ void lora_issue(int row, int li, int kb) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int c = 32 * s + 8 * kb;
        svf[m][s] = c < a.rank ? *(const u32x4*)(a.SV[m] + (int64_t)e * a.sv_es[m] +
                                                 (int64_t)row * a.rank + c)
                               : u32x4{0u, 0u, 0u, 0u};
        af[m][s] = u32x4{0u, 0u, 0u, 0u};
        if (a.a16 && li < pk.M && c < a.rank) {
          const int cl = moe_lane_clamp(a.clus[m][e], a.C), t = pk.mli / a.topk;
          af[m][s] = *(const u32x4*)(a.a16 + (((int64_t)m * a.C + cl) * a.B + t) * a.rank + c);
        }
      }
  }
  __device__ f16x8 sv_frag(int m, int s) const { return __builtin_bit_cast(f16x8, svf[m][s]); }
  __device__ f16x8 a_frag(int m, int li, int s, int kb) const {
    if (a.a16) return __builtin_bit_cast(f16x8, af[m][s]);
    const int c = 32 * s + 8 * kb;
    return li < pk.M && c < a.rank ? *(const f16x8*)(al + (m * 16 + li) * a.rank + c) : f16x8{};
  }
  // without a16: a of every (matrix, token row) into al: thread (m, t, j0) =
  // (tid / 128, (tid / 8) % 16, tid % 8) sums columns j0, j0 + 8, ...
  __device__ void prep(int, int) const {
    if (!lora() || a.a16) return;  // uniform
    const int tid = threadIdx.x, m = tid >> 7, t = (tid >> 3) & 15, r = a.rank;
    if (t < pk.M) {
      const int p = pk.mine;
      const int64_t job = a.xuall ? ((int64_t)m * a.C + moe_lane_clamp(a.clus[m][e], a.C)) * a.B +
                                        p / a.topk
                                  : (int64_t)m * a.B * a.topk + p;
      for (int j = tid & 7; j < r; j += 8)
        al[(m * 16 + t) * r + j] = __float2half(sum_strided(a.agu + job * a.su * r + j, r, a.su));
    }
    __syncthreads();
  }
  __device__ void store(int n, int t, float g, float u) const {
    a.inter[(int64_t)xl[t] * a.I + n] = swiglu_fp16(g, u);
  }
};

// Down rows of expert e for its picks over K slice s, stored apart (yb[s]):
// the combine sums the slices in order, then adds a_down SV^T.  All
// kMoeLaneThreads threads (the same launch's a_down jobs need all of them).
struct XdView {
  const MoeLaneArgs& a;
  int e;
  int* xl;
  XtPicks pk;
  __device__ const uint32_t* codes(int) const { return a.codes[2] + (int64_t)e * a.c_es[2]; }
  __device__ const __half* scales(int) const { return a.scales[2] + (int64_t)e * a.s_es[2]; }
  __device__ const __half* zeros(int) const { return a.zeros[2] + (int64_t)e * a.s_es[2]; }
  __device__ void issue_meta() { pk.issue(a); }
  __device__ int resolve(int ts, int li) { return pk.resolve(e, ts, li, xl); }
  __device__ const __half* xrow_slot() const { return a.inter + (int64_t)pk.mine * a.I; }
  __device__ void prep(int, int) const {}
  __device__ void store(int s, int n, int t, float v) const {
    a.yb[((int64_t)s * a.B * a.topk + xl[t]) * a.H + n] = v;
  }
};

// Routed part of output rows [n0, n0 + nrows) of token t into LDS routed[]:
// sum_k w_k (y_k[n] + a_down,k SV_down,k[n]^T), fmaf over the picks in pick
// order (the many-token combine's order), a_down = fp16(sum of its slices'
// partials).  All `nth` threads of the workgroup call it (barriers inside).
// LDS: adl (topk x rank halves), contrib (nrows x topk floats), routed.
// COH: y and the a_down partials were written in this launch (agent-scope
// loads).
// adl_ready: adl already holds the token's a_down values.
template <bool COH = false>
__device__ void moe_lane_routed_rows(const MoeLaneArgs& a, int t, int n0, int nrows, int nth,
                                     __half* adl, float* contrib, float* routed,
                                     bool adl_ready = false) {
  const int tid = threadIdx.x, K = a.topk, r = a.rank;
  const bool lora = r > 0 && a.SV[2] != nullptr;
  if (lora && !adl_ready)
    for (int i = tid; i < K * r; i += nth) {
      const int k = i / r, j = i - k * r;
      const float* pp = a.ad + (int64_t)(t * K + k) * a.sd * r + j;
      adl[i] = __float2half(COH ? sum_strided_coh(pp, r, a.sd) : sum_strided(pp, r, a.sd));
    }
  __syncthreads();
  for (int i = tid; i < nrows * K; i += nth) {
    const int rr = i / K, k = i - rr * K, n = min(n0 + rr, a.H - 1), pk = t * K + k;
    float y = 0.f;
    for (int q = 0; q < a.kd; ++q) {
      const float* yp = a.yb + ((int64_t)q * a.B * K + pk) * a.H + n;
      y += COH ? handoff_get(yp) : *yp;
    }
    if (lora) {
      const __half* sv = a.SV[2] + (int64_t)a.sel[pk] * a.sv_es[2] + (int64_t)n * r;
      const __half* ak = adl + k * r;
      float l = 0.f;
      for (int j = 0; j < r; j += 8) {
        const u32x4 s8 = *(const u32x4*)(sv + j), a8 = *(const u32x4*)(ak + j);
#pragma unroll
        for (int q = 0; q < 4; ++q) l = dot2(s8[q], a8[q], l);
      }
      y += l;
    }
    contrib[i] = y;
  }
  __syncthreads();
  for (int rr = tid; rr < nrows; rr += nth) {
    float acc = 0.f;
    for (int k = 0; k < K; ++k) acc = fmaf(__half2float(a.wts[t * K + k]), contrib[rr * K + k], acc);
    routed[rr] = acc;
  }
  __syncthreads();
}

// Shared down rows of token t, the combine in each row's store; the rows'
// routed parts (from row n0) are formed in LDS while the rows' first loads
// are in flight (after_issue).
struct SdItem {
  const MoeLaneArgs& a;
  int t, n0, nrows;
  __half* adl;
  float* contrib;
  float* routed;
  __device__ void after_issue() const {
    moe_lane_routed_rows(a, t, n0, nrows, kMoeLaneThreads, adl, contrib, routed);
  }
  __device__ bool lora() const { return false; }
  __device__ const uint32_t* codes() const { return a.scodes[2]; }
  __device__ const __half* scales() const { return a.sscales[2]; }
  __device__ const __half* zeros() const { return a.szeros[2]; }
  __device__ const __half* sv() const { return nullptr; }
  __device__ const __half* bias() const { return nullptr; }
  __device__ const __half* u() const { return nullptr; }
  __device__ u32x4 x8(int k) const {
    return *(const u32x4*)(a.sinter + (int64_t)t * a.SI + k);
  }
  __device__ __half load_a(int) const { return __float2half(0.f); }
  // out = fp16(routed + gate * fp16(shared)) (+ residual)
  __device__ void store(int n, float v) const {
    float acc = routed[n - n0];
    acc = fmaf(__half2float(a.sg[t]), __half2float(__float2half(v)), acc);
    float o = __half2float(__float2half(acc));
    if (a.res) o += __half2float(a.res[(int64_t)t * a.H + n]);
    a.out[(int64_t)t * a.H + n] = __float2half(o);
  }
};
// Shared down rows of token t storing sy = fp16 of each row (the combine
// follows in the routed down launch).
struct SdyItem {
  const MoeLaneArgs& a;
  int t;
  __device__ bool lora() const { return false; }
  __device__ const uint32_t* codes() const { return a.scodes[2]; }
  __device__ const __half* scales() const { return a.sscales[2]; }
  __device__ const __half* zeros() const { return a.szeros[2]; }
  __device__ const __half* sv() const { return nullptr; }
  __device__ const __half* bias() const { return nullptr; }
  __device__ const __half* u() const { return nullptr; }
  __device__ u32x4 x8(int k) const {
    return *(const u32x4*)(a.sinter + (int64_t)t * a.SI + k);
  }
  __device__ __half load_a(int) const { return __float2half(0.f); }
  __device__ void store(int n, float v) const { a.sy[(int64_t)t * a.H + n] = __float2half(v); }
};
struct SdySrc {
  const MoeLaneArgs& a;
  __device__ SdyItem bind(int t) const { return SdyItem{a, t}; }
};

struct SdSrc {
  const MoeLaneArgs& a;
  int n0, nrows;
  __half* adl;
  float* contrib;
  float* routed;
  __device__ SdItem bind(int t) const { return SdItem{a, t, n0, nrows, adl, contrib, routed}; }
};

// Shared down rows of every token in the token-tile form.  Before it
// publishes its block, K slice s of row block rb forms the routed part of the
// block's rows for tokens s, s + ks, ... (the sums of moe_lane_routed_rows, in
// its order: a_down = fp16(sum of its slices' partials) into LDS, each pick's
// y (K parts in order) + a_down SV^T, then the picks in pick order) into
// rtd[t][n]; the finishing workgroup's store combines as SdItem's.
struct SdTileView {
  const MoeLaneArgs& a;
  __half* adl;     // LDS [P][rank]
  float* contrib;  // LDS [tokens of the slice][64][topk]
  __device__ const uint32_t* codes(int) const { return a.scodes[2]; }
  __device__ const __half* scales(int) const { return a.sscales[2]; }
  __device__ const __half* zeros(int) const { return a.szeros[2]; }
  __device__ const __half* xrow(int t) const { return a.sinter + (int64_t)t * a.SI; }
  __device__ void prep(int rb, int s, int ks) const {
    const int tid = threadIdx.x, K = a.topk, r = a.rank, n0 = kT16Rows * rb;
    const bool lora = r > 0 && a.SV[2] != nullptr;
    const int nt = (a.B - s + ks - 1) / ks;  // tokens s, s + ks, ...
    if (lora)
      for (int i = tid; i < nt * K * r; i += kMoeLaneThreads) {
        const int tk = i / r, j = i - tk * r, pk = (s + ks * (tk / K)) * K + tk % K;
        adl[pk * r + j] = __float2half(sum_strided(a.ad + (int64_t)pk * a.sd * r + j, r, a.sd));
      }
    __syncthreads();
    for (int i = tid; i < nt * kT16Rows * K; i += kMoeLaneThreads) {
      const int k = i % K, tr = i / K, t = s + ks * (tr / kT16Rows);
      const int n = min(n0 + tr % kT16Rows, a.H - 1), pk = t * K + k;
      float y = 0.f;
      for (int q = 0; q < a.kd; ++q) y += a.yb[((int64_t)q * a.B * K + pk) * a.H + n];
      if (lora) {
        const __half* sv = a.SV[2] + (int64_t)a.sel[pk] * a.sv_es[2] + (int64_t)n * r;
        const __half* ak = adl + pk * r;
        float l = 0.f;
        for (int j = 0; j < r; j += 8) {
          const u32x4 s8 = *(const u32x4*)(sv + j), a8 = *(const u32x4*)(ak + j);
#pragma unroll
          for (int q = 0; q < 4; ++q) l = dot2(s8[q], a8[q], l);
        }
        y += l;
      }
      contrib[i] = y;
    }
    __syncthreads();
    for (int tr = tid; tr < nt * kT16Rows; tr += kMoeLaneThreads) {
      const int t = s + ks * (tr / kT16Rows), n = n0 + tr % kT16Rows;
      float acc = 0.f;
      for (int k = 0; k < K; ++k)
        acc = fmaf(__half2float(a.wts[t * K + k]), contrib[tr * K + k], acc);
      if (n < a.H) handoff_put(a.rtd + (int64_t)t * a.H + n, acc);
    }
  }
  __device__ void before_store() const {}
  // out = fp16(routed + gate * fp16(shared)) (+ residual)
  __device__ void store(int n, int t, float v) const {
    float acc = handoff_get(a.rtd + (int64_t)t * a.H + n);
    acc = fmaf(__half2float(a.sg[t]), __half2float(__float2half(v)), acc);
    float o = __half2float(__float2half(acc));
    if (a.res) o += __half2float(a.res[(int64_t)t * a.H + n]);
    a.out[(int64_t)t * a.H + n] = __float2half(o);
  }
};
struct SdTileSrc {
  SdTileView v;
  __device__ SdTileView bind() const { return v; }
};

// ---- router: a.nrw workgroups per token ----
// Logits of the E router rows (+ the shared-expert gate row) as fp32 dot
// products over the lanes (16-byte loads, v_dot2), each rounded to fp16 once;
// a wave loads RB rows at once (RC 8-half chunks a lane each), workgroup q
// of the token the rows of pass q (8 RB rows).  With several workgroups each
// publishes its logits and counts itself in; the last (acquiring them) routes
// the token and leaves the counter at zero for the next step.  The routing is
// moe_topk_ranks' (glq_moe.hip) for this one token: thread e ranks expert e
// by counting the keys above its own, wave 0 forms the softmax sum (a
// cross-lane sum in the same order) and the weights.
template <int RC>
__device__ void moe_lane_router(const MoeLaneArgs& a, int t, int q, unsigned char* smem) {
  constexpr int RB = RC >= 8 ? 2 : 16 / RC;  // rows per wave per pass
  uint16_t* lgh = (uint16_t*)smem;                                    // [E + 1] fp16 logits
  uint32_t* keys = (uint32_t*)(smem + ((2 * (a.E + 1) + 15) & ~15));  // [E]
  int* sl = (int*)(keys + a.E);                                       // [topk]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nrow = a.E + (a.sgw ? 1 : 0);
  const __half* hx = a.h + (int64_t)t * a.H;
  u32x4 hv[RC];
#pragma unroll
  for (int j = 0; j < RC; ++j) {
    const int k = 8 * lane + 512 * j;
    hv[j] = k < a.H ? *(const u32x4*)(hx + k) : u32x4{0u, 0u, 0u, 0u};
  }
  const int rend = a.nrw > 1 ? min(nrow, 8 * RB * (q + 1)) : nrow;
  for (int r0 = 8 * RB * q + RB * wave; r0 < rend; r0 += 8 * RB) {
    u32x4 v[RB][RC];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int r = min(r0 + i, nrow - 1);
      const __half* w = r < a.E ? a.rw + (int64_t)r * a.H : a.sgw;
#pragma unroll
      for (int j = 0; j < RC; ++j) {
        const int k = 8 * lane + 512 * j;
        v[i][j] = k < a.H ? *(const u32x4*)(w + k) : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < RC; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) sacc = dot2(v[i][j][c], hv[j][c], sacc);
      sacc = lane_group_sum<64>(sacc);
      if (lane == 0 && r0 + i < rend) {
        const __half lg = __float2half(sacc);
        lgh[r0 + i] = __half_as_ushort(lg);
        if (a.nrw > 1) handoff_put((uint16_t*)a.lgw + (int64_t)t * (a.E + 1) + r0 + i, __half_as_ushort(lg));
      }
    }
  }
  if (a.nrw > 1) {
    // arrival (glq_handoff.h); the last workgroup reads every slice's logits
    __shared__ int last;
    if (!handoff_arrive(a.rcnt + t, (unsigned)a.nrw, &last)) return;
    for (int r = tid; r < nrow; r += kMoeLaneThreads)
      lgh[r] = handoff_get((const uint16_t*)a.lgw + (int64_t)t * (a.E + 1) + r);
    if (tid == 0) handoff_reset(a.rcnt + t);
  }
  __syncthreads();
  for (int e = tid; e < a.E; e += kMoeLaneThreads) {
    keys[e] = moe_key(lgh[e], e);
    if (a.logits) a.logits[(int64_t)t * a.E + e] = __ushort_as_half(lgh[e]);
  }
  if (tid == 0)
    a.sg[t] = a.sgw ? __float2half(1.f / (1.f + expf(-__half2float(__ushort_as_half(lgh[a.E])))))
                    : __float2half(1.f);
  __syncthreads();
  for (int e = tid; e < a.E; e += kMoeLaneThreads) {
    const uint32_t ke = keys[e];
    int r = 0;
    for (int j = 0; j < a.E; ++j) r += (int)(keys[j] > ke);
    if (r < a.topk) sl[r] = e;
  }
  __syncthreads();
  if (wave == 0) {
    const float mx = moe_key_logit(keys[sl[0]]);
    float sum = 0.f;
    for (int e = lane; e < a.E; e += 64) sum += expf(moe_key_logit(keys[e]) - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    const int e = lane < a.topk ? sl[lane] : 0;
    const float w = lane < a.topk ? expf(moe_key_logit(keys[e]) - mx) / sum : 0.f;
    float ws = 0.f;
    if (a.norm)
      for (int j = 0; j < a.topk; ++j) ws += __shfl(w, j);
    if (lane < a.topk) {
      a.sel[t * a.topk + lane] = e;
      a.wts[t * a.topk + lane] = __float2half(a.norm ? w / ws : w);
    }
  }
}

// ---- x U of every token for one (matrix, cluster, K slice) by MFMA ----
// job = (m C + c) su + s.  A = x (token rows, 16-byte loads), B = U: wave w
// stages its 64 rows of the slice in LDS in two halves of 32 (row stride
// kXuTileStride halves) and reads each B operand down the columns; the 8
// waves' 16 x rank partial tiles are summed in LDS in wave order and written
// as the slice partial of every token, the layout of the (cluster, token)
// jobs (agu[((m C + c) B + t) su + s][j]).  LDS: 8 x 32 x kXuTileStride
// halves, then 8 x 4 x 256 floats.  All 512 threads call it.
__device__ void moe_lane_xu_tile(const MoeLaneArgs& a, int job, unsigned char* smem) {
  const int s = job % a.su, mc = job / a.su, m = mc / a.C, c = mc - m * a.C;
  const int row = moe_lane_clamp(a.uslot[m] ? a.uslot[m][c] : c, a.urows[m]);
  const __half* u = a.U[m] + (int64_t)row * a.H * a.rank;
  const int r = a.rank, r8 = r / 8, nct = (r + 15) / 16;
  const int k0 = s * kXuSlice, kn = min(kXuSlice, a.H - k0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, kb = lane >> 4;
  __half* ul = (__half*)smem + wave * 32 * kXuTileStride;
  f32x4 acc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int h2 = 0; h2 < 2; ++h2) {
    const int kr = 64 * wave + 32 * h2;  // slice row of the half's first row
    // U rows [kr, kr + 32) of the slice (rows past H re-read row H - 1: they
    // meet x = 0), 16-byte global loads, 8-byte LDS stores
    for (int i = lane; i < 32 * r8; i += 64) {
      const int rr = i / r8, pc = i - rr * r8;
      const int k = min(k0 + kr + rr, a.H - 1);
      const u32x4 v = *(const u32x4*)(u + (int64_t)k * r + 8 * pc);
      uint2* d = (uint2*)(ul + rr * kXuTileStride + 8 * pc);
      d[0] = uint2{v.x, v.y};
      d[1] = uint2{v.z, v.w};
    }
    const int kk = kr + 8 * kb;
    const f16x8 xv = (li < a.B && kk < kn) ? *(const f16x8*)(a.h + (int64_t)li * a.H + k0 + kk)
                                           : f16x8{};
    // the wave's LDS stores precede its reads (LDS ops of a wave run in order)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      if (ct >= nct) break;  // uniform
      const int col = ct * 16 + li;
      f16x8 bv;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        bv[j] = col < r ? (_Float16)__half2float(ul[(8 * kb + j) * kXuTileStride + col])
                        : (_Float16)0.f;
      acc[ct] = mfma_16x16x32(xv, bv, acc[ct]);
    }
  }
  __syncthreads();  // every wave is past its staging: the LDS becomes the reduction area
  float* red = (float*)smem;  // [wave][ct][i][lane]
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * 4 + ct) * 4 + i) * 64 + lane] = acc[ct][i];
  __syncthreads();
  for (int e = tid; e < nct * 256; e += kMoeLaneThreads) {
    const int ct = e >> 8, i = (e >> 6) & 3, l = e & 63;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) v += red[((w * 4 + ct) * 4 + i) * 64 + l];
    const int t = 4 * (l >> 4) + i, col = ct * 16 + (l & 15);  // D: token row, rank column
    if (t < a.B && col < r) {
      float* d = a.agu + ((((int64_t)m * a.C + c) * a.B + t) * a.su + s) * r + col;
      if (a.a16) handoff_put(d, v);
      else *d = v;
    }
  }
  if (!a.a16) return;
  // the last slice job of (matrix, cluster) to arrive: a = fp16 of the slices'
  // sums in slice order (the lane form's load_a), for every token
  __shared__ int last;
  if (!handoff_arrive(a.xucnt + mc, (unsigned)a.su, &last)) return;
  for (int e = tid; e < a.B * r; e += kMoeLaneThreads) {
    const int t = e / r, j = e - t * r;
    const float* pp = a.agu + (((int64_t)mc * a.B + t) * a.su) * r + j;
    a.a16[((int64_t)mc * a.B + t) * r + j] = __float2half(sum_strided_coh(pp, r, a.su));
  }
  if (tid == 0) handoff_reset(a.xucnt + mc);
}

// ---- kernels ----
__device__ __forceinline__ int moe_lane_wave() {
  return (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Workgroups [0, B): the router of each token; then (xuall) one per (matrix,
// cluster, token) forming a = fp16(h_t U_c); then the shared expert's
// gate/up rows.
template <int SBITS, int SLRP, int RC, bool T16>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_route_kernel(MoeLaneArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  int b = blockIdx.x;
  if (b < a.B * a.nrw) {
    moe_lane_router<RC>(a, b / a.nrw, b % a.nrw, smem);
    return;
  }
  b -= a.B * a.nrw;
  const int nxu = (int)moe_lane_nxu(a.xuall, a.C, a.B, a.su);
  if (a.xuall == 2 && b < nxu) {
    moe_lane_xu_tile(a, b, smem);
    return;
  }
  if (b < nxu) {  // job b = ((m C + c) B + t) su + s
    const int s = b % a.su, mct = b / a.su, t = mct % a.B, mc = mct / a.B;
    const int m = mc / a.C, c = mc - m * a.C;
    const int row = moe_lane_clamp(a.uslot[m] ? a.uslot[m][c] : c, a.urows[m]);
    const __half* u = a.U[m] + (int64_t)row * a.H * a.rank;
    const int k0 = s * kXuSlice;
    const float* sums = lane_xu_sum(XuJob{a.h + (int64_t)t * a.H, u}, k0,
                                    min(kXuSlice, a.H - k0), a.rank, (float*)smem);
    if ((int)threadIdx.x < a.rank) a.agu[(int64_t)b * a.rank + threadIdx.x] = sums[threadIdx.x];
    return;
  }
  b -= nxu;
  if constexpr (T16) {
    t16_run<SguTileSrc, true>(SguTileSrc{a}, a.gS16, b, (float*)smem);
  } else if constexpr (SBITS != 0) {
    const int wvb = moe_lane_wave();
    lane_run<SguSrc, SBITS, false, SLRP, 1, kMoePairPD, 1, false, false, true>(SguSrc{a}, a.gSGU,
                                                                     b * 8 + wvb, wvb, nullptr);
  }
}

// Partial a of (pick, gate/up, K slice) job b = (m P + p) su + s.
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_xu_kernel(MoeLaneArgs a) {
  extern __shared__ float lds[];
  const int P = a.B * a.topk, b = blockIdx.x, s = b % a.su, j = b / a.su;
  const int m = j >= P ? 1 : 0, p = j - m * P;
  const XuJob job{a.h + (int64_t)(p / a.topk) * a.H, moe_lane_u(a, m, a.sel[p])};
  const int k0 = s * kXuSlice;
  const float* sums = lane_xu_sum(job, k0, min(kXuSlice, a.H - k0), a.rank, lds);
  if ((int)threadIdx.x < a.rank) a.agu[(int64_t)b * a.rank + threadIdx.x] = sums[threadIdx.x];
}

template <int BITS, int LRP, int NSV>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_gu_kernel(MoeLaneArgs a) {
  const int wvb = moe_lane_wave();
  lane_run<RguSrc, BITS, false, LRP, 1, kMoePairPD, NSV, false, false, true>(
      RguSrc{a}, a.gRGU, blockIdx.x * 8 + wvb, wvb, nullptr);
}


// The routed gate/up role, then (fuse, with a shared expert) the shared
// down's rows storing sy.
template <int BITS, int LRP, int NSV, int SBITS, int SLRP, int SNP>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_gu_sd_kernel(MoeLaneArgs a) {
  const int wvb = moe_lane_wave();
  if ((int)blockIdx.x < a.ngu) {
    lane_run<RguSrc, BITS, false, LRP, 1, kMoePairPD, NSV, false, false, true>(
        RguSrc{a}, a.gRGU, blockIdx.x * 8 + wvb, wvb, nullptr);
    return;
  }
  const int b = blockIdx.x - a.ngu;
  lane_run<SdySrc, SBITS, false, SLRP, SNP, moe_lane_pd(SNP), 1, false, false>(
      SdySrc{a}, a.gSD, b * 8 + wvb, wvb, nullptr);
}

// a_down of token t's picks formed here, slice by slice in the a_down jobs'
// order (the same bits as their handed-over partials), into adl.  Every
// thread calls it.
__device__ void moe_lane_local_adown(const MoeLaneArgs& a, int t, __half* adl, float* xu) {
  for (int k = 0; k < a.topk; ++k) {
    const int pk = t * a.topk + k;
    const XuJob job{a.inter + (int64_t)pk * a.I, moe_lane_u(a, 2, a.sel[pk])};
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // sum_strided's batches of 8
    float tot = 0.f;
    for (int q = 0; q < a.sd; ++q) {
      const int k0 = q * kXuSlice;
      const float* sums = lane_xu_sum(job, k0, min(kXuSlice, a.I - k0), a.rank, xu);
      if ((int)threadIdx.x < a.rank) acc[q & 7] = sums[threadIdx.x];
      __syncthreads();  // the next slice's partials overwrite the sums
      if ((q & 7) == 7 || q == a.sd - 1) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          tot += (u <= (q & 7)) ? acc[u] : 0.f;
          acc[u] = 0.f;
        }
      }
    }
    if ((int)threadIdx.x < a.rank) adl[k * a.rank + threadIdx.x] = __float2half(tot);
  }
  __syncthreads();
}

// Rows of row block rb of token t: out = fp16(routed + gate * sy) (+ the
// residual), or fp16(routed) without a shared expert -- the arithmetic of
// SdItem::store and moe_lane_combine_kernel.  Every thread calls it.  With
// LoRA it first waits (bounded) for the token's a_down jobs; a wait that
// outlasts kMoeSpinTicks forms a_down itself (the same bits).
constexpr uint64_t kMoeSpinTicks = 100000;  // 1 ms of the 100 MHz real-time counter
constexpr int kMoeFuseWork = 256;  // output rows x picks of one fused combine, at most
__device__ void moe_lane_block_combine(const MoeLaneArgs& a, int t, int rb, float* lds,
                                       int* flag) {
  const int n0 = rb * a.rows_blk, nrows = min(a.rows_blk, a.H - n0);
  const bool lora = a.rank > 0 && a.SV[2] != nullptr;
  __half* adl = (__half*)lds;
  float* contrib = lds + (a.topk * a.rank + 1) / 2;
  float* routed = contrib + a.rows_blk * a.topk;
  bool ready = false;
  if (lora) {
    const unsigned need = (unsigned)(a.topk * a.sd);
    if (threadIdx.x == 0) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      int ok = 0;
      while (true) {
        if ((handoff_get(a.adcnt + t) & 0xffffu) >= need) {
          ok = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.spin) break;
        __builtin_amdgcn_s_sleep(2);
      }
      *flag = ok;
    }
    __syncthreads();
    if (!*flag) {  // (uniform)
      moe_lane_local_adown(a, t, adl, routed + a.rows_blk);
      ready = true;
    }
  }
  moe_lane_routed_rows<true>(a, t, n0, nrows, kMoeLaneThreads, adl, contrib, routed, ready);
  if (lora && threadIdx.x == 0) {  // this block's reader is done with the a_down partials
    const unsigned fin = ((unsigned)a.nrb << 16) | (unsigned)(a.topk * a.sd);
    const unsigned old = __hip_atomic_fetch_add(a.adcnt + t, 1u << 16, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (old + (1u << 16) == fin) handoff_reset(a.adcnt + t);
  }
  for (int r = threadIdx.x; r < nrows; r += kMoeLaneThreads) {
    const int n = n0 + r;
    float acc = routed[r];
    if (a.SI > 0)
      acc = fmaf(__half2float(a.sg[t]), __half2float(a.sy[(int64_t)t * a.H + n]), acc);
    float o = __half2float(__float2half(acc));
    if (a.res) o += __half2float(a.res[(int64_t)t * a.H + n]);
    a.out[(int64_t)t * a.H + n] = __float2half(o);
  }
}

// Partial a_down of job b = p sd + s: the sums of pick p's inter slice s
// against its down U rows (LDS; thread j < rank holds column j).
__device__ const float* moe_lane_adown_part(const MoeLaneArgs& a, int b, float* lds) {
  const int s = b % a.sd, p = b / a.sd;
  const XuJob job{a.inter + (int64_t)p * a.I, moe_lane_u(a, 2, a.sel[p])};
  const int k0 = s * kXuSlice;
  return lane_xu_sum(job, k0, min(kXuSlice, a.I - k0), a.rank, lds);
}

// Workgroups [0, nad): the a_down jobs (LoRA), job b = p sd + s; then the
// routed down rows.  fuse: a job hands its partial over and counts itself
// on its token; a down workgroup counts itself on its (token, row block), and
// the last of the block's down workgroups combines the block.  The jobs come
// first in the grid, so a combine waits only on workgroups dispatched before
// its own.
template <int BITS, int LRP, int NP>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_down_kernel(MoeLaneArgs a) {
  extern __shared__ float lds[];
  __shared__ int flag;
  const int nad = a.rank > 0 && a.SV[2] != nullptr ? a.B * a.topk * a.sd : 0;
  if ((int)blockIdx.x < nad) {  // partial a_down of (pick, K slice)
    const int b = blockIdx.x, p = b / a.sd;
    const float* sums = moe_lane_adown_part(a, b, lds);
    if ((int)threadIdx.x < a.rank) {
      float* d = a.ad + (int64_t)b * a.rank + threadIdx.x;
      if (a.fuse) handoff_put(d, sums[threadIdx.x]);
      else *d = sums[threadIdx.x];
    }
    if (a.fuse) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(a.adcnt + p / a.topk, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  const int db = blockIdx.x - nad;
  const int wvb = moe_lane_wave();
  lane_run<RdSrc<BITS>, BITS, false, LRP, NP, moe_lane_pd(NP), 1, false, false>(
      RdSrc<BITS>{a}, a.gRD, db * 8 + wvb, wvb, nullptr);
  if (!a.fuse) return;
  // the workgroup's rows: row block rb of item i = p kd + q (whole workgroups
  // per item); the block's last down workgroup combines it
  const int wgi = a.gRD.wpi / 8, i = db / wgi, rb = db - i * wgi;
  const int t = i / a.kd / a.topk;
  if (handoff_arrive(a.ccnt + t * a.nrb + rb, (unsigned)(a.topk * a.kd), &flag)) {
    moe_lane_block_combine(a, t, rb, lds, &flag);
    if (threadIdx.x == 0) handoff_reset(a.ccnt + t * a.nrb + rb);
  }
}

// Routed gate/up in the streamed token-tile form: workgroup (e, row block) of
// every expert (an expert no token picked leaves at once), whole rows.
constexpr int kXsChunk = 4;  // groups of an x chunk and of a code ring slot
constexpr int kXdWaves = kMoeLaneThreads / 64;
__global__ __launch_bounds__(kXguWaves * 64) void moe_lane_gu_xt_kernel(MoeLaneArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int xl[16];
  const int e = blockIdx.x / a.gXgu.RB, rb = blockIdx.x - e * a.gXgu.RB;
  unsigned char* sm = (unsigned char*)lds;  // x chunks, transposition areas, a
  XguView v{a, e, (__half*)(sm + xs_lds_bytes(kXsChunk) + xs_tr_bytes(kXguWaves)), xl, {}};
  xs_run<XguView, true, true, false, kXguWaves, kXsChunk, 2>(
      v, a.gXgu, rb, 0, (__half*)sm, (uint32_t*)(sm + xs_lds_bytes(kXsChunk)));
}

// Routed down in the streamed token-tile form: workgroup (e, row block, K
// slice) of every expert, each slice stored apart, then the a_down jobs (as
// moe_lane_down_kernel's).
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_down_xt_kernel(MoeLaneArgs a) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int xl[16];
  const int per = a.gXd.RB * a.gXd.ks, ntile = a.E * per;
  if ((int)blockIdx.x >= ntile) {  // the a_down jobs last: they fill the tiles' last round
    const int j = blockIdx.x - ntile;
    const float* sums = moe_lane_adown_part(a, j, lds);
    if ((int)threadIdx.x < a.rank) a.ad[(int64_t)j * a.rank + threadIdx.x] = sums[threadIdx.x];
    return;
  }
  const int b = blockIdx.x, e = b / per;
  const int rb = (b - e * per) / a.gXd.ks, sl = (b - e * per) - rb * a.gXd.ks;
  XdView v{a, e, xl, {}};
  unsigned char* sm = (unsigned char*)lds;  // x chunks, transposition areas
  xs_run<XdView, false, false, true, kXdWaves, kXsChunk, 3>(
      v, a.gXd, rb, sl, (__half*)sm, (uint32_t*)(sm + xs_lds_bytes(kXsChunk)));
}

// Each workgroup holds one token's rows (wpi a multiple of 8): first the
// routed parts of its output rows, then its shared-down rows, whose stores
// combine.
template <int SBITS, int SLRP, int SNP>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_sdown_kernel(MoeLaneArgs a) {
  extern __shared__ float lds[];
  constexpr int RPI = 64 / SLRP, PD = moe_lane_pd(SNP);
  const LaneGeom& g = a.gSD;
  const int wv0 = blockIdx.x * 8, t = wv0 / g.wpi;
  if (t >= g.items) return;  // uniform over the workgroup
  const int n0 = RPI * PD * (wv0 - t * g.wpi) * g.rpw;
  const int nrows = min(a.rows_wg, a.H - n0);
  if (nrows <= 0) return;
  __half* adl = (__half*)lds;                          // topk x rank
  float* contrib = lds + (a.topk * a.rank + 1) / 2;    // rows_wg x topk
  float* routed = contrib + a.rows_wg * a.topk;        // rows_wg
  const int wvb = moe_lane_wave();
  lane_run<SdSrc, SBITS, false, SLRP, SNP, PD, 1, false, false>(
      SdSrc{a, n0, nrows, adl, contrib, routed}, g, wv0 + wvb, wvb, nullptr);
}

// The shared down and combine in the token-tile form (4-bit shared codes).
// LDS: the tile form's partial blocks, then adl and contrib.
__global__ __launch_bounds__(kMoeLaneThreads) void moe_lane_sdown_t16_kernel(MoeLaneArgs a) {
  extern __shared__ __align__(16) float lds[];
  __half* adl = (__half*)(lds + t16_lds_bytes(false) / 4);
  float* contrib = lds + t16_lds_bytes(false) / 4 + (a.B * a.topk * a.rank + 7) / 8 * 4;
  t16_run<SdTileSrc, false>(SdTileSrc{SdTileView{a, adl, contrib}}, a.gSD16, blockIdx.x, lds);
}

// Without a shared expert: out = fp16(routed) (+ residual), 256 threads a
// workgroup, rows_wg rows of one token each.
__global__ __launch_bounds__(256) void moe_lane_combine_kernel(MoeLaneArgs a) {
  extern __shared__ float lds[];
  const int nb = (a.H + a.rows_wg - 1) / a.rows_wg;
  const int t = blockIdx.x / nb, n0 = (blockIdx.x - t * nb) * a.rows_wg;
  const int nrows = min(a.rows_wg, a.H - n0);
  __half* adl = (__half*)lds;
  float* contrib = lds + (a.topk * a.rank + 1) / 2;
  float* routed = contrib + a.rows_wg * a.topk;
  moe_lane_routed_rows(a, t, n0, nrows, 256, adl, contrib, routed);
  for (int r = threadIdx.x; r < nrows; r += 256) {
    const int n = n0 + r;
    float o = __half2float(__float2half(routed[r]));
    if (a.res) o += __half2float(a.res[(int64_t)t * a.H + n]);
    a.out[(int64_t)t * a.H + n] = __float2half(o);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

int lane_lrp(int lr) { return lr <= 16 ? 16 : lr <= 32 ? 32 : 64; }

// Geometry of a lane role: N rows of K codes per item (pairs: N rows of each
// of two matrices), about kMoeLaneWaves waves over the role.
LaneGeom role_geom(int N, int K, int bits, int rank, int items, bool pair,
                   bool whole_wgs = false) {
  LaneGeom g;
  g.N = N;
  g.K = K;
  g.G = K / 128;
  g.group = 128;
  g.zoff = 0.f;
  g.kw = K * bits / 32;
  g.rank = rank;
  g.items = items;
  g.lr = K * bits / 128;
  const int lrp = lane_lrp(g.lr), np = (g.lr + 63) / 64;
  const int pd = pair ? kMoePairPD : moe_lane_pd(np);
  g.rounds = (N + 63) / 64 * lrp * (pair ? 2 : 1) / pd;
  const int64_t total = (int64_t)items * g.rounds;
  int64_t waves = kMoeLaneWaves;
  if (const char* e = getenv("GLQ_MOE_LANE_WAVES")) waves = std::max(1, atoi(e));
  const int64_t rpw = std::max<int64_t>(1, (total + waves - 1) / waves);
  g.wpi = (int)((g.rounds + rpw - 1) / rpw);
  if (whole_wgs) g.wpi = (g.wpi + 7) / 8 * 8;  // each workgroup within one item
  g.rpw = (g.rounds + g.wpi - 1) / g.wpi;
  return g;
}

int64_t role_blocks(const LaneGeom& g) { return ((int64_t)g.items * g.wpi + 7) / 8; }

// Token-tile role of N rows of K 4-bit codes for M tokens (glq_tile16.h);
// part and cnt are set with the workspace.
T16Geom t16_geom(int N, int K, int M) {
  T16Geom t{};
  t.N = N;
  t.K = K;
  t.G = K / 128;
  t.kw = K / 8;
  t.M = M;
  t.RB = (N + kT16Rows - 1) / kT16Rows;
  t.ks = (t.G + kT16Waves - 1) / kT16Waves;
  return t;
}
int64_t t16_wgs(const T16Geom& t) { return (int64_t)t.RB * t.ks; }

// Streamed token-tile role of one expert's N rows of K 2-bit codes, row
// blocks of `rows`, ks K slices.
XsGeom xs_geom(int N, int K, int rows, int ks) {
  XsGeom t{};
  t.N = N;
  t.K = K;
  t.G = K / 128;
  t.kw = K / 16;
  t.RB = (N + rows - 1) / rows;
  t.ks = ks;
  t.kg = (t.G + ks - 1) / ks;
  return t;
}

struct MoeLanePlan {
  MoeLaneArgs a;
  int bits, sbits, rc;
  bool lora;
  int64_t off_sel, off_wts, off_sg, off_lgw, off_agu, off_inter, off_yb, off_ad, off_sinter,
      off_t16p, off_rtd, off_sy, off_a16, ws_need;
  size_t lds_route, lds_xu, lds_xut, lds_comb, lds_sd16, lds_down, lds_xgu, lds_xd;
};

}  // namespace

// The lane path takes the step when the batch is small and every projection
// fits its form (gate/up rows of at most 64 pieces, down rows of at most 256,
// H <= 4096).  p has passed the many-token path's checks (moe_plan).
static bool moe_lane_plan(const glq_moe_params* p, MoeLanePlan& P) {
  int maxb = kMoeLaneMaxB;
  if (const char* e = getenv("GLQ_MOE_LANE_MAXB")) maxb = atoi(e);
  if (getenv("GLQ_MOE_NO_LANE")) return false;
  const int64_t B = p->tokens, H = p->hidden, I = p->inter, SI = p->shared_inter;
  if (B > maxb) return false;
  const bool lora = p->rank > 0 && p->SV[0] && p->SV[1] && p->SV[2];
  const int r = lora ? (int)p->rank : 0;
  const int bits = p->bits, sbits = SI > 0 ? p->shared_bits : 0;
  if (H * bits / 128 > 64 || I * bits / 128 > 256 || H > 4096) return false;
  if (SI > 0 && (H * sbits / 128 > 64 || SI * sbits / 128 > 256)) return false;
  MoeLaneArgs& a = P.a;
  memset(&a, 0, sizeof(a));
  a.B = (int)B; a.H = (int)H; a.E = (int)p->experts; a.I = (int)I; a.SI = (int)SI;
  a.topk = (int)p->top_k;
  a.norm = p->norm_topk_prob ? 1 : 0;
  a.C = lora ? (int)p->n_clusters : 1;
  a.rank = r;
  a.h = (const __half*)p->h;
  a.rw = (const __half*)p->router_w;
  a.sgw = SI > 0 ? (const __half*)p->shared_gate_w : nullptr;
  const int64_t Ks[3] = {H, H, I}, Ns[3] = {I, I, H};
  for (int s = 0; s < 3; ++s) {
    a.codes[s] = (const uint32_t*)p->codes[s];
    a.scales[s] = (const __half*)p->scales[s];
    a.zeros[s] = (const __half*)p->zeros[s];
    a.c_es[s] = Ns[s] * (Ks[s] * bits / 32);
    a.s_es[s] = Ns[s] * (Ks[s] / 128);
    a.sv_es[s] = Ns[s] * r;
    if (lora) {
      a.U[s] = (const __half*)p->U[s];
      a.clus[s] = p->cluster_of[s];
      a.SV[s] = (const __half*)p->SV[s];
      a.urows[s] = p->u_rows[s] > 0 ? (int)p->u_rows[s] : a.C;
    } else {
      a.urows[s] = 1;
    }
    if (SI > 0) {
      a.scodes[s] = (const uint32_t*)p->shared_codes[s];
      a.sscales[s] = (const __half*)p->shared_scales[s];
      a.szeros[s] = (const __half*)p->shared_zeros[s];
    }
  }
  if (lora) {
    a.uslot[0] = p->u_slot[0];
    a.uslot[1] = p->u_slot[1];
  }
  a.out = (__half*)p->out;
  a.res = (const __half*)p->residual;
  a.logits = (__half*)p->router_logits;
  const int P_ = (int)(B * p->top_k);
  P.bits = bits;
  P.sbits = sbits;
  P.lora = lora;
  P.rc = H <= 512 ? 1 : H <= 1024 ? 2 : H <= 2048 ? 4 : 8;
  {
    // router rows per workgroup: one pass of 8 waves x RB rows
    const int rb = P.rc >= 8 ? 2 : 16 / P.rc, nrow = (int)p->experts + (SI > 0 ? 1 : 0);
    a.nrw = (nrow + 8 * rb - 1) / (8 * rb);
    // (the counters of 48 tokens fill bytes 64 .. 255 of the workspace)
    if (getenv("GLQ_MOE_LANE_ROUTER1") || B > 48) a.nrw = 1;
  }
  a.gRGU = role_geom((int)I, (int)H, bits, r, P_, true);
  // routed down rows longer than 64 pieces: K parts of whole groups, each at
  // most 64 pieces (one a lane), the smallest such count that divides the row
  a.kd = 1;
  if (I * bits / 128 > 64)
    for (int kd = 2; kd <= (int)(I / 128); ++kd)
      if ((I / 128) % kd == 0 && (I / 128 / kd) * bits <= 64) {
        a.kd = kd;
        break;
      }
  if (const char* e = getenv("GLQ_MOE_LANE_KD")) a.kd = atoi(e) == 1 ? 1 : a.kd;
  a.kdp = (int)(I / a.kd);
  a.gRD = role_geom((int)H, a.kdp, bits, 0, P_ * a.kd, false);
  a.gRD.G = (int)(I / 128);       // scale rows and code rows keep their full pitch
  a.gRD.kw = (int)(I * bits / 32);
  a.nrd = (int)role_blocks(a.gRD);
  a.su = (int)((H + kXuSlice - 1) / kXuSlice);
  a.sd = (int)((I + kXuSlice - 1) / kXuSlice);
  // Routed experts in the streamed token-tile form when the picks are at
  // least twice the experts (two token rows a tile on average; config 3 at
  // 16 tokens: 316 -> 179 us a step, at 8 tokens 179 -> 175 us): each code
  // decoded once for all of an expert's tokens instead of once per pick.
  // GLQ_MOE_XT16=0/1 overrides the choice.
  a.xt = 0;
  {
    const char* f = getenv("GLQ_MOE_XT16");
    const bool want = f ? atoi(f) != 0 : P_ >= 2 * a.E;
    if (want && bits == 2 && P_ <= 128 && H % 128 == 0 && I % 128 == 0 &&
        (!lora || (r <= 64 && r % 8 == 0))) {
      // the down's rows in K slices of at most 28 groups: config 3's 14336
      // in four
      const int gd = (int)(I / 128);
      a.xt = 1;
      a.gXgu = xs_geom((int)I, (int)H, 16 * kXguWaves, 1);
      a.gXd = xs_geom((int)H, (int)I, 16 * kXdWaves, (gd + 27) / 28);
      a.kd = a.gXd.ks;  // summed at the combine
    }
  }
  if (SI > 0) {
    a.gSGU = role_geom((int)SI, (int)H, sbits, 0, (int)B, true);
    // from kMoeT16MinB tokens the shared gate/up runs in the tile form: each
    // code decoded once for every token (4-bit codes, 8 <= H/128 <= 32)
    a.t16s = sbits == 4 && B >= kMoeT16MinB && H >= 1024 && (SI + 63) / 64 <= kMoeT16MaxRB &&
             !getenv("GLQ_MOE_NO_T16");
    if (a.t16s) a.gS16 = t16_geom((int)SI, (int)H, (int)B);
    a.gSD = role_geom((int)H, (int)SI, sbits, 0, (int)B, false, true);
    // (the shared down's routed part is formed by the K slices: at least 2)
    a.t16d = sbits == 4 && B >= kMoeT16MinB && SI > 1024 && (H + 63) / 64 <= kMoeT16MaxRB &&
             !getenv("GLQ_MOE_NO_T16");
    if (a.t16d) a.gSD16 = t16_geom((int)H, (int)SI, (int)B);
    const int lr = a.gSD.lr, rpi = 64 / lane_lrp(lr), pd = moe_lane_pd((lr + 63) / 64);
    a.rows_wg = rpi * pd * 8 * a.gSD.rpw;
  } else {
    a.rows_wg = std::max(1, 256 / a.topk);
  }
  a.ngu = (int)role_blocks(a.gRGU);
  // The combine in the routed down launch (3 launches instead of 4): the
  // down role in whole workgroups per item, each its row block, whose last
  // arriving workgroup combines the block; the shared expert's down (lane
  // form, rows of 64-lane groups) moves to the gate/up launch.  Taken with a
  // 4-bit shared expert (its down then leaves the last launch) when a block's
  // combine is light (rows x picks <= kMoeFuseWork): config 2 at 1-2 tokens.
  // Without a shared expert, or with larger blocks, the separate combine
  // launch spreads the combine wider and measured faster.
  a.fuse = 0;
  if (!getenv("GLQ_MOE_NO_FUSE") && !a.xt && bits == 2 && SI > 0 && sbits == 4 && !a.t16d &&
      lane_lrp(a.gSD.lr) == 64 && (a.gSD.lr + 63) / 64 <= 4) {
    LaneGeom g = role_geom((int)H, a.kdp, bits, 0, P_ * a.kd, false, true);
    g.G = a.gRD.G;
    g.kw = a.gRD.kw;
    const int np = (g.lr + 63) / 64, rpi = 64 / lane_lrp(g.lr);
    const int nrb = g.wpi / 8, rows_blk = 8 * g.rpw * moe_lane_pd(np) * rpi;
    if (nrb <= kMoeCombineCnt / 4 && (int64_t)B * nrb <= kMoeCombineCnt &&
        (int64_t)nrb * rows_blk >= H && rows_blk * a.topk <= kMoeFuseWork) {
      a.fuse = 1;
      // GLQ_MOE_SPIN_TICKS: the combine's wait bound (tests set 0 to take the
      // local a_down path)
      const char* e = getenv("GLQ_MOE_SPIN_TICKS");
      a.spin = e ? (uint64_t)strtoull(e, nullptr, 10) : kMoeSpinTicks;
      a.gRD = g;
      a.nrd = (int)role_blocks(g);
      a.nrb = nrb;
      a.rows_blk = rows_blk;
    }
  }
  // The header (kMoeWsHeader bytes) holds the many-token path's router
  // arrival counter (word 0), this path's per-token router counters (bytes
  // 64 ..) and its token-tile row-block counters (bytes 1024 ..), all of
  // which must be zero between steps: a workspace may serve both paths
  // (steps of different sizes).
  int64_t o = kMoeWsHeader;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += align_up(std::max<int64_t>(bytes, 1), 256);
    return at;
  };
  P.off_sel = take(4 * P_);
  P.off_wts = take(2 * P_);
  P.off_sg = take(2 * B);
  P.off_lgw = take(2 * B * (p->experts + 1));
  // a of every (cluster, token) in the router's launch when all clusters' U
  // take a few MB and the pairs are few (then it saves a launch), else of the
  // picks after routing (measured on config 2: every pair wins at B <= 2,
  // the picks from B = 4)
  const int64_t ubytes = 2 * (int64_t)a.C * H * r * 2;
  const bool uall = lora && ubytes <= kMoeLaneXuAllBytes && !getenv("GLQ_MOE_LANE_XU_GATE");
  a.xuall = 0;
  if (uall && (int64_t)a.C * B <= kMoeLaneXuAllPairs) a.xuall = 1;
  // from 8 tokens, one tile job per (matrix, cluster, slice) takes every token
  // (measured on config 2: B = 8 65.2 -> 61.2 us, B = 16 82.6 -> 78.3 us; even
  // at B = 4, where the picks' own jobs stay)
  if (uall && B >= 8 && B <= kXuTileMaxB && r <= kXuTileMaxRank && !getenv("GLQ_MOE_NO_XU_TILE"))
    a.xuall = 2;
  P.off_agu = take(4 * 2 * (int64_t)r * a.su * (a.xuall ? (int64_t)a.C * B : P_));
  // the streamed expert tiles read a as fp16, finished by the tile jobs
  P.off_a16 = take(a.xt && a.xuall == 2 && lora ? 2 * 2 * (int64_t)a.C * B * r : 0);
  P.off_inter = take(2 * (int64_t)P_ * I);
  P.off_yb = take(4 * (int64_t)a.kd * P_ * H);
  P.off_ad = take(4 * (int64_t)P_ * a.sd * r);
  P.off_sinter = take(SI > 0 ? 2 * B * SI : 0);
  // the token-tile roles' partial blocks (the shared gate/up's and the shared
  // down's run in different launches and share them) and the routed part
  const int64_t t16p = std::max(a.t16s ? t16_wgs(a.gS16) * 2 : 0, a.t16d ? t16_wgs(a.gSD16) : 0);
  P.off_t16p = take(4 * t16p * kT16Elems);
  P.off_rtd = take(a.t16d ? 4 * B * H : 0);
  P.off_sy = take(a.fuse && SI > 0 ? 2 * B * H : 0);
  P.ws_need = o;
  P.lds_route = (size_t)(((2 * (a.E + 1) + 15) & ~15) + 4 * a.E + 4 * 16);
  P.lds_xu = lora ? (size_t)LaneXu(r).lds_bytes(r) : 0;
  P.lds_xut = a.xuall == 2 ? (size_t)std::max(8 * 32 * kXuTileStride * 2, 8 * 4 * 256 * 4) : 0;
  P.lds_comb = (size_t)(4 * ((a.topk * r + 1) / 2) + 4 * a.rows_wg * (a.topk + 1));
  P.lds_down = P.lds_xu;
  if (a.fuse)  // the combine's adl, contrib and routed; after them a local a_down's scratch
    P.lds_down = std::max(P.lds_down, (size_t)(4 * ((a.topk * r + 1) / 2) +
                                               4 * a.rows_blk * (a.topk + 1)) + P.lds_xu);
  P.lds_xgu = (size_t)(xs_lds_bytes(kXsChunk) + xs_tr_bytes(kXguWaves)) + 2 * 16 * 2 * (size_t)r;
  P.lds_xd = std::max((size_t)(xs_lds_bytes(kXsChunk) + xs_tr_bytes(kXdWaves)), P.lds_xu);
  P.lds_sd16 = 0;
  if (a.t16d) {
    const int64_t nt = (B + a.gSD16.ks - 1) / a.gSD16.ks;  // tokens of a K slice's routed part
    P.lds_sd16 = (size_t)(t16_lds_bytes(false) + 16 * ((P_ * r + 7) / 8) + 4 * nt * kT16Rows * a.topk);
  }
  return true;
}

// ---- launches ----
template <int SBITS, int SLRP, int RC, bool T16>
static int launch_route_t(const MoeLanePlan& P, hipStream_t s) {
  const MoeLaneArgs& a = P.a;
  const int64_t shared = T16 ? t16_wgs(a.gS16) : SBITS ? role_blocks(a.gSGU) : 0;
  const int64_t grid = a.B * a.nrw + moe_lane_nxu(a.xuall, a.C, a.B, a.su) + shared;
  size_t lds = a.xuall == 1 ? std::max(P.lds_route, P.lds_xu)
               : a.xuall == 2 ? std::max(P.lds_route, P.lds_xut)
                              : P.lds_route;
  if (T16) lds = std::max(lds, (size_t)t16_lds_bytes(true));
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(moe_lane_route_kernel<SBITS, SLRP, RC, T16>, lds, attr);
  if (rc) return rc;
  moe_lane_route_kernel<SBITS, SLRP, RC, T16><<<dim3((unsigned)grid), dim3(kMoeLaneThreads), lds,
                                                s>>>(a);
  GLQ_LAUNCH_CHECK("moe_lane_route_kernel");
  return GLQ_OK;
}
template <int SBITS, int SLRP, int RC>
static int launch_route(const MoeLanePlan& P, hipStream_t s) {
  if constexpr (SBITS == 4)
    if (P.a.t16s) return launch_route_t<SBITS, SLRP, RC, true>(P, s);
  return launch_route_t<SBITS, SLRP, RC, false>(P, s);
}

template <int SBITS, int SLRP>
static int launch_route_rc(const MoeLanePlan& P, hipStream_t s) {
  if (P.rc == 1) return launch_route<SBITS, SLRP, 1>(P, s);
  if (P.rc == 2) return launch_route<SBITS, SLRP, 2>(P, s);
  if (P.rc == 4) return launch_route<SBITS, SLRP, 4>(P, s);
  return launch_route<SBITS, SLRP, 8>(P, s);
}

template <int BITS, int LRP, int NSV>
static int launch_gu(const MoeLanePlan& P, hipStream_t s) {
  const int64_t grid = role_blocks(P.a.gRGU);
  moe_lane_gu_kernel<BITS, LRP, NSV><<<dim3((unsigned)grid), dim3(kMoeLaneThreads), 0, s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_gu_kernel");
  return GLQ_OK;
}

template <int BITS, int LRP, int NSV, int SNP>
static int launch_gu_sd(const MoeLanePlan& P, hipStream_t s) {
  const int64_t grid = P.a.ngu + role_blocks(P.a.gSD);
  moe_lane_gu_sd_kernel<BITS, LRP, NSV, 4, 64, SNP>
      <<<dim3((unsigned)grid), dim3(kMoeLaneThreads), 0, s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_gu_sd_kernel");
  return GLQ_OK;
}
template <int BITS, int LRP, int NSV>
static int launch_gu_or_sd(const MoeLanePlan& P, hipStream_t s) {
  if (!P.a.fuse || P.a.SI == 0) return launch_gu<BITS, LRP, NSV>(P, s);
  if constexpr (BITS == 2) {
    const int snp = (P.a.gSD.lr + 63) / 64;
    if (snp == 1) return launch_gu_sd<BITS, LRP, NSV, 1>(P, s);
    if (snp == 2) return launch_gu_sd<BITS, LRP, NSV, 2>(P, s);
    if (snp == 3) return launch_gu_sd<BITS, LRP, NSV, 3>(P, s);
    return launch_gu_sd<BITS, LRP, NSV, 4>(P, s);
  }
  GLQ_CHECK(false, "fused combine needs 2-bit experts");
}

template <int BITS, int LRP, int NP>
static int launch_down(const MoeLanePlan& P, hipStream_t s) {
  const int64_t grid = P.a.nrd + (P.lora ? (int64_t)P.a.B * P.a.topk * P.a.sd : 0);
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(moe_lane_down_kernel<BITS, LRP, NP>, P.lds_down, attr);
  if (rc) return rc;
  moe_lane_down_kernel<BITS, LRP, NP><<<dim3((unsigned)grid), dim3(kMoeLaneThreads), P.lds_down,
                                        s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_down_kernel");
  return GLQ_OK;
}

// Routed gate/up and down in the token-tile form.
static int launch_xt(const MoeLanePlan& P, hipStream_t s) {
  static size_t attr_gu = 64 * 1024, attr_d = 64 * 1024;
  int rc = set_lds_limit(moe_lane_gu_xt_kernel, P.lds_xgu, attr_gu);
  if (rc) return rc;
  int64_t grid = (int64_t)P.a.E * P.a.gXgu.RB;
  moe_lane_gu_xt_kernel<<<dim3((unsigned)grid), dim3(kXguWaves * 64), P.lds_xgu, s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_gu_xt_kernel");
  rc = set_lds_limit(moe_lane_down_xt_kernel, P.lds_xd, attr_d);
  if (rc) return rc;
  grid = (P.lora ? (int64_t)P.a.B * P.a.topk * P.a.sd : 0) +
         (int64_t)P.a.E * P.a.gXd.RB * P.a.gXd.ks;
  moe_lane_down_xt_kernel<<<dim3((unsigned)grid), dim3(kMoeLaneThreads), P.lds_xd, s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_down_xt_kernel");
  return GLQ_OK;
}

static int launch_sdown_t16(const MoeLanePlan& P, hipStream_t s) {
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(moe_lane_sdown_t16_kernel, P.lds_sd16, attr);
  if (rc) return rc;
  moe_lane_sdown_t16_kernel<<<dim3((unsigned)t16_wgs(P.a.gSD16)), dim3(kMoeLaneThreads), P.lds_sd16,
                              s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_sdown_t16_kernel");
  return GLQ_OK;
}

template <int SBITS, int SLRP, int SNP>
static int launch_sdown(const MoeLanePlan& P, hipStream_t s) {
  const int64_t grid = role_blocks(P.a.gSD);
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(moe_lane_sdown_kernel<SBITS, SLRP, SNP>, P.lds_comb, attr);
  if (rc) return rc;
  moe_lane_sdown_kernel<SBITS, SLRP, SNP><<<dim3((unsigned)grid), dim3(kMoeLaneThreads),
                                            P.lds_comb, s>>>(P.a);
  GLQ_LAUNCH_CHECK("moe_lane_sdown_kernel");
  return GLQ_OK;
}

// Template arguments from the plan: LRP from a row's pieces, NP pieces per
// lane (LRP 64 only), NSV SV dwords per lane (rank <= 2 NSV LRP).
template <int BITS>
static int dispatch_gu(const MoeLanePlan& P, hipStream_t s) {
  const int lrp = lane_lrp(P.a.gRGU.lr), r = P.a.rank;
  if (lrp == 64) return launch_gu_or_sd<BITS, 64, 1>(P, s);
  if (lrp == 32)
    return r <= 64 ? launch_gu_or_sd<BITS, 32, 1>(P, s) : launch_gu_or_sd<BITS, 32, 2>(P, s);
  if (r <= 32) return launch_gu_or_sd<BITS, 16, 1>(P, s);
  return r <= 64 ? launch_gu_or_sd<BITS, 16, 2>(P, s) : launch_gu_or_sd<BITS, 16, 4>(P, s);
}

template <int BITS>
static int dispatch_down(const MoeLanePlan& P, hipStream_t s) {
  const int lr = P.a.gRD.lr, lrp = lane_lrp(lr), np = (lr + 63) / 64;
  if (lrp == 64) {
    if (np == 1) return launch_down<BITS, 64, 1>(P, s);
    if (np == 2) return launch_down<BITS, 64, 2>(P, s);
    if (np == 3) return launch_down<BITS, 64, 3>(P, s);
    return launch_down<BITS, 64, 4>(P, s);
  }
  if (lrp == 32) return launch_down<BITS, 32, 1>(P, s);
  return launch_down<BITS, 16, 1>(P, s);
}

template <int SBITS>
static int dispatch_shared(const MoeLanePlan& P, hipStream_t s, bool route) {
  if (route) {
    const int lrp = lane_lrp(P.a.gSGU.lr);
    if (lrp == 64) return launch_route_rc<SBITS, 64>(P, s);
    if (lrp == 32) return launch_route_rc<SBITS, 32>(P, s);
    return launch_route_rc<SBITS, 16>(P, s);
  }
  if (SBITS == 4 && P.a.t16d) return launch_sdown_t16(P, s);
  const int lr = P.a.gSD.lr, lrp = lane_lrp(lr), np = (lr + 63) / 64;
  if (lrp == 64) {
    if (np == 1) return launch_sdown<SBITS, 64, 1>(P, s);
    if (np == 2) return launch_sdown<SBITS, 64, 2>(P, s);
    if (np == 3) return launch_sdown<SBITS, 64, 3>(P, s);
    return launch_sdown<SBITS, 64, 4>(P, s);
  }
  if (lrp == 32) return launch_sdown<SBITS, 32, 1>(P, s);
  return launch_sdown<SBITS, 16, 1>(P, s);
}

static int moe_lane_launch(const MoeLanePlan& P, hipStream_t s) {
  const MoeLaneArgs& a = P.a;
  int rc;
  // 1. router (+ shared gate/up)
  if (P.sbits == 2) rc = dispatch_shared<2>(P, s, true);
  else if (P.sbits == 4) rc = dispatch_shared<4>(P, s, true);
  else rc = launch_route_rc<0, 16>(P, s);
  if (rc) return rc;
  // 2. a of each pick's gate and up (unless formed for every cluster in 1)
  if (P.lora && !a.xuall) {
    static size_t attr = 64 * 1024;
    rc = set_lds_limit(moe_lane_xu_kernel, P.lds_xu, attr);
    if (rc) return rc;
    moe_lane_xu_kernel<<<dim3((unsigned)(2 * a.B * a.topk * a.su)), dim3(kMoeLaneThreads),
                         P.lds_xu, s>>>(a);
    GLQ_LAUNCH_CHECK("moe_lane_xu_kernel");
  }
  if (a.xt) {
    // 3-4. routed gate/up and down (+ a_down) in the token-tile form
    rc = launch_xt(P, s);
    if (rc) return rc;
  } else {
    // 3. routed gate/up
    rc = P.bits == 2 ? dispatch_gu<2>(P, s) : dispatch_gu<4>(P, s);
    if (rc) return rc;
    // 4. routed down (+ a_down; fuse: + the combine)
    rc = P.bits == 2 ? dispatch_down<2>(P, s) : dispatch_down<4>(P, s);
    if (rc) return rc;
  }
  if (a.fuse) return GLQ_OK;
  // 5. shared down + combine, or the combine alone
  if (P.sbits == 2) return dispatch_shared<2>(P, s, false);
  if (P.sbits == 4) return dispatch_shared<4>(P, s, false);
  {
    static size_t attr = 64 * 1024;
    rc = set_lds_limit(moe_lane_combine_kernel, P.lds_comb, attr);
    if (rc) return rc;
  }
  const int64_t nb = (int64_t)a.B * ((a.H + a.rows_wg - 1) / a.rows_wg);
  moe_lane_combine_kernel<<<dim3((unsigned)nb), dim3(256), P.lds_comb, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_lane_combine_kernel");
  return GLQ_OK;
}

int64_t moe_lane_workspace_bytes(const glq_moe_params* p) {
  MoeLanePlan P;
  if (!moe_lane_plan(p, P)) return -1;
  return P.ws_need;
}

int moe_lane_decode(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                    hipStream_t s) {
  MoeLanePlan P;
  GLQ_CHECK(moe_lane_plan(p, P), "the lane path does not take this step");
  GLQ_CHECK(workspace != nullptr && workspace_bytes >= P.ws_need,
            "workspace of %lld bytes needed (got %lld)", (long long)P.ws_need,
            (long long)workspace_bytes);
  GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  char* w = (char*)workspace;
  MoeLaneArgs& a = P.a;
  a.sel = (int32_t*)(w + P.off_sel);
  a.wts = (__half*)(w + P.off_wts);
  a.sg = (__half*)(w + P.off_sg);
  a.lgw = (__half*)(w + P.off_lgw);
  // the per-token router counters sit in bytes 64 .. 127 of the header, which
  // the many-token path leaves unused (its counter is word 0): both zero
  // before the first step and after every step
  a.rcnt = (unsigned*)(w + 64);
  a.agu = (float*)(w + P.off_agu);
  a.inter = (__half*)(w + P.off_inter);
  a.yb = (float*)(w + P.off_yb);
  a.ad = (float*)(w + P.off_ad);
  a.sinter = (__half*)(w + P.off_sinter);
  a.gS16.part = a.gSD16.part = (float*)(w + P.off_t16p);
  a.gS16.cnt = (unsigned*)(w + 1024);
  a.gSD16.cnt = (unsigned*)(w + 1024 + 4 * kMoeT16MaxRB);
  a.rtd = (float*)(w + P.off_rtd);
  a.sy = (__half*)(w + P.off_sy);
  a.ccnt = (unsigned*)(w + 4096);  // header bytes 4096 .. 8191, zero between steps
  if (a.xt && a.xuall == 2 && P.lora) {
    a.a16 = (__half*)(w + P.off_a16);
    a.xucnt = (unsigned*)(w + 256);  // header bytes 256 .. 511 (2 C <= 64 counters)
  }
  a.adcnt = (unsigned*)(w + 512);  // header bytes 512 .. 575 (16 tokens)
  return moe_lane_launch(P, s);
}

// ---------------------------------------------------------------------------
// The pieces of a step whose routed experts are not GPTQ (TurboQuant experts,
// glorcq_amd/moe_block.py): routing alone, the weighted combine, SwiGLU.
// ---------------------------------------------------------------------------

// Routing of B tokens: the lane router, nrw workgroups per token.
template <int RC>
__global__ __launch_bounds__(kMoeLaneThreads) void moe_route_only_kernel(MoeLaneArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  moe_lane_router<RC>(a, blockIdx.x / a.nrw, blockIdx.x % a.nrw, smem);
}

// The first launch of a TurboQuant block's decode step: routing, the
// randomized Hadamard transform of the tokens' rows for gate and up, and the
// fp32 partials of h U for every gate and up cluster -- three jobs that need
// only h, in one launch.  Workgroups [0, B nrw): the router
// (moe_lane_router); then, with signs, B workgroups of one row's transform
// (rht_kernel's arithmetic: fp32 butterflies in LDS, one rounding); then
// pairs of (U, 256-row slice) jobs, two per workgroup (lowrank_partial over
// the B token rows) into parts[u][s] (n_u, S, B, rpad); then (SBITS > 0) the
// shared expert's gate/up rows in pairs (the lane router launch's role,
// SguSrc: sinter).
struct TurboPrepArgs {
  MoeLaneArgs a;  // the router's fields; with a shared expert, its gate/up role (gSGU)
  const float* signs;  // (H,) or null: no transform
  __half* xrot;        // (B, H)
  int logd;
  float scale;
  const __half* U;     // (n_u, H, rank)
  int n_u, S, rank, rpad;
  float* parts;        // (n_u, S, B, rpad)
};

constexpr int kPrepJobLds = (4 * 4 * 64) * 4 + 16 * kLowrankRows * 2 + 64 * kLowrankUtStride * 2;

template <int RC, int MC, int SBITS, int SLRP>
__global__ __launch_bounds__(kMoeLaneThreads) void turbo_prep_kernel(TurboPrepArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  const MoeLaneArgs& a = g.a;
  int b = blockIdx.x;
  if (b < a.B * a.nrw) {
    moe_lane_router<RC>(a, b / a.nrw, b % a.nrw, smem);
    return;
  }
  b -= a.B * a.nrw;
  if (g.signs) {
    if (b < a.B) {  // the transform of token b's row
      rht_row_f16(a.h + (int64_t)b * a.H, g.signs, g.xrot + (int64_t)b * a.H, a.H, g.logd,
                  g.scale, (float*)smem, kMoeLaneThreads);
      return;
    }
    b -= a.B;
  }
  const int njobs = g.n_u * g.S, nxw = (njobs + 1) / 2;
  if (b >= nxw) {
    if constexpr (SBITS != 0) {
      const int wvb = moe_lane_wave();
      lane_run<SguSrc, SBITS, false, SLRP, 1, kMoePairPD, 1, false, false, true>(
          SguSrc{a}, a.gSGU, (b - nxw) * 8 + wvb, wvb, nullptr);
    }
    return;
  }
  // two (U, slice) jobs: 256-thread groups side by side, each with its LDS
  const int grp = threadIdx.x >> 8, tid = threadIdx.x & 255;
  const int job = 2 * b + grp;
  const int jc = min(job, njobs - 1);  // a group past the list computes job njobs-1 and writes nothing
  const int u = jc / g.S, sl = jc - u * g.S;
  unsigned char* gl = smem + grp * kPrepJobLds;
  float* red = (float*)gl;
  __half* xl = (__half*)(red + 4 * 4 * 64);
  __half* ut = xl + 16 * kLowrankRows;
  auto xrow = [&](int m) { return a.h + (int64_t)m * a.H; };
  lowrank_partial<MC>(xrow, a.B, a.H, g.rank, g.rpad, g.U + (int64_t)u * a.H * g.rank, sl,
                      job < njobs ? g.parts + ((int64_t)u * g.S + sl) * a.B * g.rpad : nullptr,
                      red, xl, tid, ut);
}

// ---------------------------------------------------------------------------
// The down projection's inputs of a TurboQuant block's decode step, for
// every pick p, in one launch: xd[p] = fp16(inter[p] Pi^T) (the QR rotation:
// the reference's fp16(x.float() @ Pi.float().T), moe_block.py:352-356) or,
// with signs, the transform of inter[p] (rht_row_f16); and the fp32 partials
// of inter[p] U_down[cluster(sel[p])] over 256-row slices (the down GEMV's a:
// each pick's own x U, moe_block.py:661-676).
// Rotation workgroup (16-row block of xd, 16-pick block): its 4 waves split
// K; A = the picks' inter rows, B = Pi's rows (row n weighs output n,
// contiguous in k), one v_mfma_f32_16x16x32_f16 per 32 k; the waves' tiles
// summed in LDS in wave order.  Then (SNP > 0) the shared expert's down rows
// over its sinter, 4 waves a workgroup (SdySrc: sy).
// ---------------------------------------------------------------------------
struct TurboDownPrepArgs {
  const __half* inter;    // (P, I)
  const __half* Pi;       // (I, I), or null with signs
  const float* signs;     // (I,), or null
  __half* xd;             // (P, I)
  int P, I, logd;
  float scale;
  int nrot;               // workgroups of the rotation, first in the grid
  const __half* U;        // (C, I, rank), or null: no x U
  const int32_t* cluster;  // (E,) expert -> U
  const int32_t* sel;     // (P,) pick -> expert
  int E, C, S, rank, rpad;
  float* parts;           // (P, S, 1, rpad)
  int nxu;                // x U jobs, after the rotation
  MoeLaneArgs sa;         // the shared down role (scodes[2], sinter, sy, gSD)
};

constexpr int kDownPrepLds = 4 * 4 * 64 * 4 + 16 * kLowrankRows * 2;

template <int SLRP, int SNP>
__global__ __launch_bounds__(256) void turbo_down_prep_kernel(TurboDownPrepArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  if (b < g.nrot) {
    if (g.signs) {
      rht_row_f16(g.inter + (int64_t)b * g.I, g.signs, g.xd + (int64_t)b * g.I, g.I, g.logd,
                  g.scale, (float*)smem, 256);
      return;
    }
    const int nrb = (g.I + 15) / 16, rb = b % nrb, pb = b / nrb;
    const int wave = tid >> 6, lane = tid & 63, li = lane & 15, kb = lane >> 4;
    const __half* brow = g.Pi + (int64_t)min(rb * 16 + li, g.I - 1) * g.I;
    const int pa = pb * 16 + li;  // this lane's A row (pick)
    const __half* arow = g.inter + (int64_t)min(pa, g.P - 1) * g.I;
    const int nsteps = g.I / 32, q = (nsteps + 3) / 4;
    const int s0 = wave * q, s1 = min(nsteps, s0 + q);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int st = s0; st < s1; ++st) {
      const int k = 32 * st + 8 * kb;
      const f16x8 av = pa < g.P ? *(const f16x8*)(arow + k) : f16x8{};
      acc = mfma_16x16x32(av, *(const f16x8*)(brow + k), acc);
    }
    // acc[i] of lane (li, kb): pick 4kb + i, output row li of the block
    float* red = (float*)smem;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 64 + lane] = acc[i];
    __syncthreads();
    if (wave == 0) {
      const int n = rb * 16 + li;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = ((red[i * 64 + lane] + red[(4 + i) * 64 + lane]) +
                         red[(8 + i) * 64 + lane]) + red[(12 + i) * 64 + lane];
        const int p = pb * 16 + 4 * kb + i;
        if (p < g.P && n < g.I) g.xd[(int64_t)p * g.I + n] = __float2half(v);
      }
    }
    return;
  }
  b -= g.nrot;
  if (b >= g.nxu) {
    if constexpr (SNP > 0) {
      const int wvb = (int)__builtin_amdgcn_readfirstlane(tid >> 6);
      lane_run<SdySrc, 4, false, SLRP, SNP, moe_lane_pd(SNP), 1, false, false>(
          SdySrc{g.sa}, g.sa.gSD, (b - g.nxu) * 4 + wvb, wvb, nullptr);
    }
    return;
  }
  // x U job (pick, slice)
  const int p = b / g.S, sl = b - p * g.S;
  const int e = min(max(g.sel[p], 0), g.E - 1);
  const int c = min(max(g.cluster[e], 0), g.C - 1);
  float* red = (float*)smem;
  __half* xl = (__half*)(red + 4 * 4 * 64);
  auto xrow = [&](int) { return g.inter + (int64_t)p * g.I; };
  lowrank_partial<1>(xrow, 1, g.I, g.rank, g.rpad, g.U + (int64_t)c * g.I * g.rank, sl,
                     g.parts + ((int64_t)p * g.S + sl) * g.rpad, red, xl, tid);
}

// out[t][n] = fp16(sum_k w[t][k] y[t k + k][n] + sg[t] shared[t][n])
// (+ residual): the lane path's combine (fmaf over the picks in pick order,
// then the gated shared term), one thread per output.
__global__ __launch_bounds__(256) void moe_combine_kernel(const __half* y, const __half* wts,
                                                          const __half* shared, const __half* sg,
                                                          const __half* res, __half* out, int B,
                                                          int H, int topk) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)B * H) return;
  const int t = (int)(i / H), n = (int)(i - (int64_t)t * H);
  float acc = 0.f;
  for (int k = 0; k < topk; ++k)
    acc = fmaf(__half2float(wts[t * topk + k]),
               __half2float(y[((int64_t)t * topk + k) * H + n]), acc);
  if (shared) acc = fmaf(__half2float(sg[t]), __half2float(shared[i]), acc);
  float o = __half2float(__float2half(acc));
  if (res) o += __half2float(res[i]);
  out[i] = __float2half(o);
}

// out = fp16(fp16(silu(g)) * u) elementwise (act_fn(gate) * up on fp16).
__global__ __launch_bounds__(256) void swiglu_kernel(const __half* g, const __half* u, __half* out,
                                                     int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = swiglu_fp16(__half2float(g[i]), __half2float(u[i]));
}

namespace {
int moe_route_shape(int64_t B, int64_t H, int64_t E, int64_t k) {
  GLQ_CHECK(B >= 1 && B <= 4096, "tokens=%lld must be in 1..4096", (long long)B);
  GLQ_CHECK(E >= 1 && E <= 256, "experts=%lld must be in 1..256", (long long)E);
  GLQ_CHECK(k >= 1 && k <= 16 && k <= E, "top_k=%lld out of range", (long long)k);
  GLQ_CHECK(H >= 8 && H % 8 == 0 && H <= 4096, "hidden=%lld must be a multiple of 8, <= 4096",
            (long long)H);
  return GLQ_OK;
}
}  // namespace

}  // namespace glq

extern "C" int64_t glq_moe_route_workspace_bytes(int64_t tokens, int64_t experts) {
  glq::clear_error();
  if (tokens < 1 || experts < 1) return -1;
  // per-token arrival counters (zero between calls), then the logits
  return 4 * glq::align_up(tokens, 64) + 2 * tokens * (experts + 1);
}

extern "C" int glq_moe_route(const void* h, const void* router_w, const void* shared_gate_w,
                             int64_t tokens, int64_t hidden, int64_t experts, int64_t top_k,
                             int norm_topk_prob, int32_t* sel, void* weights, void* shared_gate,
                             void* logits, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  using namespace glq;
  clear_error();
  if (int rc = moe_route_shape(tokens, hidden, experts, top_k)) return rc;
  GLQ_CHECK(h && router_w && sel && weights && shared_gate, "null h, router_w or outputs");
  GLQ_CHECK(((uintptr_t)h & 15) == 0 && ((uintptr_t)router_w & 15) == 0 &&
                (!shared_gate_w || ((uintptr_t)shared_gate_w & 15) == 0),
            "h, router_w and shared_gate_w must be 16-byte aligned");
  const int64_t need = glq_moe_route_workspace_bytes(tokens, experts);
  GLQ_CHECK(workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15) == 0,
            "workspace of %lld bytes needed, 16-byte aligned", (long long)need);
  MoeLaneArgs a;
  memset(&a, 0, sizeof(a));
  a.B = (int)tokens;
  a.H = (int)hidden;
  a.E = (int)experts;
  a.topk = (int)top_k;
  a.norm = norm_topk_prob ? 1 : 0;
  a.h = (const __half*)h;
  a.rw = (const __half*)router_w;
  a.sgw = (const __half*)shared_gate_w;
  a.sel = sel;
  a.wts = (__half*)weights;
  a.sg = (__half*)shared_gate;
  a.logits = (__half*)logits;
  a.rcnt = (unsigned*)workspace;
  a.lgw = (__half*)((char*)workspace + 4 * align_up(tokens, 64));
  const int rc = hidden <= 512 ? 1 : hidden <= 1024 ? 2 : hidden <= 2048 ? 4 : 8;
  const int rb = rc >= 8 ? 2 : 16 / rc, nrow = (int)experts + (shared_gate_w ? 1 : 0);
  a.nrw = (nrow + 8 * rb - 1) / (8 * rb);
  const size_t lds = (size_t)(((2 * (experts + 1) + 15) & ~15) + 4 * experts + 4 * 16);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(tokens * a.nrw)), block(kMoeLaneThreads);
  if (rc == 1) moe_route_only_kernel<1><<<grid, block, lds, s>>>(a);
  else if (rc == 2) moe_route_only_kernel<2><<<grid, block, lds, s>>>(a);
  else if (rc == 4) moe_route_only_kernel<4><<<grid, block, lds, s>>>(a);
  else moe_route_only_kernel<8><<<grid, block, lds, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_route_only_kernel");
  return GLQ_OK;
}

extern "C" int glq_turbo_moe_prep(const void* h, const void* router_w, const void* shared_gate_w,
                                  int64_t tokens, int64_t hidden, int64_t experts, int64_t top_k,
                                  int norm_topk_prob, int32_t* sel, void* weights,
                                  void* shared_gate, void* logits, void* workspace,
                                  int64_t workspace_bytes, const float* rht_signs, void* x_rot,
                                  const void* U, int64_t n_u, int64_t rank, float* parts,
                                  const glq_moe_shared* shared, void* stream) {
  using namespace glq;
  clear_error();
  if (int rc = moe_route_shape(tokens, hidden, experts, top_k)) return rc;
  GLQ_CHECK(tokens <= 16, "tokens must be <= 16 (got %lld)", (long long)tokens);
  GLQ_CHECK(h && router_w && sel && weights && shared_gate, "null h, router_w or outputs");
  GLQ_CHECK(((uintptr_t)h & 15) == 0 && ((uintptr_t)router_w & 15) == 0 &&
                (!shared_gate_w || ((uintptr_t)shared_gate_w & 15) == 0),
            "h, router_w and shared_gate_w must be 16-byte aligned");
  GLQ_CHECK(!rht_signs || (x_rot && (hidden & (hidden - 1)) == 0),
            "the transform needs x_rot and a power-of-two hidden size");
  GLQ_CHECK(n_u >= 0 && (n_u == 0 || (U && parts && rank > 0 && rank <= 1024 && rank % 8 == 0 &&
                                      ((uintptr_t)U & 15) == 0)),
            "x U needs U (16-byte aligned), parts and a rank that is a multiple of 8");
  const int64_t need = glq_moe_route_workspace_bytes(tokens, experts);
  GLQ_CHECK(workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15) == 0,
            "workspace of %lld bytes needed, 16-byte aligned", (long long)need);
  TurboPrepArgs g;
  memset(&g, 0, sizeof(g));
  MoeLaneArgs& a = g.a;
  a.B = (int)tokens;
  a.H = (int)hidden;
  a.E = (int)experts;
  a.topk = (int)top_k;
  a.norm = norm_topk_prob ? 1 : 0;
  a.h = (const __half*)h;
  a.rw = (const __half*)router_w;
  a.sgw = (const __half*)shared_gate_w;
  a.sel = sel;
  a.wts = (__half*)weights;
  a.sg = (__half*)shared_gate;
  a.logits = (__half*)logits;
  a.rcnt = (unsigned*)workspace;
  a.lgw = (__half*)((char*)workspace + 4 * align_up(tokens, 64));
  const int rc = hidden <= 512 ? 1 : hidden <= 1024 ? 2 : hidden <= 2048 ? 4 : 8;
  const int rb = rc >= 8 ? 2 : 16 / rc, nrow = (int)experts + (shared_gate_w ? 1 : 0);
  a.nrw = (nrow + 8 * rb - 1) / (8 * rb);
  g.signs = rht_signs;
  g.xrot = (__half*)x_rot;
  int logd = 0;
  while ((1ll << logd) < hidden) ++logd;
  g.logd = logd;
  g.scale = 1.f / sqrtf((float)hidden);
  g.U = (const __half*)U;
  g.n_u = (int)n_u;
  g.S = (int)((hidden + kLowrankRows - 1) / kLowrankRows);
  g.rank = (int)rank;
  g.rpad = (int)align_up(rank, 32);
  g.parts = parts;
  int64_t nsgu = 0;
  int slrp = 0;
  if (shared) {
    GLQ_CHECK(shared->bits == 4 && shared->inter > 0 && shared->codes[0] && shared->codes[1] &&
                  shared->scales[0] && shared->scales[1] && shared->zeros[0] &&
                  shared->zeros[1] && shared->sinter && hidden % 128 == 0,
              "the shared gate/up take 4-bit codes with zero-points and hidden a multiple of "
              "128");
    for (int m = 0; m < 2; ++m) {
      a.scodes[m] = (const uint32_t*)shared->codes[m];
      a.sscales[m] = (const __half*)shared->scales[m];
      a.szeros[m] = (const __half*)shared->zeros[m];
    }
    a.SI = (int)shared->inter;
    a.sinter = (__half*)shared->sinter;
    a.gSGU = role_geom((int)shared->inter, (int)hidden, 4, 0, (int)tokens, true);
    slrp = lane_lrp(a.gSGU.lr);
    GLQ_CHECK(slrp >= 32 && a.gSGU.lr <= 64, "the shared gate/up take 33..256-row pieces");
    nsgu = role_blocks(a.gSGU);
  }
  const size_t lds_route = (size_t)(((2 * (experts + 1) + 15) & ~15) + 4 * experts + 4 * 16);
  const size_t lds = std::max({lds_route, rht_signs ? (size_t)4 * hidden : (size_t)0,
                               n_u > 0 ? (size_t)2 * kPrepJobLds : (size_t)0});
  const int64_t grid = tokens * a.nrw + (rht_signs ? tokens : 0) + (n_u * g.S + 1) / 2 + nsgu;
  hipStream_t s = (hipStream_t)stream;
  const dim3 gd((unsigned)grid), block(kMoeLaneThreads);
#define GLQ_PREP_LAUNCH(RC_, MC_, SB_, SL_)                                 \
  do {                                                                      \
    static size_t attr = 64 * 1024;                                         \
    int rc2 = set_lds_limit(turbo_prep_kernel<RC_, MC_, SB_, SL_>, lds, attr); \
    if (rc2) return rc2;                                                    \
    turbo_prep_kernel<RC_, MC_, SB_, SL_><<<gd, block, lds, s>>>(g);        \
  } while (0)
#define GLQ_PREP_SHARED(RC_, MC_)                                           \
  do {                                                                      \
    if (slrp == 0) GLQ_PREP_LAUNCH(RC_, MC_, 0, 64);                        \
    else if (slrp == 32) GLQ_PREP_LAUNCH(RC_, MC_, 4, 32);                  \
    else GLQ_PREP_LAUNCH(RC_, MC_, 4, 64);                                  \
  } while (0)
  const bool mc4 = tokens >= 3;
  if (rc == 1) { if (mc4) GLQ_PREP_SHARED(1, 4); else GLQ_PREP_SHARED(1, 1); }
  else if (rc == 2) { if (mc4) GLQ_PREP_SHARED(2, 4); else GLQ_PREP_SHARED(2, 1); }
  else if (rc == 4) { if (mc4) GLQ_PREP_SHARED(4, 4); else GLQ_PREP_SHARED(4, 1); }
  else { if (mc4) GLQ_PREP_SHARED(8, 4); else GLQ_PREP_SHARED(8, 1); }
#undef GLQ_PREP_SHARED
#undef GLQ_PREP_LAUNCH
  GLQ_LAUNCH_CHECK("turbo_prep_kernel");
  return GLQ_OK;
}

extern "C" int glq_turbo_moe_down_prep(int64_t picks, int64_t inter_dim, const void* inter,
                                       const void* Pi, const float* rht_signs, void* xd,
                                       const void* U, int64_t n_clusters,
                                       const int32_t* cluster, const int32_t* sel,
                                       int64_t experts, int64_t rank, float* parts,
                                       int64_t tokens, int64_t hidden,
                                       const glq_moe_shared* shared, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(picks >= 0 && inter_dim > 0 && experts >= 1, "bad size");
  if (picks == 0) return GLQ_OK;
  GLQ_CHECK(picks < (1 << 20) && inter_dim < (1 << 16), "sizes too large");
  GLQ_CHECK(inter && xd && sel && (Pi != nullptr) != (rht_signs != nullptr),
            "inter, xd, sel and exactly one of Pi and rht_signs required");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(inter) && (!Pi || al16(Pi)), "inter and Pi must be 16-byte aligned");
  GLQ_CHECK(Pi ? inter_dim % 32 == 0 : (inter_dim & (inter_dim - 1)) == 0,
            "inter_dim must be a multiple of 32 (Pi) or a power of two (transform)");
  const bool lora = U != nullptr && rank > 0;
  GLQ_CHECK(!lora || (parts && cluster && n_clusters >= 1 && rank % 8 == 0 && rank <= 1024 &&
                      al16(U)),
            "x U needs parts, cluster, n_clusters and a rank that is a multiple of 8");
  TurboDownPrepArgs g;
  memset(&g, 0, sizeof(g));
  g.inter = (const __half*)inter;
  g.Pi = (const __half*)Pi;
  g.signs = rht_signs;
  g.xd = (__half*)xd;
  g.P = (int)picks;
  g.I = (int)inter_dim;
  int logd = 0;
  while ((1ll << logd) < inter_dim) ++logd;
  g.logd = logd;
  g.scale = 1.f / sqrtf((float)inter_dim);
  g.nrot = Pi ? (int)(((inter_dim + 15) / 16) * ((picks + 15) / 16)) : (int)picks;
  g.U = lora ? (const __half*)U : nullptr;
  g.cluster = cluster;
  g.sel = sel;
  g.E = (int)experts;
  g.C = (int)n_clusters;
  g.S = (int)((inter_dim + kLowrankRows - 1) / kLowrankRows);
  g.rank = lora ? (int)rank : 0;
  g.rpad = (int)align_up(g.rank, 32);
  g.parts = parts;
  g.nxu = lora ? (int)(picks * g.S) : 0;
  int snp = 0, slrp = 64;
  int64_t nsd = 0;
  if (shared) {
    GLQ_CHECK(shared->bits == 4 && shared->inter > 0 && shared->inter % 128 == 0 &&
                  hidden > 0 && tokens >= 1 && tokens <= 16 && shared->codes[2] &&
                  shared->scales[2] && shared->zeros[2] && shared->sinter && shared->sy,
              "the shared down takes 4-bit codes, inter a multiple of 128, 1..16 tokens");
    MoeLaneArgs& sa = g.sa;
    sa.B = (int)tokens;
    sa.H = (int)hidden;
    sa.SI = (int)shared->inter;
    sa.scodes[2] = (const uint32_t*)shared->codes[2];
    sa.sscales[2] = (const __half*)shared->scales[2];
    sa.szeros[2] = (const __half*)shared->zeros[2];
    sa.sinter = (__half*)shared->sinter;
    sa.sy = (__half*)shared->sy;
    sa.gSD = role_geom((int)hidden, (int)shared->inter, 4, 0, (int)tokens, false);
    const int lr = sa.gSD.lr;
    slrp = lane_lrp(lr);
    snp = (lr + 63) / 64;
    GLQ_CHECK(snp <= 4 && (snp == 1 || slrp == 64), "shared inter too wide for the lane form");
    nsd = ((int64_t)sa.gSD.items * sa.gSD.wpi + 3) / 4;
  }
  const int64_t grid = g.nrot + g.nxu + nsd;
  GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
  const size_t lds = std::max<size_t>(kDownPrepLds, rht_signs ? 4 * (size_t)inter_dim : 0);
  hipStream_t s = (hipStream_t)stream;
  int rc = GLQ_OK;
#define GLQ_DPREP(L, N)                                                                     \
  do {                                                                                      \
    static size_t attr = 64 * 1024;                                                         \
    rc = set_lds_limit(turbo_down_prep_kernel<L, N>, lds, attr);                            \
    if (rc) return rc;                                                                      \
    turbo_down_prep_kernel<L, N><<<dim3((unsigned)grid), dim3(256), lds, s>>>(g);          \
  } while (0)
  if (snp == 0) GLQ_DPREP(64, 0);
  else if (slrp == 16) GLQ_DPREP(16, 1);
  else if (slrp == 32) GLQ_DPREP(32, 1);
  else if (snp == 1) GLQ_DPREP(64, 1);
  else if (snp == 2) GLQ_DPREP(64, 2);
  else if (snp == 3) GLQ_DPREP(64, 3);
  else GLQ_DPREP(64, 4);
#undef GLQ_DPREP
  GLQ_LAUNCH_CHECK("turbo_down_prep_kernel");
  return GLQ_OK;
}

extern "C" int glq_moe_combine(const void* y, const void* weights, const void* shared,
                               const void* shared_gate, const void* residual, int64_t tokens,
                               int64_t hidden, int64_t top_k, void* out, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(tokens >= 0 && hidden >= 1 && top_k >= 1 && top_k <= 16, "bad sizes");
  GLQ_CHECK(tokens * hidden < (1ll << 31), "tokens * hidden must be < 2^31");
  if (tokens == 0) return GLQ_OK;
  GLQ_CHECK(y && weights && out && (!shared || shared_gate), "null y, weights, out or gate");
  const int64_t n = tokens * hidden;
  moe_combine_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      (const __half*)y, (const __half*)weights, (const __half*)shared,
      (const __half*)shared_gate, (const __half*)residual, (__half*)out, (int)tokens,
      (int)hidden, (int)top_k);
  GLQ_LAUNCH_CHECK("moe_combine_kernel");
  return GLQ_OK;
}

extern "C" int glq_swiglu(const void* gate, const void* up, int64_t n, void* out, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(n >= 0 && n < (1ll << 40), "bad size");
  if (n == 0) return GLQ_OK;
  GLQ_CHECK(gate && up && out, "null pointer");
  swiglu_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(
      (const __half*)gate, (const __half*)up, (__half*)out, n);
  GLQ_LAUNCH_CHECK("swiglu_kernel");
  return GLQ_OK;
}
