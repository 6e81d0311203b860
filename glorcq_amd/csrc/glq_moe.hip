// MoE block decode step on MI355X: GraphCompatibleMoeBlock.forward
// (inference/moe_block.py:381-436) for B <= 64 tokens, in four launches (five
// when x U is gated on routing) with all routing on the device (no host sync,
// so the step captures in a hipGraph):
//
//  1. moe_route_kernel (256-thread workgroups): router tiles (16 router rows
//     x 16 tokens, MFMA, fp32 sums rounded to fp16 once) write the logits and
//     the shared-expert gate sigmoid(fp16 logit); the router workgroup that
//     arrives last routes every token (softmax, top-k, optional
//     renormalisation, moe_block.py:386-392) and writes the ids, weights and
//     dispatch tables (expert-major pair lists cut into blocks of <= 8
//     tokens) once for the step; the other workgroups form fp32 partials of
//     x U_c for every cluster c of gate and up with MFMA (the cluster-shared
//     precompute, moe_block.py:290-322) and clear the a_down accumulators.
//     With many more clusters than picks those jobs run as moe_xu_kernel
//     after the router, each skipping an unpicked cluster.  Workgroups past
//     the others run the shared expert's gate/up (it does not depend on
//     routing).
//  2. moe_gate_up_kernel: every routed workgroup runs gate and up of one
//     block's expert over a range of 16-row tiles in one pass (two-matrix
//     K-split stream), writing inter = fp16(silu(g) * u) and adding the
//     workgroup's share of a_down = inter U_down[c(e)] to fixed-point
//     accumulators; workgroups past the routed blocks run the shared
//     expert's down projection per (token block, K part).
//  3. moe_down_kernel: routed down projections per (block, K part) with the
//     low-rank term from a_down; fp32 partial outputs.
//  4. moe_combine_kernel: out = fp16(sum_k w_k y_k + sigmoid-gate * fp16(shared))
//     (+ the caller's residual).
//
// Only the selected experts' weights are read (the reference's graph mode
// reads all E, moe_block.py:742-890), and a cluster's U is read once per step
// for all of its experts.  The atomics are 64-bit integer adds of the a_down
// shares (below), whose sum does not depend on their order, and the router's
// arrival counter, which only picks the workgroup that routes: every result
// is the same on every run.
#include <algorithm>
#include <cstring>

#include "glq_handoff.h"
#include "glq_moe_route.h"
#include "glq_stream.h"

namespace glq {

constexpr int kMoeTB = 8;          // tokens per routed block (one MFMA pass for 2-bit)
constexpr int kMoeDepth = 4;       // ring slots per wave (3 chunks in flight)
constexpr int kMoeMaxE = 256;
constexpr int kMoeMaxP = 512;      // tokens * top_k
constexpr int kMoeMaxB = 64;
constexpr int kMoeXBudget = 48 * 1024;  // bytes of staged x per down-projection unit
constexpr int kMoeMaxChunks = 6;        // code chunks per down-projection K part
// a_down = inter U_down is summed over the gate/up workgroups of a block with
// 64-bit integer atomics on values scaled by 2^24: integer addition does not
// depend on the order of the updates, so the sum (and the step's output) is
// the same on every run.  |a_down| < 2^39 fits; the resolution 2^-24 is far
// below the fp16 rounding of a_down that follows.
constexpr float kAdqScale = 16777216.f;

struct MoeArgs {
  int B, H, E, I, topk, norm, C, rank, rpad, SI;
  int nrb;     // router workgroups (16 router rows x 16 tokens each)
  int xurows;  // U rows per x U partial job
  int nbm;     // routed token blocks the grids are sized for
  int sus;     // K-slices of the gate/up x U partials
  int nxu1;    // x U jobs in the router's launch (0 when gated)
  int nxc;     // gated: picked-cluster slots per projection, min(C, B * topk)
  int wgu;     // workgroups per routed block (gate/up)
  int tpu;     // tiles per workgroup (gate/up, routed)
  int stb;     // tokens per shared-expert block
  int nsb;     // shared-expert token blocks
  int wgsu, tpsu;  // shared gate/up: workgroups per token block, tiles per workgroup
  int sr, kr;      // routed down: K parts, codes per part
  int wgd, tpd;    // routed down: workgroups per (block, part), tiles per workgroup
  int ss, ks;      // shared down: K parts, codes per part
  int wgsd, tpsd;  // shared down: workgroups per (token block, part), tiles per workgroup
  int bits, sbits;
  int tl_off;      // LDS byte offset of the routed block's token list (gate/up)
  int pl_off;      // LDS byte offset of the routed block's pair list (down)
  StreamShape shGU, shSGU, shD, shSD;
  const __half* h;
  const __half* rw;
  const __half* sgw;
  const uint32_t* codes[3];
  const __half* scales[3];
  const __half* zeros[3];
  int64_t c_es[3], s_es[3], u_es[3], sv_es[3];
  const __half* U[3];
  const int32_t* clus[3];
  const int32_t* uslot[2];  // gate/up: pool row of each cluster's U (nullptr: row = cluster)
  int urows[3];             // rows of U[s]
  const __half* SV[3];
  const uint32_t* scodes[3];
  const __half* sscales[3];
  const __half* szeros[3];
  // workspace and outputs
  int32_t* sel;    // [B*topk] expert ids
  __half* wts;     // [B*topk] routing weights
  __half* sg;      // [B] shared-expert gate
  float* xu;       // [2][C][sus][B][rpad] gate/up x U partials
  __half* inter;   // [nbm][TB][I]
  unsigned long long* adq;  // [nbm][TB][rpad] a_down sums, fixed point (kAdqScale)
  __half* sinter;  // [B][SI]
  float* yb;       // [sr][B * topk][H] routed down outputs per (token, k) pair (fp32)
  float* sdp;      // [ss][B][H] shared down partial outputs (fp32)
  __half* out;
  const __half* res;  // added to out (fp16 + fp16), or nullptr
  __half* logits;
  __half* lgb;     // [B][E] fp16 router logits (workspace)
  // dispatch tables, built once per step by the router's last workgroup:
  // [0] blocks, then bexp[nbm], bM[nbm], then kMoeTB pair ids per block
  // (t * topk + k; slots past bM repeat the block's first pair), then (gated
  // x U) the number of picked gate and up clusters and their lists [2][nxc]
  int* tab;
  unsigned* rcount;  // router workgroups arrived (zero between steps)
};

// ---------------------------------------------------------------------------
// Dispatch tables, rebuilt in LDS by each workgroup that needs them from the
// top-k ids.  Pair p = t*topk + k.  Each expert's pairs are listed with tokens
// ascending (the token order of torch.where over the expert mask,
// inference/quantized_linear.py:413-416) and cut into blocks of <= kMoeTB.
// ---------------------------------------------------------------------------
struct MoeTables {
  int *sel, *cnt, *off, *boff, *list, *pos, *bexp, *bfirst, *bM, *nblk;
};

__host__ __device__ inline int moe_tables_words(int P, int E, int nbm) {
  return 3 * P + 3 * E + 3 * nbm + 1;
}

__device__ inline MoeTables moe_tables(int* w, int P, int E, int nbm) {
  MoeTables t;
  t.sel = w;
  t.cnt = t.sel + P;
  t.off = t.cnt + E;
  t.boff = t.off + E;
  t.list = t.boff + E;
  t.pos = t.list + P;
  t.bexp = t.pos + P;
  t.bfirst = t.bexp + nbm;
  t.bM = t.bfirst + nbm;
  t.nblk = t.bM + nbm;
  return t;
}

// Builds the tables (all 256 threads); returns the number of blocks.
// `sel_global`: read the top-k ids from the workspace (else t.sel holds them).
__device__ int moe_dispatch(const MoeArgs& a, const MoeTables& t, bool sel_global = true) {
  const int P = a.B * a.topk, E = a.E, tid = threadIdx.x;
  for (int i = tid; i < P; i += 256) {
    const int e = sel_global ? a.sel[i] : t.sel[i];
    t.sel[i] = (e >= 0 && e < E) ? e : -1;
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    int c = 0;
#pragma unroll 8
    for (int p = 0; p < P; ++p) c += (int)(t.sel[p] == e);
    t.cnt[e] = c;
  }
  __syncthreads();
  if (tid < 64) {  // exclusive scans over experts (4 per lane) of pairs and blocks
    int cs[4], bs[4], lc = 0, lb = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * tid + i;
      const int c = e < E ? t.cnt[e] : 0;
      cs[i] = lc;
      bs[i] = lb;
      lc += c;
      lb += (c + kMoeTB - 1) / kMoeTB;
    }
    int ic = lc, ib = lb;
    for (int d = 1; d < 64; d <<= 1) {
      const int uc = __shfl_up(ic, d), ub = __shfl_up(ib, d);
      if (tid >= d) {
        ic += uc;
        ib += ub;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * tid + i;
      if (e < E) {
        t.off[e] = ic - lc + cs[i];
        t.boff[e] = ib - lb + bs[i];
      }
    }
    if (tid == 63) *t.nblk = ib;
  }
  __syncthreads();
  for (int p = tid; p < P; p += 256) {
    const int e = t.sel[p];
    if (e < 0) {
      t.pos[p] = -1;
      continue;
    }
    int r = 0;
#pragma unroll 8
    for (int q = 0; q < p; ++q) r += (int)(t.sel[q] == e);
    t.list[t.off[e] + r] = p;
    const int b = t.boff[e] + r / kMoeTB;
    t.pos[p] = b * kMoeTB + r % kMoeTB;
    if (r % kMoeTB == 0) {
      t.bexp[b] = e;
      t.bfirst[b] = t.off[e] + r;
      t.bM[b] = min(kMoeTB, t.cnt[e] - r);
    }
  }
  __syncthreads();
  return *t.nblk;
}

__device__ __forceinline__ int align_up_dev(int v, int a) { return (v + a - 1) / a * a; }


// ---------------------------------------------------------------------------
// 1. Router + gate/up cluster partials (256-thread workgroups)
// ---------------------------------------------------------------------------
constexpr int kRouteThreads = 256;

__host__ __device__ inline int moe_lg_stride(int E) { return ((E + 3) & ~3) + 4; }

// Softmax, top-k (and optional renormalisation) of every token at once
// (moe_block.py:386-392), by all 256 threads, from the routing keys of every
// (token, expert) in LDS (16-byte aligned rows).  Thread (t, e) counts the
// keys above its own -- the experts ahead of e in (logit descending, index
// ascending); ties go to the lower index, and as the probabilities
// exp(l - max) / sum are monotonic in the logit (distinct fp16 logits give
// distinct fp32 probabilities) this is the probability order -- and an expert
// of rank j < topk lands in sel[t * topk + j]: one compare per pair, no
// dependent passes.  Then (`publish`) one wave per token forms the softmax
// sum (lanes over experts, then a cross-lane sum) and the weights of the
// picks, and writes ids and fp16 weights to the workspace.
__device__ void moe_topk_ranks(const MoeArgs& a, const uint32_t* lgk, int* sel, bool publish) {
  const int E = a.E, tid = threadIdx.x, LS = moe_lg_stride(E), E4 = E & ~3;
  for (int q = tid; q < a.B * E; q += 256) {
    const int t = q / E, e = q - t * E;
    const uint32_t* row = lgk + t * LS;
    const uint32_t ke = row[e];
    int r = 0;
#pragma unroll 4
    for (int j = 0; j < E4; j += 4) {  // 16-byte LDS reads, broadcast across the token's lanes
      const uint4 v = *(const uint4*)(row + j);
      r += (int)(v.x > ke) + (int)(v.y > ke) + (int)(v.z > ke) + (int)(v.w > ke);
    }
    for (int j = E4; j < E; ++j) r += (int)(row[j] > ke);
    if (r < a.topk) sel[t * a.topk + r] = e;
  }
  __syncthreads();
  if (!publish) return;
  const int lane = tid & 63;
  for (int t = tid >> 6; t < a.B; t += 4) {
    const uint32_t* row = lgk + t * LS;
    const float mx = moe_key_logit(row[sel[t * a.topk]]);
    float sum = 0.f;
    for (int e = lane; e < E; e += 64) sum += expf(moe_key_logit(row[e]) - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    // lane j < topk: the j-th pick's probability; the renormalising sum
    // over the picks (in pick order) when norm_topk_prob
    const int e = lane < a.topk ? sel[t * a.topk + lane] : 0;
    const float w = lane < a.topk ? expf(moe_key_logit(row[e]) - mx) / sum : 0.f;
    float ws = 0.f;
    if (a.norm)
      for (int j = 0; j < a.topk; ++j) ws += __shfl(w, j);
    if (lane < a.topk) {
      a.sel[t * a.topk + lane] = e;
      a.wts[t * a.topk + lane] = __float2half(a.norm ? w / ws : w);
    }
  }
}

// Router logits of tokens [16 rb, 16 rb + 16) x router rows [16 tile,
// 16 tile + 16) (the rows after the E experts: the shared-expert gate), one
// MFMA tile (A = h rows staged in LDS, B = router rows) with K split over the
// 4 waves: every router-row load of a wave goes out before it waits, and the
// rows of a tile come from one workgroup per tile, so no CU pulls the whole
// router matrix.  fp32 sums rounded to fp16 once -> workspace (and the
// caller's router_logits); the shared-expert gate sigmoid(fp16 logit) -> sg.
constexpr int kRouteBatch = 8;  // MFMA k-steps (32 codes each) a wave loads at once
__device__ void moe_route_tile(const MoeArgs& a, int id, unsigned char* smem) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int nrow = a.E + (a.sgw ? 1 : 0);
  const int ntile = (nrow + 15) / 16;
  const int tile = id % ntile, rb = id / ntile;
  const int t0 = rb * 16, nt = min(16, a.B - t0);
  const int hstride = a.H + 8;
  __half* hl = (__half*)smem;                       // [nt][H + 8]
  float* red = (float*)(smem + 16 * hstride * 2);  // [4 waves][256]
  const int kseg = a.H / 4;                         // codes per wave (H % 256 == 0)
  const int steps = kseg / 32;
  const int n = min(tile * 16 + li, nrow - 1);
  const __half* wr = (n < a.E ? a.rw + (int64_t)n * a.H : a.sgw) + wave * kseg + 8 * kb;
  const __half* hr = hl + min(li, nt - 1) * hstride + wave * kseg + 8 * kb;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < steps; s0 += kRouteBatch) {
    f16x8 wv[kRouteBatch];
#pragma unroll
    for (int u = 0; u < kRouteBatch; ++u)
      wv[u] = s0 + u < steps ? *(const f16x8*)(wr + 32 * (s0 + u)) : f16x8{};
    if (s0 == 0) {  // h rows into LDS while the router rows are in flight
      for (int idx = tid; idx < nt * (a.H / 8); idx += kRouteThreads) {
        const int m = idx / (a.H / 8), k8 = idx - m * (a.H / 8);
        *(f16x8*)(hl + m * hstride + 8 * k8) = *(const f16x8*)(a.h + (int64_t)(t0 + m) * a.H + 8 * k8);
      }
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kRouteBatch; ++u)
      if (s0 + u < steps) acc = mfma_16x16x32(*(const f16x8*)(hr + 32 * (s0 + u)), wv[u], acc);
  }
  // acc[i]: token 4kb + i, router row li of the tile
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave * 256 + (4 * kb + i) * 16 + li] = acc[i];
  __syncthreads();
  {  // token m = tid / 16, row tile*16 + tid % 16; waves summed in order
    const int m = tid >> 4, r = tile * 16 + (tid & 15);
    const float sum = red[tid] + red[256 + tid] + red[512 + tid] + red[768 + tid];
    const __half lgh = __float2half(sum);
    if (m < nt && r < a.E) {
      handoff_put((uint16_t*)a.lgb + (int64_t)(t0 + m) * a.E + r, __half_as_ushort(lgh));
      if (a.logits) a.logits[(int64_t)(t0 + m) * a.E + r] = lgh;
    }
    if (m < nt && r == a.E && a.sgw)
      a.sg[t0 + m] = __float2half(1.f / (1.f + expf(-__half2float(lgh))));
  }
  if (!a.sgw && tile == 0 && tid < nt) a.sg[t0 + tid] = __float2half(1.f);
}

// x U_c partials of one job (projection s in {gate, up}, cluster c, K-slice q
// of xurows rows): part[t][r] = sum_{k in slice} x[t][k] U_c[k][r], fp32.
// The x and U slices reach LDS by 16-byte loads (both row-major); wave w takes
// rank tiles w, w + 4 over the whole slice with v_mfma_f32_16x16x32_f16
// (A = x rows, 16-byte LDS reads; B = 8 U values of one rank column), so the
// sums need no cross-wave step and leave from registers.
//
// A job leaves at once when no expert's projection s uses cluster c (a
// projection may have fewer clusters than C).  Gated (`gated`, the launch
// after the router's), jobs run over the router's list of picked clusters
// instead -- min(C, B * topk) slots per projection, unused slots leave at
// once -- so a step reads only the picked clusters' U slices.
__device__ void moe_xu_job(const MoeArgs& a, int job, unsigned char* smem, bool gated) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  int s, c, q;
  if (gated) {  // job -> (projection, picked-cluster slot, slice) from the router's lists
    const int per = a.nxc * a.sus;
    s = job / per;
    const int rem = job - s * per, i = rem / a.sus;
    q = rem - i * a.sus;
    const int* pc = a.tab + 1 + (2 + kMoeTB) * a.nbm;
    if (i >= pc[s]) return;  // uniform over the workgroup
    c = pc[2 + s * a.nxc + i];
  } else {
    s = job / (a.C * a.sus);
    const int rem = job - s * a.C * a.sus;
    c = rem / a.sus;
    q = rem - c * a.sus;
    int act = 0;
    for (int e = tid; e < a.E; e += kRouteThreads) act |= (int)(a.clus[s][e] == c);
    if (!__syncthreads_or(act)) return;
  }
  const int xr = a.xurows;
  const int k0 = q * xr, kl = min(xr, a.H - k0);  // kl is a multiple of 128
  const int ntt = (a.B + 15) / 16;                // token tiles
  const int nrt = (a.rank + 15) / 16;             // rank tiles (<= 8)
  const int xstride = xr + 8, ustride = a.rank + 8;
  __half* xl = (__half*)smem;                                           // [B][xr + 8]
  __half* ul = (__half*)(smem + align_up_dev(a.B * xstride * 2, 16));  // [xr][rank + 8]
  const int urow = min(max(a.uslot[s] ? a.uslot[s][c] : c, 0), a.urows[s] - 1);
  const __half* U = a.U[s] + (int64_t)urow * a.u_es[s] + (int64_t)k0 * a.rank;
  const int r8 = a.rank / 8, nu = kl * r8;
  for (int b0 = 0; b0 < nu; b0 += 8 * kRouteThreads) {  // U slice, 16 B per load,
    f16x8 buf[8];                                        // 8 loads in flight per thread
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // unconditional: indices past the slice re-read its last piece
      const int idx = min(b0 + j * kRouteThreads + tid, nu - 1);
      const int k = idx / r8, j8 = idx - k * r8;
      buf[j] = *(const f16x8*)(U + (int64_t)k * a.rank + 8 * j8);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int idx = b0 + j * kRouteThreads + tid;
      if (idx < nu) {
        const int k = idx / r8, j8 = idx - k * r8;
        *(f16x8*)(ul + k * ustride + 8 * j8) = buf[j];
      }
    }
  }
  for (int idx = tid; idx < a.B * (kl / 8); idx += kRouteThreads) {
    const int m = idx / (kl / 8), k8 = idx - m * (kl / 8);
    *(f16x8*)(xl + m * xstride + 8 * k8) = *(const f16x8*)(a.h + (int64_t)m * a.H + k0 + 8 * k8);
  }
  float* out = a.xu + (((int64_t)s * a.C + c) * a.sus + q) * a.B * a.rpad;
  for (int idx = tid; idx < a.B * (a.rpad - nrt * 16); idx += kRouteThreads) {
    const int w = a.rpad - nrt * 16, m = idx / w, j = nrt * 16 + idx - m * w;
    out[(int64_t)m * a.rpad + j] = 0.f;  // rank padding
  }
  __syncthreads();
  const int ksteps = kl / 32;
  for (int rt = wave; rt < nrt; rt += 4) {
    f32x4 acc[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int col = min(rt * 16 + li, a.rank - 1);
    for (int u = 0; u < ksteps; ++u) {
      const int k = 32 * u + 8 * kb;
      f16x8 bv;
#pragma unroll
      for (int e = 0; e < 8; ++e) bv[e] = (_Float16)ul[(k + e) * ustride + col];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        if (tt < ntt) {  // rows past B read a staged row and are not stored
          const int m = min(tt * 16 + li, a.B - 1);
          acc[tt] = mfma_16x16x32(*(const f16x8*)(xl + m * xstride + k), bv, acc[tt]);
        }
    }
    // acc[tt][i]: token tt*16 + 4kb + i, rank column rt*16 + li
    const int j = rt * 16 + li;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = tt * 16 + 4 * kb + i;
        if (tt < ntt && m < a.B) out[(int64_t)m * a.rpad + j] = j < a.rank ? acc[tt][i] : 0.f;
      }
  }
}

// Routing of every token and the dispatch tables, once per step, by the
// router workgroup that finishes last (the logits of all tokens are then in
// the workspace): routing keys staged in LDS, top-k ranks (ids and weights
// published for the combine), expert-major pair lists cut into blocks, the
// tables written to the workspace for the gate/up and down launches.
__device__ void moe_route_finalize(const MoeArgs& a, unsigned char* smem) {
  const int tid = threadIdx.x, nl = a.B * a.E, LS = moe_lg_stride(a.E), P = a.B * a.topk;
  uint32_t* lgk = (uint32_t*)smem;
  const MoeTables t =
      moe_tables((int*)(smem + align_up_dev(4 * a.B * LS, 16)), P, a.E, a.nbm);
  for (int i = tid; i < nl / 8; i += kRouteThreads) {  // 16 bytes of the flat [B][E] array
    const uint32_t* lw = (const uint32_t*)a.lgb + 4 * i;
    const uint32_t w[4] = {handoff_get(lw), handoff_get(lw + 1), handoff_get(lw + 2),
                           handoff_get(lw + 3)};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int f = 8 * i + u, tk = f / a.E, e = f - tk * a.E;
      lgk[tk * LS + e] = moe_key(w[u >> 1] >> (16 * (u & 1)), e);
    }
  }
  for (int f = nl / 8 * 8 + tid; f < nl; f += kRouteThreads) {
    const int tk = f / a.E, e = f - tk * a.E;
    lgk[tk * LS + e] = moe_key(handoff_get((const uint16_t*)a.lgb + f), e);
  }
  __syncthreads();
  moe_topk_ranks(a, lgk, t.sel, true);
  __syncthreads();
  const int nblk = moe_dispatch(a, t, false);
  int* g = a.tab;
  if (tid == 0) g[0] = nblk;
  for (int b = tid; b < a.nbm; b += kRouteThreads) {
    const bool used = b < nblk;
    g[1 + b] = used ? t.bexp[b] : 0;
    g[1 + a.nbm + b] = used ? t.bM[b] : 0;
  }
  for (int i = tid; i < nblk * kMoeTB; i += kRouteThreads) {
    const int b = i / kMoeTB, m = i - b * kMoeTB;
    g[1 + 2 * a.nbm + i] = t.list[t.bfirst[b] + min(m, t.bM[b] - 1)];
  }
  if (a.nxc > 0) {  // gated x U: the picked gate and up clusters, compacted
    int* flag = t.nblk + 1;      // [2][C]
    int* cnt = flag + 2 * a.C;   // [2]
    for (int i = tid; i < 2 * a.C; i += kRouteThreads) flag[i] = 0;
    if (tid < 2) cnt[tid] = 0;
    __syncthreads();
    for (int i = tid; i < 2 * P; i += kRouteThreads) {
      const int sp = i / P, e = t.sel[i - sp * P];
      if (e >= 0) flag[sp * a.C + min(max(a.clus[sp][e], 0), a.C - 1)] = 1;
    }
    __syncthreads();
    int* pc = g + 1 + (2 + kMoeTB) * a.nbm;
    for (int i = tid; i < 2 * a.C; i += kRouteThreads)
      if (flag[i]) {  // list order does not matter: each job writes its own cluster's slot
        const int sp = i / a.C, slot = atomicAdd(cnt + sp, 1);
        if (slot < a.nxc) pc[2 + sp * a.nxc + slot] = i - sp * a.C;
      }
    __syncthreads();
    if (tid < 2) pc[tid] = min(cnt[tid], a.nxc);
  }
}

// The x U jobs in a launch of their own, after the router's, each gated on
// its cluster being picked (steps whose clusters outnumber the picks).
__global__ __launch_bounds__(kRouteThreads) void moe_xu_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  moe_xu_job(a, blockIdx.x, smem, true);
}

// ---------------------------------------------------------------------------
// 2. Gate/up (two-matrix stream) for routed blocks and the shared expert
// ---------------------------------------------------------------------------
struct RoutedGateUp {
  const MoeArgs& a;
  const int* tok;  // LDS: the block's token ids
  int b, wg, e, M;
  int cg, cu, cd;  // clusters of the expert's gate, up and down projections
  __device__ int m_rows(int) const { return M; }
  __device__ const __half* xrow(int, int m) const { return a.h + (int64_t)tok[m] * a.H; }
  __device__ StreamMat mat(int, int s) const {
    return StreamMat{a.codes[s] + e * a.c_es[s], a.scales[s] + e * a.s_es[s],
                     a.zeros[s] + e * a.s_es[s], a.SV[s] ? a.SV[s] + e * a.sv_es[s] : nullptr,
                     nullptr};
  }
  __device__ __half load_a(int, int s, int m, int j) const {
    const int c = s == 0 ? cg : cu;
    const float* p = a.xu + (((int64_t)s * a.C + c) * a.sus * a.B + tok[m]) * a.rpad + j;
    return __float2half(sum_strided(p, (int64_t)a.B * a.rpad, a.sus));
  }
  __device__ const __half* post(int) const {
    return a.U[2] ? a.U[2] + cd * a.u_es[2] : nullptr;
  }
  __device__ void store_inter(int, int m, int n, __half v) const {
    a.inter[((int64_t)b * kMoeTB + m) * a.I + n] = v;
  }
  __device__ void store_post(int, int m, int j, float v) const {
    const long long q = llrintf(v * kAdqScale);
    atomicAdd(a.adq + ((int64_t)b * kMoeTB + m) * a.rpad + j, (unsigned long long)q);
  }
  __device__ void store(int, int, int, float) const {}
};

struct SharedGateUp {
  const MoeArgs& a;
  int sb;
  __device__ int m_rows(int) const { return min(a.stb, a.B - sb * a.stb); }
  __device__ const __half* xrow(int, int m) const {
    return a.h + (int64_t)(sb * a.stb + m) * a.H;
  }
  __device__ StreamMat mat(int, int s) const {
    return StreamMat{a.scodes[s], a.sscales[s], a.szeros[s], nullptr, nullptr};
  }
  __device__ __half load_a(int, int, int, int) const { return __float2half(0.f); }
  __device__ const __half* post(int) const { return nullptr; }
  __device__ void store_inter(int, int m, int n, __half v) const {
    a.sinter[(int64_t)(sb * a.stb + m) * a.SI + n] = v;
  }
  __device__ void store_post(int, int, int, float) const {}
  __device__ void store(int, int, int, float) const {}
};

// Launch 1: router tiles (+ the last one's routing), the x U jobs when not
// gated, and the shared expert's gate/up, which does not depend on routing
// (workgroups past the others), so it overlaps the router; the shared down
// then runs in the gate/up launch, overlapping the routed experts.
template <int BS>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int last;
  if (a.rank > 0) {  // this step's a_down accumulators start at zero
    const int64_t nq = (int64_t)a.nbm * kMoeTB * a.rpad;
    for (int64_t i = (int64_t)blockIdx.x * kRouteThreads + threadIdx.x; i < nq;
         i += (int64_t)gridDim.x * kRouteThreads)
      a.adq[i] = 0ull;
  }
  if ((int)blockIdx.x < a.nrb) {
    moe_route_tile(a, blockIdx.x, smem);
    // arrival (glq_handoff.h): the last router workgroup builds the step's
    // routing and tables and leaves the counter at zero for the next step
    if (handoff_arrive(a.rcount, (unsigned)a.nrb, &last)) {
      moe_route_finalize(a, smem);
      if (threadIdx.x == 0) handoff_reset(a.rcount);
    }
  } else if ((int)blockIdx.x < a.nrb + a.nxu1) {
    moe_xu_job(a, blockIdx.x - a.nrb, smem, false);
  } else if constexpr (BS != 0) {
    const int id = blockIdx.x - a.nrb - a.nxu1;
    const int sb = id / a.wgsu, wg = id - sb * a.wgsu;
    const int t0 = wg * a.tpsu, t1 = min(a.shSGU.tiles, t0 + a.tpsu);
    gemv_stream_ks<BS, BS == 2 ? 2 : 1, kMoeDepth, false, BS == 2, 2>(SharedGateUp{a, sb},
                                                                     a.shSGU, 0, t0, t1, smem);
  }
}

template <int BS>
__device__ void moe_shared_down_job(const MoeArgs& a, int id, unsigned char* smem);

template <int BR, int BS>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int nr = a.nbm * a.wgu;
  if ((int)blockIdx.x < nr) {
    const int b = blockIdx.x / a.wgu, wg = blockIdx.x - b * a.wgu;
    int* tok = (int*)(smem + a.tl_off);  // [kMoeTB] tokens, expert, M, then 3E cluster ids
    int cl[3];  // cluster ids of every expert, loaded alongside the top-k ids
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int i = tid + 256 * u;
      cl[u] = (a.rank > 0 && i < 3 * a.E) ? a.clus[i / a.E][i % a.E] : 0;
    }
    {
      // the block's expert and tokens from the step's dispatch tables (all
      // four reads independent: one memory round trip)
      const int* g = a.tab;
      const int nblk = g[0], be = g[1 + b], bm = g[1 + a.nbm + b];
      const int pr = g[1 + 2 * a.nbm + b * kMoeTB + (tid & (kMoeTB - 1))];
      if (b >= nblk) return;  // uniform over the workgroup
      if (tid < kMoeTB) tok[tid] = tid < bm ? pr / a.topk : 0;
      if (tid == 0) {
        tok[kMoeTB] = be;
        tok[kMoeTB + 1] = bm;
      }
#pragma unroll
      for (int u = 0; u < 3; ++u)
        if (tid + 256 * u < 3 * a.E) tok[16 + tid + 256 * u] = cl[u];
      __syncthreads();
    }
    const int e = tok[kMoeTB], M = tok[kMoeTB + 1];
    auto clamp_c = [&](int c) { return min(max(c, 0), a.C - 1); };
    const int cg = clamp_c(tok[16 + e]), cu = clamp_c(tok[16 + a.E + e]);
    const int cd = min(max(tok[16 + 2 * a.E + e], 0), a.urows[2] - 1);  // row of U[2]
    __syncthreads();  // the tables' LDS is reused by the stream from here on
    const int t0 = wg * a.tpu, t1 = min(a.shGU.tiles, t0 + a.tpu);
    gemv_stream_ks<BR, 1, kMoeDepth, false, BR == 2, 2>(
        RoutedGateUp{a, tok, b, wg, e, M, cg, cu, cd}, a.shGU, 0, t0, t1, smem);
  } else if constexpr (BS != 0) {  // the shared expert's down (its gate/up ran in launch 1)
    moe_shared_down_job<BS>(a, blockIdx.x - nr, smem);
  }
}

// ---------------------------------------------------------------------------
// 3. Down projections (routed per block and K part; shared per token block and
//    K part)
// ---------------------------------------------------------------------------
// Shape of K part `part` of a down projection whose parts hold `kp` codes.
__device__ inline StreamShape moe_part_shape(const StreamShape& base, int Kfull, int kp,
                                             int part, int bits) {
  StreamShape s = base;
  const int k0 = part * kp;
  s.K = min(kp, Kfull - k0);
  s.nchunk = (s.K * bits / 8 + 127) / 128;
  s.goff = k0 / 128;
  s.gend = base.G - s.goff;
  s.rowlast = base.kw * 4 - k0 * bits / 8 - 16;
  return s;
}

struct RoutedDown {
  const MoeArgs& a;
  const int* pair;  // LDS: the block's pair indices (t * top_k + k)
  int b, e, M, part, k0;
  __device__ int m_rows(int) const { return M; }
  __device__ const __half* xrow(int, int m) const {
    return a.inter + ((int64_t)b * kMoeTB + m) * a.I + k0;
  }
  __device__ StreamMat mat(int, int) const {
    const int go = k0 / 128;
    return StreamMat{a.codes[2] + e * a.c_es[2] + k0 * a.bits / 32,
                     a.scales[2] + e * a.s_es[2] + go, a.zeros[2] + e * a.s_es[2] + go,
                     (part == 0 && a.SV[2]) ? a.SV[2] + e * a.sv_es[2] : nullptr, nullptr};
  }
  __device__ __half load_a(int, int, int m, int j) const {
    const long long q = (long long)a.adq[((int64_t)b * kMoeTB + m) * a.rpad + j];
    return __float2half((float)((double)q * (1.0 / kAdqScale)));
  }
  __device__ void store(int, int m, int n, float v) const {
    a.yb[((int64_t)part * a.B * a.topk + pair[m]) * a.H + n] = v;
  }
};

struct SharedDown {
  const MoeArgs& a;
  int sb, part, k0;
  __device__ int m_rows(int) const { return min(a.stb, a.B - sb * a.stb); }
  __device__ const __half* xrow(int, int m) const {
    return a.sinter + (int64_t)(sb * a.stb + m) * a.SI + k0;
  }
  __device__ StreamMat mat(int, int) const {
    const int go = k0 / 128;
    return StreamMat{a.scodes[2] + k0 * a.sbits / 32, a.sscales[2] + go, a.szeros[2] + go,
                     nullptr, nullptr};
  }
  __device__ __half load_a(int, int, int, int) const { return __float2half(0.f); }
  __device__ void store(int, int m, int n, float v) const {
    a.sdp[((int64_t)part * a.B + sb * a.stb + m) * a.H + n] = v;
  }
};

// The shared expert's down projection for (token block, K part, tile range)
// `id`, in the gate/up launch (its inter is ready after launch 1).
template <int BS>
__device__ void moe_shared_down_job(const MoeArgs& a, int id, unsigned char* smem) {
  const int sb = id / (a.ss * a.wgsd);
  const int rem = id - sb * a.ss * a.wgsd;
  const int part = rem / a.wgsd, wg = rem - part * a.wgsd;
  const StreamShape sh = moe_part_shape(a.shSD, a.SI, a.ks, part, BS);
  const int t0 = wg * a.tpsd, t1 = min(sh.tiles, t0 + a.tpsd);
  gemv_stream_ks<BS, BS == 2 ? 2 : 1, kMoeDepth, false, BS == 2, 1>(
      SharedDown{a, sb, part, part * a.ks}, sh, 0, t0, t1, smem);
}

template <int BR, int BS>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nr = a.nbm * a.sr * a.wgd;
  if ((int)blockIdx.x < nr) {
    const int b = blockIdx.x / (a.sr * a.wgd);
    const int rem = blockIdx.x - b * a.sr * a.wgd;
    const int part = rem / a.wgd, wg = rem - part * a.wgd;
    int e, M;
    int* pair = (int*)(smem + a.pl_off);  // past the stream layout and the tables
    {
      const int* g = a.tab;
      const int nblk = g[0];
      e = g[1 + b];
      M = g[1 + a.nbm + b];
      const int pr = g[1 + 2 * a.nbm + b * kMoeTB + (threadIdx.x & (kMoeTB - 1))];
      if (b >= nblk) return;
      if (threadIdx.x < kMoeTB) pair[threadIdx.x] = pr;
      __syncthreads();
    }
    const StreamShape sh = moe_part_shape(a.shD, a.I, a.kr, part, BR);
    const int t0 = wg * a.tpd, t1 = min(sh.tiles, t0 + a.tpd);
    gemv_stream_ks<BR, 1, kMoeDepth, false, BR == 2, 1>(
        RoutedDown{a, pair, b, e, M, part, part * a.kr}, sh, 0, t0, t1, smem);
  }
}

// ---------------------------------------------------------------------------
// 4. Combine: out[t] = fp16(sum_k w_tk y_(t,k) + gate_t * fp16(shared_t))
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeArgs a) {
  const int nb = (a.H + 255) / 256;
  const int t = blockIdx.x / nb;
  const int n = (blockIdx.x - t * nb) * 256 + threadIdx.x;
  if (n >= a.H) return;
  const int P = a.B * a.topk;
  float acc = 0.f;
  for (int k = 0; k < a.topk; ++k) {
    const int p = t * a.topk + k;
    float y = 0.f;
    for (int part = 0; part < a.sr; ++part) y += a.yb[((int64_t)part * P + p) * a.H + n];
    acc = fmaf(__half2float(a.wts[p]), y, acc);
  }
  if (a.SI > 0) {
    float s = 0.f;
    for (int part = 0; part < a.ss; ++part) s += a.sdp[((int64_t)part * a.B + t) * a.H + n];
    acc = fmaf(__half2float(a.sg[t]), __half2float(__float2half(s)), acc);
  }
  float o = __half2float(__float2half(acc));
  if (a.res) o += __half2float(a.res[(int64_t)t * a.H + n]);  // the layer's residual add
  a.out[(int64_t)t * a.H + n] = __float2half(o);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct MoePlan {
  MoeArgs a;
  int64_t ws_need;
  size_t lds_route, lds_xu, lds_gu, lds_d, lds_c, lds_shgu, lds_shd;
  int64_t grid_route, grid_xu, grid_gu, grid_d, grid_c;
  bool xu_gated;  // x U jobs in their own launch, gated on routing
  int64_t off_rcnt, off_tab, off_sel, off_lgb, off_wts, off_sg, off_xu, off_inter, off_adq, off_sinter, off_yb, off_sdp;
};

StreamShape moe_stream_shape(int K, int N, int bits, int rank, int mmax, int kpart) {
  StreamShape s;
  s.K = kpart;
  s.N = N;
  s.G = K / 128;
  s.rank = rank;
  s.rpad = (int)align_up(rank, 32);
  s.sym = 0;
  s.zoff = 0.f;
  s.kw = K * bits / 32;
  s.nchunk = (kpart * bits / 8 + 127) / 128;
  s.nsvc = rank > 0 ? (rank + 63) / 64 : 0;
  s.tiles = (N + 15) / 16;
  s.xstride = stream_kpad(kpart, bits) + 8;
  s.mmax = mmax;
  s.apad = 64 * (s.nsvc > 0 ? s.nsvc : 1) + 8;
  s.goff = 0;
  s.gend = s.G;
  s.rowlast = s.kw * 4 - 16;
  return s;
}

// K parts of a down projection: the fewest parts whose x slice (mmax rows)
// fits the staging budget and whose codes fit kMoeMaxChunks chunks per row
// (a wave's serial work per tile); parts hold whole chunks.
void moe_ksplit(int K, int mmax, int bits, int& parts, int& kp) {
  const int unit = bits == 2 ? 512 : 256;  // codes per 128-byte chunk
  int cap = kMoeXBudget / (2 * mmax) / unit * unit;
  cap = std::min(cap, kMoeMaxChunks * unit);
  if (cap < unit) cap = unit;
  parts = (K + cap - 1) / cap;
  kp = (int)align_up((K + parts - 1) / parts, unit);
  parts = (K + kp - 1) / kp;
}

// Tiles per workgroup (all four waves work on each tile): as few as keep the
// launch near kMoeTargetWgs workgroups, so small batches spread over the chip
// and large ones amortise each workgroup's prologue.
constexpr int64_t kMoeTargetWgs = 768;
int moe_tiles_per_wg(int64_t units, int tiles) {
  const int64_t t = (units * tiles + kMoeTargetWgs - 1) / kMoeTargetWgs;
  return (int)std::max<int64_t>(1, std::min<int64_t>(tiles, t));
}

int stream_slot_bytes(int bits) { return stream_slot<true>() - (bits == 2 ? 0 : 256); }

int moe_plan(const glq_moe_params* p, MoePlan& P) {
  GLQ_CHECK(p != nullptr, "null params");
  const int64_t B = p->tokens, H = p->hidden, E = p->experts, I = p->inter, k = p->top_k;
  const int64_t C = p->n_clusters, SI = p->shared_inter;
  const bool lora = p->rank > 0 && p->SV[0] && p->SV[1] && p->SV[2];
  const int64_t r = lora ? p->rank : 0;
  GLQ_CHECK(B >= 1 && B <= kMoeMaxB, "tokens=%lld must be in 1..%d", (long long)B, kMoeMaxB);
  GLQ_CHECK(E >= 1 && E <= kMoeMaxE, "experts=%lld must be in 1..%d", (long long)E, kMoeMaxE);
  GLQ_CHECK(k >= 1 && k <= 16 && k <= E && B * k <= kMoeMaxP, "top_k=%lld out of range",
            (long long)k);
  GLQ_CHECK(p->group == 128, "group must be 128 (got %d)", p->group);
  GLQ_CHECK(p->bits == 2 || p->bits == 4, "bits must be 2 or 4");
  GLQ_CHECK(SI == 0 || p->shared_bits == 2 || p->shared_bits == 4,
            "shared_bits must be 2 or 4");
  GLQ_CHECK(H >= 256 && H % 256 == 0 && H <= (1 << 16), "hidden=%lld must be a multiple of 256",
            (long long)H);
  GLQ_CHECK(I >= 128 && I % 128 == 0 && I <= (1 << 17), "inter=%lld must be a multiple of 128",
            (long long)I);
  GLQ_CHECK(SI >= 0 && SI % 128 == 0 && SI <= (1 << 17),
            "shared_inter=%lld must be a multiple of 128", (long long)SI);
  if (lora) {
    GLQ_CHECK(r % 8 == 0 && r <= 128, "rank=%lld must be a multiple of 8, <= 128", (long long)r);
    GLQ_CHECK(C >= 1, "n_clusters must be >= 1 with a rank");
    for (int s = 0; s < 3; ++s) {
      GLQ_CHECK(p->U[s] && p->cluster_of[s], "U and cluster_of are needed with a rank");
      GLQ_CHECK(p->u_rows[s] >= 0 && p->u_rows[s] < (1ll << 24), "u_rows out of range");
    }
  }
  GLQ_CHECK(p->h && p->router_w && p->out, "null h, router_w or out");
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  GLQ_CHECK(al16(p->h) && al16(p->router_w) && (!p->shared_gate_w || al16(p->shared_gate_w)),
            "h and router weights must be 16-byte aligned");
  for (int s = 0; s < 3; ++s) {
    GLQ_CHECK(p->codes[s] && p->scales[s] && p->zeros[s], "null routed weights (proj %d)", s);
    GLQ_CHECK(al16(p->codes[s]) && (!lora || (al16(p->U[s]) && al16(p->SV[s]))),
              "codes, U and SV must be 16-byte aligned");
    if (SI > 0)
      GLQ_CHECK(p->shared_codes[s] && p->shared_scales[s] && p->shared_zeros[s] &&
                    al16(p->shared_codes[s]),
                "null or unaligned shared-expert weights (proj %d)", s);
  }

  MoeArgs& a = P.a;
  memset(&a, 0, sizeof(a));
  a.B = (int)B; a.H = (int)H; a.E = (int)E; a.I = (int)I; a.topk = (int)k;
  a.norm = p->norm_topk_prob ? 1 : 0;
  a.C = lora ? (int)C : 1;
  a.rank = (int)r;
  a.rpad = (int)align_up(r > 0 ? r : 1, 32);
  a.SI = (int)SI;
  a.bits = p->bits;
  a.sbits = SI > 0 ? p->shared_bits : 0;
  const int P_ = (int)(B * k);
  a.nbm = (int)std::min<int64_t>(E, P_) + P_ / kMoeTB;
  // U rows per x U job: gated steps (few picked clusters, many idle jobs)
  // and larger batches take short slices, small ungated batches longer ones
  a.xurows = (a.rank <= 64 && B <= 16 && !(lora && a.C > 4 * P_)) ? 512 : 256;
  a.sus = (int)((H + a.xurows - 1) / a.xurows);
  const int mr = (int)std::min<int64_t>(B, kMoeTB);  // staged rows per routed block
  // gate/up: K = H, N = I
  a.nrb = (int)(((E + (p->shared_gate_w ? 1 : 0) + 15) / 16) * ((B + 15) / 16));
  a.shGU = moe_stream_shape((int)H, (int)I, a.bits, a.rank, mr, (int)H);
  a.tpu = moe_tiles_per_wg(a.nbm, a.shGU.tiles);
  a.wgu = (a.shGU.tiles + a.tpu - 1) / a.tpu;
  // routed down: K = I (K parts), N = H
  moe_ksplit((int)I, mr, a.bits, a.sr, a.kr);
  a.shD = moe_stream_shape((int)I, (int)H, a.bits, a.rank, mr, a.kr);
  a.tpd = moe_tiles_per_wg((int64_t)a.nbm * a.sr, a.shD.tiles);
  a.wgd = (a.shD.tiles + a.tpd - 1) / a.tpd;
  if (SI > 0) {
    a.stb = a.sbits == 2 ? 16 : 16;
    a.stb = (int)std::min<int64_t>(B, a.stb);
    a.nsb = (int)((B + a.stb - 1) / a.stb);
    a.shSGU = moe_stream_shape((int)H, (int)SI, a.sbits, 0, a.stb, (int)H);
    a.tpsu = moe_tiles_per_wg(a.nsb, a.shSGU.tiles);
    a.wgsu = (a.shSGU.tiles + a.tpsu - 1) / a.tpsu;
    moe_ksplit((int)SI, a.stb, a.sbits, a.ss, a.ks);
    a.shSD = moe_stream_shape((int)SI, (int)H, a.sbits, 0, a.stb, a.ks);
    a.tpsd = moe_tiles_per_wg((int64_t)a.nsb * a.ss, a.shSD.tiles);
    a.wgsd = (a.shSD.tiles + a.tpsd - 1) / a.tpsd;
  }
  // LDS
  const int tbl = moe_tables_words(P_, (int)E, a.nbm) * 4;
  const int pcols = a.rank > 0 ? 64 * a.shGU.nsvc : 0;
  const StreamLds Lgu = stream_lds(kMoeDepth, stream_slot_bytes(a.bits), mr, (int)H, a.bits,
                                   a.shGU.xstride, a.shGU.apad, 2, pcols);
  // the block's token list sits past the stream layout (with its K-split
  // partial tiles)
  a.tl_off = (int)align_up(Lgu.total + stream_ks_bytes(2), 16);
  size_t lgu = (size_t)a.tl_off + 16 * 4 + 3 * 4 * (size_t)E;
  const StreamLds Ld = stream_lds(kMoeDepth, stream_slot_bytes(a.bits), mr, a.kr, a.bits,
                                  a.shD.xstride, a.shD.apad, 1, 0);
  size_t ld = Ld.total + stream_ks_bytes(1);
  a.pl_off = (int)align_up(ld, 16);  // the routed block's pair list
  ld = a.pl_off + 16 * 4;
  P.lds_shgu = 0;
  P.lds_shd = 0;
  if (SI > 0) {
    const StreamLds Ls = stream_lds(kMoeDepth, stream_slot_bytes(a.sbits), a.stb, (int)H,
                                    a.sbits, a.shSGU.xstride, a.shSGU.apad, 2, 0);
    P.lds_shgu = Ls.total + stream_ks_bytes(2);  // in the router's launch
    const StreamLds Lsd = stream_lds(kMoeDepth, stream_slot_bytes(a.sbits), a.stb, a.ks,
                                     a.sbits, a.shSD.xstride, a.shSD.apad, 1, 0);
    P.lds_shd = Lsd.total + stream_ks_bytes(1);
  }
  lgu = std::max(lgu, P.lds_shd);  // the shared down runs in the gate/up launch
  GLQ_CHECK(lgu <= 160 * 1024 && ld <= 160 * 1024, "MoE shapes exceed the LDS budget");
  P.lds_gu = lgu;
  P.lds_d = ld;
  P.lds_c = 0;
  {
    const size_t router = (size_t)16 * (H + 8) * 2 + (size_t)4 * 256 * 4;
    const size_t xu = (size_t)align_up(B * (a.xurows + 8) * 2, 16) +
                      (size_t)a.xurows * (a.rank + 8) * 2;
    P.lds_route = std::max(router, lora ? xu : (size_t)0);
    // the router's last workgroup stages B rows of routing keys and the tables
    P.lds_route = std::max(P.lds_route, (size_t)align_up(4 * B * moe_lg_stride((int)E), 16) +
                                            (size_t)tbl + 4 * (2 * (size_t)a.C + 2));
    P.lds_route = std::max(P.lds_route, P.lds_shgu);  // the shared gate/up runs here
    // the gated jobs stage B rows of routing keys first
    P.lds_xu = std::max(xu, (size_t)4 * B * moe_lg_stride((int)E));
    GLQ_CHECK(std::max(P.lds_route, P.lds_xu) <= 160 * 1024,
              "hidden=%lld with %lld tokens exceeds the router's LDS budget", (long long)H,
              (long long)B);
  }
  // grids
  // x U jobs gated on routing (a launch of their own) when the clusters
  // outnumber four times the (token, expert) picks, i.e. when most clusters
  // of a step go unpicked; GLQ_MOE_XU_GATE=0/1 forces either form
  P.xu_gated = lora && a.C > 4 * P_;
  if (const char* g = getenv("GLQ_MOE_XU_GATE")) P.xu_gated = lora && atoi(g) != 0;
  a.nxu1 = lora && !P.xu_gated ? 2 * a.C * a.sus : 0;
  a.nxc = P.xu_gated ? std::min(a.C, P_) : 0;
  P.grid_route = a.nrb + a.nxu1 + (SI > 0 ? (int64_t)a.nsb * a.wgsu : 0);
  P.grid_xu = lora ? 2 * (int64_t)a.nxc * a.sus : 0;
  P.grid_gu = (int64_t)a.nbm * a.wgu + (SI > 0 ? (int64_t)a.nsb * a.ss * a.wgsd : 0);
  P.grid_d = (int64_t)a.nbm * a.sr * a.wgd;
  P.grid_c = B * ((H + 255) / 256);
  // workspace
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  P.off_rcnt = take(4);  // must be zero before the first step; every step leaves it zero
  o = kMoeWsHeader;      // the rest of the header: the lane path's counters
  // (the picked-cluster lists are sized whether or not this step is gated,
  // so the workspace size does not depend on the form)
  P.off_tab = take(4 * (1 + (2 + kMoeTB) * (int64_t)a.nbm + 2 + 2 * std::min<int64_t>(a.C, P_)));
  P.off_sel = take(4 * P_);
  P.off_lgb = take(2 * B * E);
  P.off_wts = take(2 * P_);
  P.off_sg = take(2 * B);
  P.off_xu = take(lora ? 4 * 2 * a.C * a.sus * B * a.rpad : 0);
  P.off_inter = take(2 * (int64_t)a.nbm * kMoeTB * I);
  P.off_adq = take(lora ? 8 * (int64_t)a.nbm * kMoeTB * a.rpad : 0);
  P.off_sinter = take(2 * B * SI);
  P.off_yb = take(4 * (int64_t)a.sr * P_ * H);
  P.off_sdp = take(SI > 0 ? 4 * (int64_t)a.ss * B * H : 0);
  P.ws_need = o;

  a.h = (const __half*)p->h;
  a.rw = (const __half*)p->router_w;
  a.sgw = (const __half*)p->shared_gate_w;
  const int64_t NK[3][2] = {{I, H}, {I, H}, {H, I}};  // (N, K) per projection
  for (int s = 0; s < 3; ++s) {
    const int64_t N = NK[s][0], K = NK[s][1];
    a.codes[s] = (const uint32_t*)p->codes[s];
    a.scales[s] = (const __half*)p->scales[s];
    a.zeros[s] = (const __half*)p->zeros[s];
    a.c_es[s] = N * K * a.bits / 32;
    a.s_es[s] = N * (K / 128);
    a.U[s] = lora ? (const __half*)p->U[s] : nullptr;
    a.u_es[s] = K * r;
    a.clus[s] = lora ? p->cluster_of[s] : nullptr;
    if (s < 2) a.uslot[s] = lora ? p->u_slot[s] : nullptr;
    a.urows[s] = (int)(p->u_rows[s] > 0 ? p->u_rows[s] : C);
    a.SV[s] = lora ? (const __half*)p->SV[s] : nullptr;
    a.sv_es[s] = N * r;
    a.scodes[s] = SI > 0 ? (const uint32_t*)p->shared_codes[s] : nullptr;
    a.sscales[s] = SI > 0 ? (const __half*)p->shared_scales[s] : nullptr;
    a.szeros[s] = SI > 0 ? (const __half*)p->shared_zeros[s] : nullptr;
  }
  a.out = (__half*)p->out;
  a.res = (const __half*)p->residual;
  a.logits = (__half*)p->router_logits;
  return GLQ_OK;
}

template <int BR, int BS>
int moe_launch(MoePlan& P, hipStream_t s) {
  static size_t attr_gu = 64 * 1024, attr_d = 64 * 1024, attr_c = 64 * 1024;
  static size_t attr_r = 64 * 1024, attr_x = 64 * 1024;
  const MoeArgs& a = P.a;
  int rc = set_lds_limit(moe_route_kernel<BS>, P.lds_route, attr_r);
  if (rc) return rc;
  moe_route_kernel<BS><<<dim3((unsigned)P.grid_route), dim3(kRouteThreads), P.lds_route, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_route_kernel");
  if (P.xu_gated) {
    rc = set_lds_limit(moe_xu_kernel, P.lds_xu, attr_x);
    if (rc) return rc;
    moe_xu_kernel<<<dim3((unsigned)P.grid_xu), dim3(kRouteThreads), P.lds_xu, s>>>(a);
    GLQ_LAUNCH_CHECK("moe_xu_kernel");
  }
  rc = set_lds_limit(moe_gate_up_kernel<BR, BS>, P.lds_gu, attr_gu);
  if (rc) return rc;
  moe_gate_up_kernel<BR, BS><<<dim3((unsigned)P.grid_gu), dim3(256), P.lds_gu, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_gate_up_kernel");
  rc = set_lds_limit(moe_down_kernel<BR, BS>, P.lds_d, attr_d);
  if (rc) return rc;
  moe_down_kernel<BR, BS><<<dim3((unsigned)P.grid_d), dim3(256), P.lds_d, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_down_kernel");
  rc = set_lds_limit(moe_combine_kernel, P.lds_c, attr_c);
  if (rc) return rc;
  moe_combine_kernel<<<dim3((unsigned)P.grid_c), dim3(256), P.lds_c, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_combine_kernel");
  return GLQ_OK;
}

}  // namespace
}  // namespace glq

namespace glq {
// A step of kMoeLaneMaxB < B <= kMoeLaneChunkMax tokens with few tokens per
// expert (B top_k <= 4 E) runs as consecutive lane steps of at most
// kMoeLaneMaxB tokens (routing and the combine are per token, so the chunks
// give the same results as one step would).  Measured: config 2 at 20 / 32
// tokens 179 -> 124 / 222 -> 145 us; config 3 at 32 tokens (8 per expert)
// stays on the many-token path (585 us there, 608 chunked).
constexpr int64_t kMoeLaneChunkMax = 32;

// The parameters of tokens [t0, t0 + n) of a step.
glq_moe_params moe_chunk(const glq_moe_params* p, int64_t t0, int64_t n) {
  glq_moe_params q = *p;
  q.tokens = n;
  q.h = (const char*)p->h + t0 * p->hidden * 2;
  q.out = (char*)p->out + t0 * p->hidden * 2;
  if (p->residual) q.residual = (const char*)p->residual + t0 * p->hidden * 2;
  if (p->router_logits) q.router_logits = (char*)p->router_logits + t0 * p->experts * 2;
  return q;
}

// Workspace bytes of the chunked lane form, or -1 when the step does not take it.
int64_t moe_chunked_lane_bytes(const glq_moe_params* p) {
  if (p->tokens <= kMoeLaneMaxB || p->tokens > kMoeLaneChunkMax ||
      p->tokens * p->top_k > 4 * p->experts || getenv("GLQ_MOE_NO_CHUNK"))
    return -1;
  int64_t need = 0;
  for (int64_t t0 = 0; t0 < p->tokens; t0 += kMoeLaneMaxB) {
    const glq_moe_params q = moe_chunk(p, t0, std::min<int64_t>(kMoeLaneMaxB, p->tokens - t0));
    const int64_t b = moe_lane_workspace_bytes(&q);
    if (b < 0) return -1;
    need = std::max(need, b);
  }
  return need;
}
}  // namespace glq

extern "C" int64_t glq_moe_workspace_bytes(const glq_moe_params* p) {
  glq::clear_error();
  glq::MoePlan P;
  if (glq::moe_plan(p, P) != GLQ_OK) return -1;
  const int64_t lane = glq::moe_lane_workspace_bytes(p);  // the path glq_moe_decode takes
  if (lane >= 0) return lane;
  const int64_t chunked = glq::moe_chunked_lane_bytes(p);
  return chunked >= 0 ? chunked : P.ws_need;
}

extern "C" int glq_moe_decode(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  using namespace glq;
  clear_error();
  MoePlan P;
  int rc = moe_plan(p, P);
  if (rc) return rc;
  if (moe_lane_workspace_bytes(p) >= 0)  // a few tokens: the lane path
    return moe_lane_decode(p, workspace, workspace_bytes, (hipStream_t)stream);
  if (moe_chunked_lane_bytes(p) >= 0) {  // up to kMoeLaneChunkMax: lane steps in turn
    for (int64_t t0 = 0; t0 < p->tokens; t0 += kMoeLaneMaxB) {
      const glq_moe_params q = moe_chunk(p, t0, std::min<int64_t>(kMoeLaneMaxB, p->tokens - t0));
      rc = moe_lane_decode(&q, workspace, workspace_bytes, (hipStream_t)stream);
      if (rc) return rc;
    }
    return GLQ_OK;
  }
  GLQ_CHECK(workspace != nullptr && workspace_bytes >= P.ws_need,
            "workspace of %lld bytes needed (got %lld)", (long long)P.ws_need,
            (long long)workspace_bytes);
  GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  char* w = (char*)workspace;
  MoeArgs& a = P.a;
  a.rcount = (unsigned*)(w + P.off_rcnt);
  a.tab = (int*)(w + P.off_tab);
  a.sel = (int32_t*)(w + P.off_sel);
  a.lgb = (__half*)(w + P.off_lgb);
  a.wts = (__half*)(w + P.off_wts);
  a.sg = (__half*)(w + P.off_sg);
  a.xu = (float*)(w + P.off_xu);
  a.inter = (__half*)(w + P.off_inter);
  a.adq = (unsigned long long*)(w + P.off_adq);
  a.sinter = (__half*)(w + P.off_sinter);
  a.yb = (float*)(w + P.off_yb);
  a.sdp = (float*)(w + P.off_sdp);
  hipStream_t s = (hipStream_t)stream;
  const int br = a.bits, bs = a.sbits;
  if (br == 2 && bs == 4) return moe_launch<2, 4>(P, s);
  if (br == 2 && bs == 0) return moe_launch<2, 0>(P, s);
  if (br == 2 && bs == 2) return moe_launch<2, 2>(P, s);
  if (br == 4 && bs == 4) return moe_launch<4, 4>(P, s);
  if (br == 4 && bs == 0) return moe_launch<4, 0>(P, s);
  return moe_launch<4, 2>(P, s);
}
