// MoE block decode step on MI355X: GraphCompatibleMoeBlock.forward
// (inference/moe_block.py:381-436) for B <= 64 tokens, in four launches with
// all routing on the device (no host sync, so the step captures in a hipGraph):
//
//  1. moe_route_kernel: one workgroup per token computes the router logits
//     (fp32 sums rounded to fp16), fp32 softmax, top-k with optional
//     renormalisation (moe_block.py:386-392) and the shared-expert gate; the
//     other workgroups form K-sliced fp32 partials of x U_c for every cluster
//     c of gate and up (the cluster-shared precompute, moe_block.py:290-322).
//  2. moe_gate_up_kernel: every workgroup rebuilds the dispatch tables from
//     the top-k ids (expert-major pair lists cut into blocks of <= 8 tokens)
//     and runs gate and up of one block's expert over a range of 16-row tiles
//     in one pass (two-matrix stream), writing inter = fp16(silu(g) * u) and
//     the workgroup's partial of a_down = inter U_down[c(e)]; workgroups past
//     the routed blocks run the shared expert's gate/up the same way.
//  3. moe_down_kernel: routed down projections per (block, K part) with the
//     low-rank term from the summed a_down partials, and the shared expert's
//     down projection per (token block, K part); fp32 partial outputs.
//  4. moe_combine_kernel: out = fp16(sum_k w_k y_k + sigmoid-gate * fp16(shared)).
//
// Only the selected experts' weights are read (the reference's graph mode
// reads all E, moe_block.py:742-890), and a cluster's U is read once per step
// for all of its experts.  No atomics: every sum has a fixed order.
#include <algorithm>
#include <cstring>

#include "glq_stream.h"

namespace glq {

constexpr int kMoeTB = 8;          // tokens per routed block (one MFMA pass for 2-bit)
constexpr int kMoeDepth = 3;       // ring slots per wave
constexpr int kMoeMaxE = 256;
constexpr int kMoeMaxP = 512;      // tokens * top_k
constexpr int kMoeMaxB = 64;
constexpr int kMoeXBudget = 48 * 1024;  // bytes of staged x per down-projection unit

struct MoeArgs {
  int B, H, E, I, topk, norm, C, rank, rpad, SI;
  int nbm;     // routed token blocks the grids are sized for
  int sus;     // K-slices of the gate/up x U partials
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
  float* adp;      // [nbm][wgu][TB][rpad] a_down partials
  __half* sinter;  // [B][SI]
  float* yb;       // [sr][nbm][TB][H] routed down outputs (fp32)
  float* sdp;      // [ss][B][H] shared down partial outputs (fp32)
  __half* out;
  __half* logits;
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
__device__ int moe_dispatch(const MoeArgs& a, const MoeTables& t) {
  const int P = a.B * a.topk, E = a.E, tid = threadIdx.x;
  for (int i = tid; i < P; i += 256) {
    const int e = a.sel[i];
    t.sel[i] = (e >= 0 && e < E) ? e : -1;
  }
  __syncthreads();
  for (int e = tid; e < E; e += 256) {
    int c = 0;
    for (int p = 0; p < P; ++p) c += t.sel[p] == e;
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
    for (int q = 0; q < p; ++q) r += t.sel[q] == e;
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

__device__ __forceinline__ int moe_cluster(const MoeArgs& a, int s, int e) {
  const int c = a.clus[s][e];
  return min(max(c, 0), a.C - 1);
}

// ---------------------------------------------------------------------------
// 1. Router + gate/up cluster partials
// ---------------------------------------------------------------------------
__device__ void moe_route_token(const MoeArgs& a, int t, float* lg) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const __half* hr = a.h + (int64_t)t * a.H;
  const int nrow = a.E + (a.sgw ? 1 : 0);
  for (int e = wave; e < nrow; e += 4) {
    const __half* wr = e < a.E ? a.rw + (int64_t)e * a.H : a.sgw;
    float acc = 0.f;
    for (int k = 8 * lane; k < a.H; k += 512) {
      const f16x8 hv = *(const f16x8*)(hr + k);
      const f16x8 wv = *(const f16x8*)(wr + k);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc = fmaf((float)hv[c], (float)wv[c], acc);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) acc += __shfl_xor(acc, d);
    if (lane == 0) lg[e] = __half2float(__float2half(acc));  // fp16 logits
  }
  __syncthreads();
  if (wave != 0) return;
  // softmax over E in fp32 (lane holds experts lane + 64i)
  float v[4], pr[4];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < a.E ? lg[e] : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) mx = fmaxf(mx, __shfl_xor(mx, d));
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pr[i] = lane + 64 * i < a.E ? expf(v[i] - mx) : 0.f;
    sum += pr[i];
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d);
#pragma unroll
  for (int i = 0; i < 4; ++i) pr[i] = lane + 64 * i < a.E ? pr[i] / sum : -1.f;
  // top-k: k rounds of (largest probability, lowest index)
  float wk = 0.f, wsum = 0.f;
  int ek = 0;
  for (int k = 0; k < a.topk; ++k) {
    float bv = -2.f;
    int bi = 1 << 30;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (pr[i] > bv) {  // ascending index within the lane: strict > keeps the lowest
        bv = pr[i];
        bi = lane + 64 * i;
      }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const float ov = __shfl_xor(bv, d);
      const int oi = __shfl_xor(bi, d);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + 64 * i == bi) pr[i] = -1.f;
    if (lane == k) {
      wk = bv;
      ek = bi;
    }
    wsum += bv;
  }
  if (lane < a.topk) {
    const float w = a.norm ? wk / wsum : wk;
    a.sel[t * a.topk + lane] = ek;
    a.wts[t * a.topk + lane] = __float2half(w);
  }
  if (a.logits)
    for (int e = lane; e < a.E; e += 64) a.logits[(int64_t)t * a.E + e] = __float2half(lg[e]);
  if (lane == 0)
    a.sg[t] = a.sgw ? __float2half(1.f / (1.f + expf(-lg[a.E]))) : __float2half(1.f);
}

__global__ __launch_bounds__(256) void moe_route_kernel(MoeArgs a) {
  __shared__ float lg[kMoeMaxE + 1];
  __shared__ float red[4 * 4 * 64];
  __shared__ __half xl[16 * kLowrankRows];
  if ((int)blockIdx.x < a.B) {
    moe_route_token(a, blockIdx.x, lg);
    return;
  }
  // x U_c partials: (projection s in {gate, up}, cluster c, K-slice q)
  const int id = blockIdx.x - a.B;
  const int s = id / (a.C * a.sus), rem = id - s * a.C * a.sus;
  const int c = rem / a.sus, q = rem - c * a.sus;
  const __half* U = a.U[s] + (int64_t)c * a.u_es[s];
  for (int m0 = 0; m0 < a.B; m0 += 16) {
    const int M = min(16, a.B - m0);
    auto xrow = [&](int m) { return a.h + (int64_t)(m0 + m) * a.H; };
    float* out = a.xu + ((((int64_t)s * a.C + c) * a.sus + q) * a.B + m0) * a.rpad;
    if (M == 1)
      lowrank_partial<1>(xrow, M, a.H, a.rank, a.rpad, U, q, out, red, xl);
    else if (M == 2)
      lowrank_partial<2>(xrow, M, a.H, a.rank, a.rpad, U, q, out, red, xl);
    else
      lowrank_partial<4>(xrow, M, a.H, a.rank, a.rpad, U, q, out, red, xl);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// 2. Gate/up (two-matrix stream) for routed blocks and the shared expert
// ---------------------------------------------------------------------------
struct RoutedGateUp {
  const MoeArgs& a;
  const int* tok;  // LDS: the block's token ids
  int b, wg, e, M;
  __device__ int m_rows(int) const { return M; }
  __device__ const __half* xrow(int, int m) const { return a.h + (int64_t)tok[m] * a.H; }
  __device__ StreamMat mat(int, int s) const {
    return StreamMat{a.codes[s] + e * a.c_es[s], a.scales[s] + e * a.s_es[s],
                     a.zeros[s] + e * a.s_es[s], a.SV[s] ? a.SV[s] + e * a.sv_es[s] : nullptr,
                     nullptr};
  }
  __device__ __half load_a(int, int s, int m, int j) const {
    const int c = moe_cluster(a, s, e);
    const float* p = a.xu + (((int64_t)s * a.C + c) * a.sus * a.B + tok[m]) * a.rpad + j;
    float v = 0.f;
    for (int q = 0; q < a.sus; ++q) v += p[(int64_t)q * a.B * a.rpad];
    return __float2half(v);
  }
  __device__ const __half* post(int) const {
    return a.U[2] ? a.U[2] + moe_cluster(a, 2, e) * a.u_es[2] : nullptr;
  }
  __device__ void store_inter(int, int m, int n, __half v) const {
    a.inter[((int64_t)b * kMoeTB + m) * a.I + n] = v;
  }
  __device__ void store_post(int, int m, int j, float v) const {
    a.adp[(((int64_t)b * a.wgu + wg) * kMoeTB + m) * a.rpad + j] = v;
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

template <int BR, int BS>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x;
  const int nr = a.nbm * a.wgu;
  if ((int)blockIdx.x < nr) {
    const int b = blockIdx.x / a.wgu, wg = blockIdx.x - b * a.wgu;
    int* tok = (int*)(smem + a.tl_off);
    {
      const MoeTables t = moe_tables((int*)smem, a.B * a.topk, a.E, a.nbm);
      const int nblk = moe_dispatch(a, t);
      if (b >= nblk) return;  // uniform over the workgroup
      if (tid < kMoeTB) {
        const int M = t.bM[b];
        tok[tid] = tid < M ? t.list[t.bfirst[b] + tid] / a.topk : 0;
      }
      if (tid == 0) {
        tok[kMoeTB] = t.bexp[b];
        tok[kMoeTB + 1] = t.bM[b];
      }
      __syncthreads();
    }
    const int e = tok[kMoeTB], M = tok[kMoeTB + 1];
    __syncthreads();  // the tables' LDS is reused by the stream from here on
    const int t0 = wg * a.tpu, t1 = min(a.shGU.tiles, t0 + a.tpu);
    gemv_stream<BR, 1, kMoeDepth, false, BR == 2, 2>(RoutedGateUp{a, tok, b, wg, e, M}, a.shGU,
                                                    0, t0, t1, smem);
  } else if constexpr (BS != 0) {
    const int id = blockIdx.x - nr;
    const int sb = id / a.wgsu, wg = id - sb * a.wgsu;
    const int t0 = wg * a.tpsu, t1 = min(a.shSGU.tiles, t0 + a.tpsu);
    gemv_stream<BS, BS == 2 ? 2 : 1, kMoeDepth, false, BS == 2, 2>(SharedGateUp{a, sb}, a.shSGU,
                                                                  0, t0, t1, smem);
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
    const float* p = a.adp + ((int64_t)b * a.wgu * kMoeTB + m) * a.rpad + j;
    float v = 0.f;
    for (int w = 0; w < a.wgu; ++w) v += p[(int64_t)w * kMoeTB * a.rpad];
    return __float2half(v);
  }
  __device__ void store(int, int m, int n, float v) const {
    a.yb[(((int64_t)part * a.nbm + b) * kMoeTB + m) * a.H + n] = v;
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

template <int BR, int BS>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nr = a.nbm * a.sr * a.wgd;
  if ((int)blockIdx.x < nr) {
    const int b = blockIdx.x / (a.sr * a.wgd);
    const int rem = blockIdx.x - b * a.sr * a.wgd;
    const int part = rem / a.wgd, wg = rem - part * a.wgd;
    int e, M;
    {
      const MoeTables t = moe_tables((int*)smem, a.B * a.topk, a.E, a.nbm);
      const int nblk = moe_dispatch(a, t);
      if (b >= nblk) return;
      e = t.bexp[b];
      M = t.bM[b];
      __syncthreads();
    }
    const StreamShape sh = moe_part_shape(a.shD, a.I, a.kr, part, BR);
    const int t0 = wg * a.tpd, t1 = min(sh.tiles, t0 + a.tpd);
    gemv_stream<BR, 1, kMoeDepth, false, BR == 2, 1>(RoutedDown{a, b, e, M, part, part * a.kr},
                                                    sh, 0, t0, t1, smem);
  } else if constexpr (BS != 0) {
    const int id = blockIdx.x - nr;
    const int sb = id / (a.ss * a.wgsd);
    const int rem = id - sb * a.ss * a.wgsd;
    const int part = rem / a.wgsd, wg = rem - part * a.wgsd;
    const StreamShape sh = moe_part_shape(a.shSD, a.SI, a.ks, part, BS);
    const int t0 = wg * a.tpsd, t1 = min(sh.tiles, t0 + a.tpsd);
    gemv_stream<BS, BS == 2 ? 2 : 1, kMoeDepth, false, BS == 2, 1>(
        SharedDown{a, sb, part, part * a.ks}, sh, 0, t0, t1, smem);
  }
}

// ---------------------------------------------------------------------------
// 4. Combine: out[t] = fp16(sum_k w_tk y_(t,k) + gate_t * fp16(shared_t))
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int t = blockIdx.x / ((a.H + 255) / 256);
  const int n = (blockIdx.x - t * ((a.H + 255) / 256)) * 256 + threadIdx.x;
  const MoeTables tb = moe_tables((int*)smem, a.B * a.topk, a.E, a.nbm);
  moe_dispatch(a, tb);
  if (n >= a.H) return;
  float acc = 0.f;
  for (int k = 0; k < a.topk; ++k) {
    const int p = t * a.topk + k, pos = tb.pos[p];
    if (pos < 0) continue;
    float y = 0.f;
    for (int part = 0; part < a.sr; ++part)
      y += a.yb[((int64_t)part * a.nbm * kMoeTB + pos) * a.H + n];
    acc = fmaf(__half2float(a.wts[p]), y, acc);
  }
  if (a.SI > 0) {
    float s = 0.f;
    for (int part = 0; part < a.ss; ++part) s += a.sdp[((int64_t)part * a.B + t) * a.H + n];
    acc = fmaf(__half2float(a.sg[t]), __half2float(__float2half(s)), acc);
  }
  a.out[(int64_t)t * a.H + n] = __float2half(acc);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct MoePlan {
  MoeArgs a;
  int64_t ws_need;
  size_t lds_gu, lds_d, lds_c;
  int64_t grid_route, grid_gu, grid_d, grid_c;
  int64_t off_sel, off_wts, off_sg, off_xu, off_inter, off_adp, off_sinter, off_yb, off_sdp;
};

StreamShape moe_stream_shape(int K, int N, int bits, int rank, int mmax, int kpart) {
  StreamShape s;
  s.K = kpart;
  s.N = N;
  s.G = K / 128;
  s.rank = rank;
  s.rpad = (int)align_up(rank, 32);
  s.sym = 0;
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

// K parts of a down projection: the fewest parts whose x slice (mmax rows,
// multiples of 256 codes) fits the staging budget.
void moe_ksplit(int K, int mmax, int& parts, int& kp) {
  int cap = kMoeXBudget / (2 * mmax) / 256 * 256;
  if (cap < 256) cap = 256;
  parts = (K + cap - 1) / cap;
  kp = (int)align_up((K + parts - 1) / parts, 256);
  parts = (K + kp - 1) / kp;
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
    for (int s = 0; s < 3; ++s)
      GLQ_CHECK(p->U[s] && p->cluster_of[s], "U and cluster_of are needed with a rank");
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
  a.sus = (int)((H + kLowrankRows - 1) / kLowrankRows);
  const int mr = (int)std::min<int64_t>(B, kMoeTB);  // staged rows per routed block
  // gate/up: K = H, N = I
  a.shGU = moe_stream_shape((int)H, (int)I, a.bits, a.rank, mr, (int)H);
  a.tpu = 4;
  a.wgu = (a.shGU.tiles + a.tpu - 1) / a.tpu;
  // routed down: K = I (K parts), N = H
  moe_ksplit((int)I, mr, a.sr, a.kr);
  a.shD = moe_stream_shape((int)I, (int)H, a.bits, a.rank, mr, a.kr);
  a.tpd = 4;
  a.wgd = (a.shD.tiles + a.tpd - 1) / a.tpd;
  if (SI > 0) {
    a.stb = a.sbits == 2 ? 16 : 16;
    a.stb = (int)std::min<int64_t>(B, a.stb);
    a.nsb = (int)((B + a.stb - 1) / a.stb);
    a.shSGU = moe_stream_shape((int)H, (int)SI, a.sbits, 0, a.stb, (int)H);
    a.tpsu = 4;
    a.wgsu = (a.shSGU.tiles + a.tpsu - 1) / a.tpsu;
    moe_ksplit((int)SI, a.stb, a.ss, a.ks);
    a.shSD = moe_stream_shape((int)SI, (int)H, a.sbits, 0, a.stb, a.ks);
    a.tpsd = 4;
    a.wgsd = (a.shSD.tiles + a.tpsd - 1) / a.tpsd;
  }
  // LDS
  const int tbl = moe_tables_words(P_, (int)E, a.nbm) * 4;
  const int pcols = a.rank > 0 ? 64 * a.shGU.nsvc : 0;
  const StreamLds Lgu = stream_lds(kMoeDepth, stream_slot_bytes(a.bits), mr, (int)H, a.bits,
                                   a.shGU.xstride, a.shGU.apad, 2, pcols);
  // the block's token list sits past both the stream layout and the tables
  a.tl_off = (int)align_up(std::max(Lgu.total, tbl), 16);
  size_t lgu = (size_t)a.tl_off + 16 * 4;
  const StreamLds Ld = stream_lds(kMoeDepth, stream_slot_bytes(a.bits), mr, a.kr, a.bits,
                                  a.shD.xstride, a.shD.apad, 1, 0);
  size_t ld = std::max<size_t>(Ld.total, tbl);
  if (SI > 0) {
    const StreamLds Ls = stream_lds(kMoeDepth, stream_slot_bytes(a.sbits), a.stb, (int)H,
                                    a.sbits, a.shSGU.xstride, a.shSGU.apad, 2, 0);
    lgu = std::max<size_t>(lgu, Ls.total);
    const StreamLds Lsd = stream_lds(kMoeDepth, stream_slot_bytes(a.sbits), a.stb, a.ks,
                                     a.sbits, a.shSD.xstride, a.shSD.apad, 1, 0);
    ld = std::max<size_t>(ld, Lsd.total);
  }
  GLQ_CHECK(lgu <= 160 * 1024 && ld <= 160 * 1024, "MoE shapes exceed the LDS budget");
  P.lds_gu = lgu;
  P.lds_d = ld;
  P.lds_c = tbl;
  // grids
  P.grid_route = B + (lora ? 2 * a.C * a.sus : 0);
  P.grid_gu = (int64_t)a.nbm * a.wgu + (SI > 0 ? (int64_t)a.nsb * a.wgsu : 0);
  P.grid_d = (int64_t)a.nbm * a.sr * a.wgd + (SI > 0 ? (int64_t)a.nsb * a.ss * a.wgsd : 0);
  P.grid_c = B * ((H + 255) / 256);
  // workspace
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o = align_up(o + bytes, 256);
    return at;
  };
  P.off_sel = take(4 * P_);
  P.off_wts = take(2 * P_);
  P.off_sg = take(2 * B);
  P.off_xu = take(lora ? 4 * 2 * a.C * a.sus * B * a.rpad : 0);
  P.off_inter = take(2 * (int64_t)a.nbm * kMoeTB * I);
  P.off_adp = take(lora ? 4 * (int64_t)a.nbm * a.wgu * kMoeTB * a.rpad : 0);
  P.off_sinter = take(2 * B * SI);
  P.off_yb = take(4 * (int64_t)a.sr * a.nbm * kMoeTB * H);
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
    a.SV[s] = lora ? (const __half*)p->SV[s] : nullptr;
    a.sv_es[s] = N * r;
    a.scodes[s] = SI > 0 ? (const uint32_t*)p->shared_codes[s] : nullptr;
    a.sscales[s] = SI > 0 ? (const __half*)p->shared_scales[s] : nullptr;
    a.szeros[s] = SI > 0 ? (const __half*)p->shared_zeros[s] : nullptr;
  }
  a.out = (__half*)p->out;
  a.logits = (__half*)p->router_logits;
  return GLQ_OK;
}

template <int BR, int BS>
int moe_launch(MoePlan& P, hipStream_t s) {
  static size_t attr_gu = 64 * 1024, attr_d = 64 * 1024, attr_c = 64 * 1024;
  const MoeArgs& a = P.a;
  moe_route_kernel<<<dim3((unsigned)P.grid_route), dim3(256), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("moe_route_kernel");
  int rc = set_lds_limit(moe_gate_up_kernel<BR, BS>, P.lds_gu, attr_gu);
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

extern "C" int64_t glq_moe_workspace_bytes(const glq_moe_params* p) {
  glq::clear_error();
  glq::MoePlan P;
  if (glq::moe_plan(p, P) != GLQ_OK) return -1;
  return P.ws_need;
}

extern "C" int glq_moe_decode(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  using namespace glq;
  clear_error();
  MoePlan P;
  int rc = moe_plan(p, P);
  if (rc) return rc;
  GLQ_CHECK(workspace != nullptr && workspace_bytes >= P.ws_need,
            "workspace of %lld bytes needed (got %lld)", (long long)P.ws_need,
            (long long)workspace_bytes);
  GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  char* w = (char*)workspace;
  MoeArgs& a = P.a;
  a.sel = (int32_t*)(w + P.off_sel);
  a.wts = (__half*)(w + P.off_wts);
  a.sg = (__half*)(w + P.off_sg);
  a.xu = (float*)(w + P.off_xu);
  a.inter = (__half*)(w + P.off_inter);
  a.adp = (float*)(w + P.off_adp);
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
