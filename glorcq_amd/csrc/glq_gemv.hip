// Dense fused dequant-GEMV + low-rank correction for decode (1 <= M <= 16):
// one problem, or `items` independent problems of one shape in one launch.
//
// Launch plan (both on the caller's stream, no host sync, graph-capturable):
//   1. lowrank_partial_kernel  grid items x P   a-partials over K-slices of U
//                              (skipped when the caller passes a = x U, or
//                              there is no correction)
//   2. gemv_dense_kernel       grid items x tiles   codes -> y, + a SV^T + bias
// Launch 2 sums launch 1's P fp32 partials of a and rounds a to fp16 once,
// matching the reference's fp16 `x @ U` (inference/quantized_linear.py:344).
// Stream order replaces any cross-workgroup handshake: on gfx950 every
// agent-scope release/acquire between workgroups costs an L2 writeback or
// invalidate (the 8 XCD L2s are not coherent with each other).

#include <stdlib.h>

#include <mutex>

#include "glq_stream.h"

namespace glq {

struct DenseArgs {
  const uint32_t* codes;
  int64_t codes_es;  // int32 words between items
  const __half* scales;
  const __half* zeros;
  int64_t sz_es;
  const __half* sv;
  int64_t sv_es;
  const __half* u;
  int64_t u_es;
  const __half* bias;
  int64_t bias_es;
  const __half* x;
  int64_t x_es;
  __half* y;
  int64_t y_es;
  const __half* xu;  // caller's a (items x M x rank), or null
  int64_t xu_es;
  const float* apart;  // launch-1 partials (items x P x M x rpad), or null
  int items, M, P, tiles;
  TileShape sh;
  // routed picks (glq_lowrank_xu_routed): item i takes U row ucl[usel[i]];
  // null usel (every other launch): U of item i
  const int32_t* usel = nullptr;
  const int32_t* ucl = nullptr;
  int nsel = 0, nu = 0;
  // item i's U is U + uidx[i] * u_es (null: U + i * u_es); nuidx U matrices;
  // xu_u: the caller's a is one row block per U (item i reads xu + uidx[i] *
  // xu_es), not one per item
  const int32_t* uidx = nullptr;
  int nuidx = 0;
  bool xu_u = false;
  // apart_u: the caller's partials are one block per U (item i reads block
  // uidx[i]), not one per item
  bool apart_u = false;
  // a = x U formed in the token-tile launch (t16_xu_job): xt_jobs workgroups
  // of (item, pair of K slices) come first; item i's word xt_cnt[i] holds
  // its slices' arrivals, kXtReady once a is written, then 1 << 16 per
  // row-block workgroup that has read it; zero between launches
  int xt_jobs = 0;
  int xt_rb = 0;             // row blocks an item (its readers)
  unsigned* xt_cnt = nullptr;
  float* xt_part = nullptr;  // (items, P, M, rpad) slice partials
  __half* xt_a = nullptr;    // (items, M, rank)
  uint64_t xt_spin = 0;
  // a = x U of the one-token lane launch handed over by xj jobs an item
  // (lane_xj_job: K slices of kLowrankRows rows) in front of the grid, into
  // xt_part (items, xj, rank) as bit-inverted words (0: not yet written);
  // xt_cnt[i] counts the jobs (1 each) and the row workgroups (xt_rb an
  // item, 1 << 16 each) done with item i's words, and the last of them
  // clears the words: both zero between launches.  xj = 0: every row
  // workgroup forms a itself.
  int xj = 0;
  int xj_jobs = 0;
  __device__ int64_t u_index(int item) const {
    return uidx ? (int64_t)min(max(uidx[item], 0), nuidx - 1) : (int64_t)item;
  }
  __device__ const __half* xu_rows(int item) const {
    return xu + (xu_u ? u_index(item) : (int64_t)item) * xu_es;
  }
  __device__ int64_t apart_block(int item) const {
    return apart_u ? u_index(item) : (int64_t)item;
  }
};

// Item data of a dense launch: item i is at base + i * stride.
struct DenseSrc {
  const DenseArgs& a;
  __device__ int m_rows(int) const { return a.M; }
  __device__ const __half* xrow(int item, int m) const {
    return a.x + (int64_t)item * a.x_es + (int64_t)m * a.sh.K;
  }
  __device__ const uint32_t* codes(int item) const { return a.codes + (int64_t)item * a.codes_es; }
  __device__ const __half* scales(int item) const { return a.scales + (int64_t)item * a.sz_es; }
  __device__ const __half* zeros(int item) const { return a.zeros + (int64_t)item * a.sz_es; }
  __device__ const __half* sv(int item) const {
    return a.sv ? a.sv + (int64_t)item * a.sv_es : nullptr;
  }
  __device__ const __half* bias(int item) const {
    return a.bias ? a.bias + (int64_t)item * a.bias_es : nullptr;
  }
  __device__ StreamMat mat(int item, int) const {
    return StreamMat{codes(item), scales(item), a.sh.sym ? scales(item) : zeros(item), sv(item),
                     bias(item)};
  }
  __device__ __half load_a(int item, int, int m, int j) const { return load_a(item, m, j); }
  __device__ __half load_a(int item, int m, int j) const {
    if (a.xu) return a.xu_rows(item)[(int64_t)m * a.sh.rank + j];
    const float* p = a.apart + (a.apart_block(item) * a.P * a.M + m) * a.sh.rpad + j;
    return __float2half(sum_strided(p, (int64_t)a.M * a.sh.rpad, a.P));
  }
  __device__ void store(int item, int m, int n, float v) const {
    a.y[(int64_t)item * a.y_es + (int64_t)m * a.sh.N + n] = __float2half(v);
  }
};

}  // namespace glq

#include "glq_lane.h"
#include "glq_tile16.h"

namespace glq {

// Dense items of the lane kernel: item i at base + i * stride, one token row.
struct DenseLaneItem {
  const DenseArgs& a;
  int item;
  __device__ bool lora() const { return a.sv != nullptr && a.sh.rank > 0; }
  __device__ const uint32_t* codes() const { return a.codes + (int64_t)item * a.codes_es; }
  __device__ const __half* scales() const { return a.scales + (int64_t)item * a.sz_es; }
  __device__ const __half* zeros() const { return a.zeros + (int64_t)item * a.sz_es; }
  __device__ const __half* sv() const { return a.sv + (int64_t)item * a.sv_es; }
  __device__ const __half* bias() const { return a.bias + (int64_t)item * a.bias_es; }
  __device__ const __half* u() const { return a.u + a.u_index(item) * a.u_es; }
  __device__ u32x4 x8(int k) const { return *(const u32x4*)(a.x + (int64_t)item * a.x_es + k); }
  __device__ __half load_a(int j) const {
    if (a.xu) return a.xu_rows(item)[j];
    const float* pp = a.apart + a.apart_block(item) * a.P * a.M * a.sh.rpad + j;
    return __float2half(sum_strided(pp, (int64_t)a.M * a.sh.rpad, a.P));
  }
  __device__ void store(int n, float v) const {
    a.y[(int64_t)item * a.y_es + n] = __float2half(v);
  }
  // with x U jobs in the XU launch: a = fp16(x U) in LDS from their sums
  // (lane_run calls it after the first round's quantized sums)
  __device__ bool xu_defer() const { return a.xj > 0 && lora(); }
  __device__ __half* xu_wait(int K, int rank, float* xu_lds) const;
};
struct DenseLaneSrc {
  const DenseArgs& a;
  __device__ DenseLaneItem bind(int item) const { return DenseLaneItem{a, item}; }
};

struct LaneArgs {
  DenseArgs a;
  LaneGeom g;
};

// Item `item` of a dense launch in the token-tile form (glq_tile16.h: 4-bit
// asymmetric codes, each decoded once for all M <= 16 token rows): y = Q(x)
// + a SV^T + bias, a = fp16 of the x U partials' sum (DenseSrc::load_a),
// staged in LDS by prep.
__device__ void t16_xu_wait(const DenseArgs& a, int item, __half* al, float* lds);

struct DenseTileView {
  const DenseArgs& a;
  int item;
  __half* al;  // LDS [M][rank]
  float* lds;  // the launch's LDS (the fused form's local x U)
  __device__ DenseTileView bind() const { return *this; }
  __device__ const uint32_t* codes(int) const { return a.codes + (int64_t)item * a.codes_es; }
  __device__ const __half* scales(int) const { return a.scales + (int64_t)item * a.sz_es; }
  __device__ const __half* zeros(int) const { return a.zeros + (int64_t)item * a.sz_es; }
  __device__ const __half* xrow(int t) const {
    return a.x + (int64_t)item * a.x_es + (int64_t)t * a.sh.K;
  }
  __device__ void before_store() const {
    if (a.sv && a.xt_jobs) t16_xu_wait(a, item, al, lds);  // (uniform)
  }
  __device__ void prep(int, int, int) const {
    const int r = a.sh.rank;
    if (!a.sv || a.xt_jobs) return;  // uniform over the workgroup
    const DenseSrc d{a};
    for (int i = threadIdx.x; i < a.M * r; i += kT16Waves * 64) {
      const int t = i / r;
      al[i] = d.load_a(item, t, i - t * r);
    }
    __syncthreads();
  }
  __device__ void store(int n, int t, float v) const {
    if (a.sv) {
      const int r = a.sh.rank;
      const __half* sv = a.sv + (int64_t)item * a.sv_es + (int64_t)n * r;
      const __half* at = al + t * r;
      float l = 0.f;
      for (int j = 0; j < r; j += 8) {
        const u32x4 s8 = *(const u32x4*)(sv + j), a8 = *(const u32x4*)(at + j);
#pragma unroll
        for (int q = 0; q < 4; ++q) l = dot2(s8[q], a8[q], l);
      }
      v += l;
    }
    if (a.bias) v += __half2float(a.bias[(int64_t)item * a.bias_es + n]);
    a.y[(int64_t)item * a.y_es + (int64_t)t * a.sh.N + n] = __float2half(v);
  }
};

// LDS (floats) of one 256-thread group of lowrank_partial<4>: red, the x
// slice, U transposed, and a 16 x 128 output block.
constexpr int kXtGroupLds = 4 * 4 * 64 + 16 * kLowrankRows / 2 + 64 * kLowrankUtStride / 2;
constexpr int kXtLds = (2 * kXtGroupLds + 2 * 16 * 128) * 4;  // bytes: two groups, two blocks
constexpr unsigned kXtReady = 0x8000u;

__device__ __forceinline__ unsigned t16_xu_final(const DenseArgs& a) {
  return ((unsigned)a.xt_rb << 16) | kXtReady | (unsigned)a.P;
}

// Slices 2 jp and 2 jp + 1 of item i's x U partials, one per 256-thread half
// of the workgroup (lowrank_partial<4>: MFMA tiles, U transposed in LDS);
// COH: into global memory for other workgroups, else into LDS.  Every thread
// calls it.
template <bool COH>
__device__ void t16_xu_pair(const DenseArgs& a, int item, int jp, float* lds, float* out0,
                            float* out1) {
  const int half = threadIdx.x >> 8, tid = threadIdx.x & 255, sp = 2 * jp + half;
  float* g = lds + half * kXtGroupLds;
  __half* xl = (__half*)(g + 4 * 4 * 64);
  __half* ut = xl + 16 * kLowrankRows;
  const __half* X = a.x + (int64_t)item * a.x_es;
  auto xrow = [&](int m) { return X + (int64_t)m * a.sh.K; };
  float* out = half ? out1 : out0;
  if (sp >= a.P) out = nullptr;
  lowrank_partial<4, decltype(xrow), COH>(xrow, a.M, a.sh.K, a.sh.rank, a.sh.rpad,
                                           a.u + a.u_index(item) * a.u_es, min(sp, a.P - 1),
                                           out, g, xl, tid, ut);
}

// Job (item, slice pair): its partials handed over; the item's last slice to
// arrive sums the slices in slice order into a = fp16 (agent-scope stores)
// and marks the item ready.
__device__ void t16_xu_job(const DenseArgs& a, int job, float* lds) {
  __shared__ int last;
  const int npair = (a.P + 1) / 2, item = job / npair, jp = job - item * npair;
  const int rp = a.sh.rpad, M = a.M, rank = a.sh.rank;
  float* parts = a.xt_part + (int64_t)item * a.P * M * rp;
  t16_xu_pair<true>(a, item, jp, lds, parts + (int64_t)(2 * jp) * M * rp,
              parts + (int64_t)(2 * jp + 1) * M * rp);
  const unsigned mine = (unsigned)min(2, a.P - 2 * jp);  // slices this job formed
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(a.xt_cnt + item, mine, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) + mine == (unsigned)a.P;
  __syncthreads();
  if (!last) return;
  for (int i = threadIdx.x; i < M * rank; i += kT16Waves * 64) {
    const int m = i / rank, j = i - m * rank;
    const __half v = __float2half(sum_strided_coh(parts + m * rp + j, (int64_t)M * rp, a.P));
    handoff_put((uint16_t*)a.xt_a + (int64_t)item * M * rank + i, __half_as_ushort(v));
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(a.xt_cnt + item, kXtReady, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (old + kXtReady == t16_xu_final(a)) handoff_reset(a.xt_cnt + item);
  }
}

// Before a row block's stores: item's a into LDS al.  A wait that outlasts
// xt_spin forms it here, slice by slice in the jobs' order (the same bits).
// Every thread calls it.
__device__ void t16_xu_wait(const DenseArgs& a, int item, __half* al, float* lds) {
  __shared__ int ok;
  const int M = a.M, rank = a.sh.rank, rp = a.sh.rpad, tid = threadIdx.x;
  __syncthreads();  // every thread is past the block sums: the LDS is free
  if (tid == 0) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    int r = 1;
    while (!(handoff_get(a.xt_cnt + item) & kXtReady)) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > a.xt_spin) {
        r = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    ok = r;
  }
  __syncthreads();
  if (ok) {
    for (int i = tid; i < M * rank; i += kT16Waves * 64)
      al[i] = __ushort_as_half(handoff_get((const uint16_t*)a.xt_a + (int64_t)item * M * rank + i));
  } else {
    float* outs = lds + 2 * kXtGroupLds;  // two 16 x rpad partial blocks
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // elements tid + 512 q
    for (int jp = 0; jp < (a.P + 1) / 2; ++jp) {
      t16_xu_pair<false>(a, item, jp, lds, outs, outs + 16 * 128);
      __syncthreads();
      for (int h = 0; h < 2 && 2 * jp + h < a.P; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i = tid + kT16Waves * 64 * q, m = i / rank, j = i - m * rank;
          if (m < M) acc[q] += outs[h * 16 * 128 + m * rp + j];
        }
      __syncthreads();
    }
    const int pad = (8 - a.P % 8) % 8;  // sum_strided's zeros after the last batch
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      for (int z = 0; z < pad; ++z) acc[q] += 0.f;
      const int i = tid + kT16Waves * 64 * q, m = i / rank;
      if (m < M) al[i] = __float2half(acc[q]);
    }
  }
  __syncthreads();
  if (tid == 0) {  // this row block has read item's a
    const unsigned old = __hip_atomic_fetch_add(a.xt_cnt + item, 1u << 16, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    if (old + (1u << 16) == t16_xu_final(a)) handoff_reset(a.xt_cnt + item);
  }
}

// Workgroup b = item RB + row block: one K slice (GPW groups a wave cover the
// row); with the in-launch x U, its jobs come first.
template <int GPW>
__global__ __launch_bounds__(kT16Waves * 64) void gemv_t16_kernel(DenseArgs a, T16Geom tg) {
  extern __shared__ __align__(16) float lds[];
  if ((int)blockIdx.x < a.xt_jobs) {  // (uniform)
    t16_xu_job(a, blockIdx.x, lds);
    return;
  }
  const int b = blockIdx.x - a.xt_jobs, item = b / tg.RB;
  __half* al = (__half*)(lds + t16_lds_bytes(false) / 4);
  t16_run<DenseTileView, false, GPW>(DenseTileView{a, item, al, lds}, tg, b - item * tg.RB,
                                     lds);
}

constexpr int kLaneXjMax = 16;  // x U jobs an item (K up to 16 kLowrankRows)

// Item's counter: jobs add 1 once their words are stored, row workgroups
// 1 << 16 once they have read them; the last of all clears the item's words
// and the counter (threads t, t + n, ... of the caller).
__device__ __forceinline__ unsigned lane_xj_final(const DenseArgs& a) {
  return ((unsigned)a.xt_rb << 16) | (unsigned)a.xj;
}
__device__ void lane_xj_clear(const DenseArgs& a, int item, int t, int n) {
  uint32_t* w = (uint32_t*)a.xt_part + (int64_t)item * a.xj * a.sh.rank;
  for (int i = t; i < a.xj * a.sh.rank; i += n) handoff_put(w + i, 0u);
  if (t == 0) handoff_reset(a.xt_cnt + item);
}

// x U job `job` of the lane launch (512 threads): item job / xj, K rows
// [kLowrankRows j, kLowrankRows (j + 1)) of j = job % xj summed by
// lane_xu_sum; the rank fp32 sums handed over bit-inverted (a word of the
// partials is 0 until its job writes it: no sum has the bits 0xffffffff,
// a NaN payload that fp16 inputs cannot give), then the arrival that counts
// the workgroups done with the words.
__device__ void lane_xj_job(const DenseArgs& a, int job, float* xu_lds) {
  const int item = job / a.xj, j = job - item * a.xj, rank = a.sh.rank;
  const int k0 = j * kLowrankRows;
  const float* s = lane_xu_sum(DenseLaneItem{a, item}, k0, min(kLowrankRows, a.sh.K - k0), rank,
                               xu_lds);
  uint32_t* part = (uint32_t*)a.xt_part + ((int64_t)item * a.xj + j) * rank;
  if ((int)threadIdx.x < rank) handoff_put(part + threadIdx.x, ~__float_as_uint(s[threadIdx.x]));
  __shared__ int last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(a.xt_cnt + item, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) + 1u == lane_xj_final(a);
  __syncthreads();
  if (last) lane_xj_clear(a, item, threadIdx.x, blockDim.x);
}

// a from the x U jobs: the workgroup polls the item's xj x rank words
// (thread t words t + 512 q) until none is 0 and stages the sums in LDS, and
// each of the first rank threads sums its column in slice order
// (sum_strided's order and zeros); a wait that outlasts xt_spin has the
// workgroup form the slices with the jobs' code and sum them in the same
// order (the same bits).
__device__ __half* DenseLaneItem::xu_wait(int K, int rank, float* xu_lds) const {
  __shared__ int fail;
  const LaneXu L(rank);
  __half* ah = (__half*)(xu_lds + L.ks * rank + L.nseg * rank);
  const int t = threadIdx.x, n = a.xj, nw = n * rank;  // nw <= ks rank (4096 floats)
  if (t == 0) fail = 0;
  __syncthreads();
  {
    const uint32_t* w = (const uint32_t*)a.xt_part + (int64_t)item * nw;
    constexpr int Q = kLaneXjMax * 128 / 512;  // words a thread (rank <= 128)
    uint32_t b[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) b[q] = t + 512 * q < nw ? handoff_get(w + t + 512 * q) : 1u;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      bool all = a.xt_spin > 0;  // a bound of 0: no wait (the slices formed here)
#pragma unroll
      for (int q = 0; q < Q; ++q) all = all && b[q] != 0u;
      if (all) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 >= a.xt_spin) {
        fail = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int q = 0; q < Q; ++q)
        if (b[q] == 0u) b[q] = handoff_get(w + t + 512 * q);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q)
      if (t + 512 * q < nw) xu_lds[t + 512 * q] = __uint_as_float(~b[q]);
  }
  __syncthreads();
  float acc = 0.f;
  if (t < rank)
    for (int q = 0; q < n; ++q) acc += xu_lds[q * rank + t];
  __syncthreads();
  if (fail) {
    acc = 0.f;
    for (int j = 0; j < n; ++j) {
      const int k0 = j * kLowrankRows;
      const float* s = lane_xu_sum<DenseLaneItem, 0>(*this, k0, min(kLowrankRows, K - k0), rank,
                                                      xu_lds);
      if (t < rank) acc += s[t];
      __syncthreads();  // the next slice rewrites s
    }
  }
  for (int z = n; z % 8; ++z) acc += 0.f;  // sum_strided's zeros after the last batch
  if (t < rank) ah[t] = __float2half(acc);
  __syncthreads();
  if (t < 64) {  // wave 0: this workgroup is done with the item's words (the others go on)
    unsigned old = 0;
    if (t == 0)
      old = __hip_atomic_fetch_add(a.xt_cnt + item, 1u << 16, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old + (1u << 16) == lane_xj_final(a)) lane_xj_clear(a, item, t, 64);
  }
  return ah;
}

// XJ (with XU): the x U jobs come first, then the row workgroups.
template <int BITS, bool SYM, int LRP, int NP, int PD, int NSV, bool HASB, bool XU, bool XJ>
__global__ __launch_bounds__(XU ? 512 : 256) void gemv_lane_kernel(LaneArgs la) {
  extern __shared__ float xu_lds[];
  constexpr int WPB = XU ? 8 : 4;  // waves per workgroup
  int b = blockIdx.x;
  if constexpr (XJ) {
    if (b < la.a.xj_jobs) {  // (uniform)
      lane_xj_job(la.a, b, xu_lds);
      return;
    }
    b -= la.a.xj_jobs;
  }
  const DenseLaneSrc src{la.a};
  const int wvb = (int)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  lane_run<DenseLaneSrc, BITS, SYM, LRP, NP, PD, NSV, HASB, XU, false, XJ>(
      src, la.g, b * WPB + wvb, wvb, xu_lds);
}


template <int MC>
__global__ __launch_bounds__(256) void lowrank_partial_kernel(DenseArgs a) {
  __shared__ float red[4 * 4 * 64];
  __shared__ __align__(16) __half xl[16 * kLowrankRows];
  __shared__ __align__(16) __half ut[MC == 4 ? 64 * kLowrankUtStride : 8];
  const int item = blockIdx.x / a.P, p = blockIdx.x - item * a.P;
  const __half* X = a.x + (int64_t)item * a.x_es;
  const int K = a.sh.K;
  auto xrow = [&](int m) { return X + (int64_t)m * K; };
  int64_t ui = a.u_index(item);
  if (a.usel) {
    const int e = min(max(a.usel[item], 0), a.nsel - 1);
    ui = min(max(a.ucl[e], 0), a.nu - 1);
  }
  lowrank_partial<MC>(xrow, a.M, K, a.sh.rank, a.sh.rpad, a.u + ui * a.u_es, p,
                      (float*)a.apart + ((int64_t)item * a.P + p) * a.M * a.sh.rpad, red, xl,
                      (int)threadIdx.x, ut);
}

// a = fp16(sum over the P K-slices of the partials): items x M x rank.
__global__ __launch_bounds__(256) void lowrank_finalize_kernel(const float* __restrict__ apart,
                                                              int items, int P, int M, int rank,
                                                              int rpad, __half* __restrict__ xu,
                                                              int64_t xu_es) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = (int64_t)M * rank;
  if (idx >= items * per) return;
  const int item = (int)(idx / per);
  const int r = (int)(idx - item * per);
  const int m = r / rank, j = r - m * rank;
  const float* p = apart + ((int64_t)item * P * M + m) * rpad + j;
  float sacc = 0.f;
  for (int q = 0; q < P; ++q) sacc += p[(int64_t)q * M * rpad];
  xu[(int64_t)item * xu_es + r] = __float2half(sacc);
}

template <int BITS, int T, int MP>
__global__ __launch_bounds__(256) void gemv_dense_kernel(DenseArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int item = blockIdx.x / a.tiles, tile = blockIdx.x - item * a.tiles;
  gemv_tile<BITS, T, MP>(DenseSrc{a}, a.sh, item, tile, smem);
}

struct DenseStreamArgs {
  DenseArgs a;
  StreamShape ss;
  int wpi;  // workgroups per item
  int tpw;  // 16-row tiles per workgroup
  int ks;   // K-split form: all four waves on each tile
};

template <int BITS, int MP, int D, bool SYM, bool SZ2>
__global__ __launch_bounds__(256) void gemv_stream_dense_kernel(DenseStreamArgs sa) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int item = blockIdx.x / sa.wpi, wg = blockIdx.x - item * sa.wpi;
  const int t0 = wg * sa.tpw, t1 = min(sa.ss.tiles, t0 + sa.tpw);
  if (sa.ks)
    gemv_stream_ks<BITS, MP, D, SYM, SZ2, 1>(DenseSrc{sa.a}, sa.ss, item, t0, t1, smem);
  else
    gemv_stream<BITS, MP, D, SYM, SZ2, 1>(DenseSrc{sa.a}, sa.ss, item, t0, t1, smem);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kMaxLds = 160 * 1024;
constexpr int kStreamDepth = 3;  // ring slots per wave (2 chunks in flight; 4 workgroups per CU)

static int64_t lowrank_slices(int64_t K) { return (K + kLowrankRows - 1) / kLowrankRows; }

static int64_t workspace_need(int64_t items, int64_t M, int64_t K, int64_t rank) {
  if (rank <= 0) return 0;
  const int64_t rpad = align_up(rank, 32);
  return align_up(items * lowrank_slices(K) * M * rpad * 4, 256);
}

// The GEMV entry points' workspace: kGemvSyncBytes of counter words and
// kLaneXjBytes of the lane launch's x U words (both zero before the first
// call and left zero by every call; no other form writes them), the x U
// partials, and the token-tile form's a (items x M x rank fp16).
constexpr int64_t kGemvSyncBytes = 4096;
constexpr int64_t kLaneXjBytes = 64 << 10;
constexpr int64_t kGemvHeadBytes = kGemvSyncBytes + kLaneXjBytes;
static int64_t gemv_workspace_need(int64_t items, int64_t M, int64_t K, int64_t rank) {
  if (rank <= 0) return 0;
  return kGemvHeadBytes + workspace_need(items, M, K, rank) + align_up(items * M * rank * 2, 256);
}

// Codes per K-phase: the whole K when x fits the staging budget, else the
// largest multiple of both the group size and the step (256 codes for 2-bit,
// 128 for 4-bit) that does.
constexpr int kXStageBudget = 40 * 1024;
int64_t gemv_phase_len(int64_t M, int64_t K, int64_t group, int bits) {
  const int64_t step = bits == 2 ? 256 : 128;
  int64_t unit = group;
  while (unit % step) unit += group;  // lcm(group, step); group is a multiple of 128
  int64_t kp = (kXStageBudget / (2 * M) - 8) / unit * unit;
  if (kp < unit) kp = unit;
  return kp >= K ? K : kp;
}

size_t gemv_lds_bytes(const TileShape& sh, int T) {
  return (size_t)lds_layout(sh.mmax, sh.kp, sh.kp / sh.group, T, sh.xstride, sh.apad).total;
}

template <int BITS, int T, int MP>
static int launch_dense_mp(const DenseArgs& a, size_t lds, hipStream_t s) {
  static size_t attr_bytes = 64 * 1024;
  int rc = set_lds_limit(gemv_dense_kernel<BITS, T, MP>, lds, attr_bytes);
  if (rc) return rc;
  const int64_t grid = (int64_t)a.items * a.tiles;
  gemv_dense_kernel<BITS, T, MP><<<dim3((unsigned)grid), dim3(256), lds, s>>>(a);
  GLQ_LAUNCH_CHECK("gemv_dense_kernel");
  return GLQ_OK;
}

// 2-bit tiles take a second MFMA pass for token rows 8..15.
template <int BITS, int T>
static int launch_dense(const DenseArgs& a, size_t lds, hipStream_t s) {
  if (BITS == 2 && a.sh.mmax > 8) return launch_dense_mp<BITS, T, 2>(a, lds, s);
  return launch_dense_mp<BITS, T, 1>(a, lds, s);
}

int gemv_pick_tiles(int64_t items, int64_t N) {
  const char* env = getenv("GLQ_GEMV_TILES");
  if (env) {
    const int t = atoi(env);
    if (t == 1 || t == 2 || t == 4) return t;
  }
  const int64_t jobs16 = items * ((N + 15) / 16);
  if (jobs16 >= 4 * 1024) return 4;
  if (jobs16 >= 2 * 1024) return 2;
  return 1;
}

// Checks shared by every GEMV entry point; fills sh.
int gemv_check_shape(int64_t M, int64_t K, int64_t N, int bits, int64_t group, int sym,
                     int64_t rank, TileShape& sh) {
  GLQ_CHECK(bits == 2 || bits == 4, "bits must be 2 or 4 (got %d)", bits);
  GLQ_CHECK(sym >= 0 && sym <= 2, "sym must be 0, 1 or 2 (got %d)", sym);
  GLQ_CHECK(M <= 16, "GEMV path takes 1 <= M <= 16 rows (got M=%lld)", (long long)M);
  const int pc = 128 / bits;  // codes per 16-byte piece
  GLQ_CHECK(K > 0 && K % pc == 0, "K=%lld must be a positive multiple of %d at %d bits",
            (long long)K, pc, bits);
  GLQ_CHECK(group > 0 && group % pc == 0 && K % group == 0,
            "group=%lld must be a multiple of %d dividing K=%lld", (long long)group, pc,
            (long long)K);
  GLQ_CHECK(N < (1ll << 30) && K < (1ll << 24), "shape too large");
  if (rank > 0)
    GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
              (long long)rank);
  sh.K = (int)K;
  sh.N = (int)N;
  sh.G = (int)(K / group);
  sh.group = (int)group;
  sh.rank = rank > 0 ? (int)rank : 0;
  sh.sym = sym == 1 ? 1 : 0;
  sh.zoff = sym == 2 ? (float)(1 << (bits - 1)) : 0.f;
  sh.kw = (int)(K * bits / 32);
  sh.rpad = (int)align_up(sh.rank, 32);
  sh.kp = (int)gemv_phase_len(M, K, group, bits);
  sh.xstride = sh.kp + 8;
  sh.apad = sh.rpad + 8;
  sh.mmax = (int)M;
  return GLQ_OK;
}

// Streaming path (glq_stream.h): group 128, N even (scales, zero-points and
// bias move as aligned dwords), rank <= 128, and x + rings within the LDS
// budget.
bool stream_shape(int64_t M, const TileShape& sh, int bits, StreamShape& ss, size_t& lds,
                  bool& sz2) {
  if (getenv("GLQ_GEMV_NO_STREAM")) return false;
  if (sh.group != 128 || sh.N % 2 != 0 || sh.rank > 128) return false;
  ss.K = sh.K;
  ss.N = sh.N;
  ss.G = sh.G;
  ss.rank = sh.rank;
  ss.rpad = sh.rpad;
  ss.sym = sh.sym;
  ss.zoff = sh.zoff;
  ss.kw = sh.kw;
  ss.nchunk = (int)(((int64_t)sh.kw * 4 + 127) / 128);
  ss.nsvc = sh.rank > 0 ? (sh.rank + 63) / 64 : 0;
  ss.tiles = (sh.N + 15) / 16;
  ss.xstride = stream_kpad(sh.K, bits) + 8;
  ss.mmax = (int)M;
  ss.apad = 64 * (ss.nsvc > 0 ? ss.nsvc : 1) + 8;
  ss.goff = 0;
  ss.gend = sh.G;
  ss.rowlast = sh.kw * 4 - 16;
  sz2 = bits == 2 && (sh.G % 2) != 0;
  const int slot = kStreamCodeBytes + (sz2 ? 512 : 256);
  lds = (size_t)stream_lds(kStreamDepth, slot, (int)M, sh.K, bits, ss.xstride, ss.apad).total;
  return lds <= (size_t)kMaxLds;
}

// Workgroups per item: aim for about 4 per CU over the whole launch
// (GLQ_STREAM_WGS overrides the target).
// A launch whose tiles would leave most CUs idle (fewer than 256 workgroups
// at one tile per wave) with long tiles (>= 4 chunks) takes the K-split
// form instead: one tile per workgroup, its chunks dealt over the four waves,
// so each wave's serial chain is a quarter of the tile (GLQ_STREAM_KS=0/1
// forces either form).
void stream_split(int64_t items, int tiles, int nchunk, bool allow_ks, int& wpi, int& tpw,
                  int& ks) {
  int64_t target = 1024;
  if (const char* e = getenv("GLQ_STREAM_WGS")) target = atoll(e) > 0 ? atoll(e) : target;
  ks = items * ((tiles + 3) / 4) < 256 && nchunk >= 4;
  if (const char* e = getenv("GLQ_STREAM_KS")) ks = atoi(e) != 0;
  ks = ks && allow_ks;
  int64_t w = (target + items - 1) / items;
  const int64_t wmax = ks ? tiles : (tiles + 3) / 4;  // at least one tile per wave / workgroup
  if (w > wmax) w = wmax;
  if (w < 1) w = 1;
  tpw = (int)((tiles + w - 1) / w);
  wpi = (tiles + tpw - 1) / tpw;
}

template <int BITS, int MP, bool SYM, bool SZ2>
static int launch_stream_k(const DenseStreamArgs& sa, int64_t items, size_t lds, hipStream_t s) {
  static size_t attr_bytes = 64 * 1024;
  auto kern = gemv_stream_dense_kernel<BITS, MP, kStreamDepth, SYM, SZ2>;
  int rc = set_lds_limit(kern, lds, attr_bytes);
  if (rc) return rc;
  const int64_t grid = items * sa.wpi;
  GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
  kern<<<dim3((unsigned)grid), dim3(256), lds, s>>>(sa);
  GLQ_LAUNCH_CHECK("gemv_stream_dense_kernel");
  return GLQ_OK;
}

template <bool SYM>
static int launch_stream_sym(const DenseStreamArgs& sa, int64_t items, int bits, bool sz2,
                             size_t lds, hipStream_t s) {
  if (bits == 2) {
    if (sa.ss.mmax > 8) {
      if (sz2) return launch_stream_k<2, 2, SYM, true>(sa, items, lds, s);
      return launch_stream_k<2, 2, SYM, false>(sa, items, lds, s);
    }
    if (sz2) return launch_stream_k<2, 1, SYM, true>(sa, items, lds, s);
    return launch_stream_k<2, 1, SYM, false>(sa, items, lds, s);
  }
  return launch_stream_k<4, 1, SYM, false>(sa, items, lds, s);
}

static int launch_stream(const DenseStreamArgs& sa, int64_t items, int bits, bool sz2,
                         size_t lds, hipStream_t s) {
  if (sa.ss.sym) return launch_stream_sym<true>(sa, items, bits, sz2, lds, s);
  return launch_stream_sym<false>(sa, items, bits, sz2, lds, s);
}

// Lane-sliced path (glq_lane.h): one token row, groups of whole 16-byte
// pieces, a code row of at most 128 pieces (two pieces a lane past 64: the
// 4096-code rows of a 4-bit o projection), rank <= 128.
constexpr int kLanePD = 4;              // iterations of loads in flight per wave
constexpr int64_t kLaneWaves = 4096;    // target waves per launch (4 per SIMD)
constexpr int kLaneMaxPieces = 128;

static bool lane_row_shape(const TileShape& sh, int bits) {
  if (getenv("GLQ_GEMV_NO_LANE")) return false;
  return sh.group % (128 / bits) == 0 && sh.rank <= 128 &&
         (int64_t)sh.K * bits / 128 <= kLaneMaxPieces;
}

static bool lane_shape(int64_t M, const TileShape& sh, int bits) {
  return M == 1 && lane_row_shape(sh, bits);
}

// The tile and streaming kernels step over 128-code chunks, one group each
// (or several whole groups).
static bool tile_shape(const TileShape& sh) { return sh.K % 128 == 0 && sh.group % 128 == 0; }

// Bytes of LDS the fused-x U form needs (partials of a, then a in fp16).
static size_t lane_xu_lds(const LaneArgs& la) {
  return (size_t)LaneXu(la.g.rank).lds_bytes(la.g.rank);
}

template <int BITS, bool SYM, int LRP, int NP, int NSV, bool HASB>
static int launch_lane_k(const LaneArgs& la, bool xu, hipStream_t s) {
  const int64_t waves = (int64_t)la.g.items * la.g.wpi;
  if (xu) {
    const int64_t grid = waves / 8 + la.a.xj_jobs;  // wpi is a multiple of 8
    GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
    const size_t lds = lane_xu_lds(la);
    if (la.a.xj > 0) {
      static size_t attr_j = 64 * 1024;
      int rc = set_lds_limit(gemv_lane_kernel<BITS, SYM, LRP, NP, kLanePD, NSV, HASB, true, true>,
                             lds, attr_j);
      if (rc) return rc;
      gemv_lane_kernel<BITS, SYM, LRP, NP, kLanePD, NSV, HASB, true, true>
          <<<dim3((unsigned)grid), dim3(512), lds, s>>>(la);
    } else {
      static size_t attr = 64 * 1024;
      int rc = set_lds_limit(gemv_lane_kernel<BITS, SYM, LRP, NP, kLanePD, NSV, HASB, true, false>,
                             lds, attr);
      if (rc) return rc;
      gemv_lane_kernel<BITS, SYM, LRP, NP, kLanePD, NSV, HASB, true, false>
          <<<dim3((unsigned)grid), dim3(512), lds, s>>>(la);
    }
  } else {
    const int64_t grid = (waves + 3) / 4;
    GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
    gemv_lane_kernel<BITS, SYM, LRP, NP, kLanePD, NSV, HASB, false, false>
        <<<dim3((unsigned)grid), dim3(256), 0, s>>>(la);
  }
  GLQ_LAUNCH_CHECK("gemv_lane_kernel");
  return GLQ_OK;
}

// SV dwords per lane: rank / 2 spread over the LRP lanes of a row.
template <int BITS, bool SYM, int LRP, int NP, bool HASB>
static int launch_lane_sv(const LaneArgs& la, bool xu, hipStream_t s) {
  const int nsv = (la.g.rank / 2 + LRP - 1) / LRP;
  if (nsv <= 1) return launch_lane_k<BITS, SYM, LRP, NP, 1, HASB>(la, xu, s);
  if constexpr (LRP <= 32) {
    if (nsv <= 2) return launch_lane_k<BITS, SYM, LRP, NP, 2, HASB>(la, xu, s);
  }
  if constexpr (LRP == 16) return launch_lane_k<BITS, SYM, LRP, NP, 4, HASB>(la, xu, s);
  GLQ_CHECK(false, "rank %d too large for the lane path", la.a.sh.rank);
}

template <int BITS, bool SYM, bool HASB>
static int launch_lane_lrp(const LaneArgs& la, bool xu, hipStream_t s) {
  if (la.g.lr <= 16) return launch_lane_sv<BITS, SYM, 16, 1, HASB>(la, xu, s);
  if (la.g.lr <= 32) return launch_lane_sv<BITS, SYM, 32, 1, HASB>(la, xu, s);
  if (la.g.lr <= 64) return launch_lane_sv<BITS, SYM, 64, 1, HASB>(la, xu, s);
  return launch_lane_sv<BITS, SYM, 64, 2, HASB>(la, xu, s);
}

template <int BITS>
static int launch_lane_bits(const LaneArgs& la, bool xu, hipStream_t s) {
  const bool hb = la.a.bias != nullptr;
  if (la.a.sh.sym) return hb ? launch_lane_lrp<BITS, true, true>(la, xu, s)
                             : launch_lane_lrp<BITS, true, false>(la, xu, s);
  return hb ? launch_lane_lrp<BITS, false, true>(la, xu, s)
            : launch_lane_lrp<BITS, false, false>(la, xu, s);
}

// xu: a = x U formed in the launch (8-wave workgroups, wpi a multiple of 8).
static int launch_lane(const DenseArgs& a, int bits, bool xu, hipStream_t s) {
  LaneArgs la;
  la.a = a;
  LaneGeom& g = la.g;
  g.N = a.sh.N;
  g.K = a.sh.K;
  g.G = a.sh.G;
  g.group = a.sh.group;
  g.zoff = a.sh.zoff;
  g.kw = a.sh.kw;
  g.rank = a.sh.rank;
  g.items = a.items;
  g.lr = a.sh.K * bits / 128;
  const int lrp = g.lr <= 16 ? 16 : g.lr <= 32 ? 32 : 64;
  g.rounds = (a.sh.N + 63) / 64 * lrp / kLanePD;
  // about kLaneWaves waves over the launch
  const int64_t total = (int64_t)a.items * g.rounds;
  int64_t rpw = (total + kLaneWaves - 1) / kLaneWaves;
  if (const char* e = getenv("GLQ_LANE_RPW")) rpw = atoll(e) > 0 ? atoll(e) : rpw;
  g.rpw = (int)std::min<int64_t>(std::max<int64_t>(rpw, 1), g.rounds);
  g.wpi = (g.rounds + g.rpw - 1) / g.rpw;
  if (xu) {  // whole 8-wave workgroups per item, the rounds spread over all of them
    g.wpi = (g.wpi + 7) / 8 * 8;
    g.rpw = (g.rounds + g.wpi - 1) / g.wpi;
    la.a.xt_rb = g.wpi / 8;
    la.a.xj_jobs = la.a.xj * a.items;
  }
  return bits == 2 ? launch_lane_bits<2>(la, xu, s) : launch_lane_bits<4>(la, xu, s);
}

// Token-tile form (glq_tile16.h) for 4..16 token rows of 4-bit asymmetric
// group-128 codes whose rows fit one workgroup (K <= 4096: 8 waves of up to 4
// groups), rank <= 128: each code decoded once for all the rows where the
// streaming kernel decodes it once and takes a dot2 per row (VALU-bound
// there).  Returns the groups a wave (1, 2, 4), or 0 when the form does not
// apply.
static int t16_gemv_gpw(int64_t M, const TileShape& sh, int bits) {
  int minm = 4;
  if (const char* e = getenv("GLQ_GEMV_T16_MINM")) minm = atoi(e);
  if (getenv("GLQ_GEMV_NO_T16") || M < minm || bits != 4 || sh.sym || sh.zoff != 0.f ||
      sh.group != 128 || sh.K % 128 != 0 || sh.rank > 128)
    return 0;
  const int G = sh.K / 128;
  return G <= kT16Waves ? 1 : G <= 2 * kT16Waves ? 2 : G <= 4 * kT16Waves ? 4 : 0;
}

template <int GPW>
static int launch_t16_gemv(const DenseArgs& a, hipStream_t s) {
  T16Geom tg{};
  tg.N = a.sh.N;
  tg.K = a.sh.K;
  tg.G = a.sh.G;
  tg.kw = a.sh.kw;
  tg.M = a.M;
  tg.RB = (a.sh.N + kT16Rows - 1) / kT16Rows;
  tg.ks = 1;
  size_t lds = (size_t)t16_lds_bytes(false) + 2 * (size_t)a.M * a.sh.rank;
  if (a.xt_jobs) lds = std::max(lds, (size_t)kXtLds);
  static size_t attr = 64 * 1024;
  int rc = set_lds_limit(gemv_t16_kernel<GPW>, lds, attr);
  if (rc) return rc;
  gemv_t16_kernel<GPW><<<dim3((unsigned)(a.xt_jobs + (int64_t)a.items * tg.RB)),
                         dim3(kT16Waves * 64), lds, s>>>(a, tg);
  GLQ_LAUNCH_CHECK("gemv_t16_kernel");
  return GLQ_OK;
}

static int gemv_impl(int64_t items, const void* x, int64_t x_stride, int64_t M,
                     int64_t K, int64_t N, const int32_t* codes,
                     int64_t codes_stride, int bits, const void* scales,
                     const void* zeros, int64_t sz_stride, int64_t group, int sym,
                     const void* U, int64_t u_stride, const void* SV,
                     int64_t sv_stride, int64_t rank, const void* xU,
                     int64_t xu_stride, const void* bias, int64_t bias_stride,
                     void* y, int64_t y_stride, void* workspace,
                     int64_t workspace_bytes_given, void* stream,
                     const int32_t* u_index = nullptr, int64_t n_u = 0,
                     const float* parts = nullptr, int64_t n_parts = 0) {
  clear_error();
  GLQ_CHECK(items >= 0 && M >= 0 && K >= 0 && N >= 0, "negative size");
  if (items == 0 || M == 0 || N == 0) return GLQ_OK;
  const bool lora = SV != nullptr && rank > 0;
  if (parts) {  // a given as fp32 partials: no U, no xU
    GLQ_CHECK(lora && n_parts >= 1 && n_parts < (1 << 20), "partials need SV, rank and P >= 1");
    U = nullptr;
    xU = nullptr;
  }
  TileShape sh;
  int rc = gemv_check_shape(M, K, N, bits, group, sym, lora ? rank : 0, sh);
  if (rc) return rc;
  GLQ_CHECK(x && codes && scales && y && (sym == 1 || zeros), "null data pointer");
  if (lora) GLQ_CHECK(U != nullptr || xU != nullptr || parts != nullptr,
                      "LoRA needs U or a precomputed xU");
  GLQ_CHECK(tile_shape(sh) || lane_row_shape(sh, bits),
            "K=%lld, group=%lld at %d bits: rows or groups that are not whole 128-code "
            "chunks take the lane kernel only (at most %d codes a row, rank <= 128)",
            (long long)K, (long long)group, bits, 64 * 128 / bits);
  if (!tile_shape(sh) && M > 1) {
    GLQ_CHECK(parts == nullptr, "given partials take whole 128-code groups when M > 1");
    // one lane launch per token row (x, a and y rows of the items advance together)
    for (int64_t m = 0; m < M; ++m) {
      rc = gemv_impl(items, (const __half*)x + m * K, x_stride, 1, K, N, codes, codes_stride,
                     bits, scales, zeros, sz_stride, group, sym, U, u_stride, SV, sv_stride,
                     rank, xU ? (const __half*)xU + m * rank : nullptr, xu_stride, bias,
                     bias_stride, (__half*)y + m * N, y_stride, workspace,
                     workspace_bytes_given, stream, u_index, n_u);
      if (rc) return rc;
    }
    return GLQ_OK;
  }
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x) && al16(codes) && (!lora || al16(SV)) && (!lora || !U || al16(U)),
            "x, codes, U and SV must be 16-byte aligned");
  GLQ_CHECK(items == 1 || (x_stride % 8 == 0 && codes_stride % 4 == 0 &&
                           (!lora || sv_stride % 8 == 0) && (!lora || !U || u_stride % 8 == 0)),
            "item strides must keep 16-byte alignment");
  const bool need_partials = lora && xU == nullptr && parts == nullptr;
  // one token row with U given: the lane kernel forms a = x U itself (one
  // launch, no workspace); GLQ_LANE_NO_XU=1 keeps the separate partial-sum launch
  const bool lane_xu = need_partials && lane_shape(M, sh, bits) && !getenv("GLQ_LANE_NO_XU");
  // the token-tile form with x U formed in its own launch (GLQ_T16_XU2=1: the
  // separate partial-sum launch)
  const bool t16_xu = need_partials && !lane_shape(M, sh, bits) && t16_gemv_gpw(M, sh, bits) &&
                      M <= 16 && items <= kGemvSyncBytes / 4 && !getenv("GLQ_T16_XU2");
  const int64_t need = need_partials && !lane_xu ? gemv_workspace_need(items, M, K, rank) : 0;
  if (need > 0) {
    GLQ_CHECK(workspace != nullptr && workspace_bytes_given >= need,
              "workspace of %lld bytes needed (got %lld)", (long long)need,
              (long long)workspace_bytes_given);
    GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  }

  const int T = gemv_pick_tiles(items, N);
  DenseArgs a = {};
  a.codes = (const uint32_t*)codes;
  a.codes_es = codes_stride;
  a.scales = (const __half*)scales;
  a.zeros = (const __half*)zeros;
  a.sz_es = sz_stride;
  a.sv = lora ? (const __half*)SV : nullptr;
  a.sv_es = sv_stride;
  a.u = (const __half*)U;
  a.u_es = u_stride;
  a.bias = (const __half*)bias;
  a.bias_es = bias_stride;
  a.x = (const __half*)x;
  a.x_es = x_stride;
  a.y = (__half*)y;
  a.y_es = y_stride;
  a.xu = lora ? (const __half*)xU : nullptr;
  a.xu_es = xu_stride;
  // workspace: the counter words and the lane launch's x U words (zero
  // between calls), then the x U partials (and the token-tile form's a)
  a.apart = need_partials && !lane_xu ? (const float*)((char*)workspace + kGemvHeadBytes)
                                      : parts;
  a.items = (int)items;
  a.M = (int)M;
  a.P = need_partials && !lane_xu ? (int)lowrank_slices(K) : (int)n_parts;
  a.tiles = (int)((N + 16 * T - 1) / (16 * T));
  a.sh = sh;
  a.uidx = u_index;
  a.nuidx = (int)std::min<int64_t>(n_u, 1 << 30);
  a.xu_u = u_index != nullptr && a.xu != nullptr;
  a.apart_u = u_index != nullptr && parts != nullptr;

  GLQ_CHECK(items * a.tiles < (1ll << 31) && items * a.P < (1ll << 31), "too many workgroups");
  hipStream_t s = (hipStream_t)stream;
  if (lane_xu) {
    // x U in K slices by jobs in front of the launch when the workspace
    // holds their counters and sums (GLQ_LANE_XJ=0: each row workgroup
    // forms a over the whole row)
    const char* xj = getenv("GLQ_LANE_XJ");
    if (workspace != nullptr && ((uintptr_t)workspace & 255) == 0 &&
        workspace_bytes_given >= gemv_workspace_need(items, M, K, rank) &&
        items <= kGemvSyncBytes / 4 && lowrank_slices(K) <= kLaneXjMax &&
        items * lowrank_slices(K) * rank * 4 <= kLaneXjBytes &&
        !(xj && atoi(xj) == 0)) {
      a.xj = (int)lowrank_slices(K);
      a.xt_cnt = (unsigned*)workspace;
      a.xt_part = (float*)((char*)workspace + kGemvSyncBytes);
      // GLQ_LANE_SPIN_TICKS: the row workgroups' wait bound (tests set 0 to
      // take the local x U)
      const char* e = getenv("GLQ_LANE_SPIN_TICKS");
      a.xt_spin = e ? (uint64_t)strtoull(e, nullptr, 10) : 100000;  // 1 ms
    }
    return launch_lane(a, bits, true, s);
  }
  if (t16_xu) {
    a.xt_jobs = (int)(items * ((a.P + 1) / 2));
    a.xt_rb = (int)((N + kT16Rows - 1) / kT16Rows);
    a.xt_cnt = (unsigned*)workspace;
    a.xt_part = (float*)a.apart;
    a.xt_a = (__half*)((char*)workspace + kGemvHeadBytes + workspace_need(items, M, K, rank));
    // GLQ_T16_SPIN_TICKS: the stores' wait bound (tests set 0 to take the
    // local x U)
    const char* e = getenv("GLQ_T16_SPIN_TICKS");
    a.xt_spin = e ? (uint64_t)strtoull(e, nullptr, 10) : 100000;  // 1 ms
  } else if (need_partials) {
    const dim3 grid((unsigned)(items * a.P));
    if (M == 1) lowrank_partial_kernel<1><<<grid, dim3(256), 0, s>>>(a);
    else if (M == 2) lowrank_partial_kernel<2><<<grid, dim3(256), 0, s>>>(a);
    else lowrank_partial_kernel<4><<<grid, dim3(256), 0, s>>>(a);
    GLQ_LAUNCH_CHECK("lowrank_partial_kernel");
  }
  if (lane_shape(M, sh, bits)) return launch_lane(a, bits, false, s);
  if (const int gpw = t16_gemv_gpw(M, sh, bits)) {
    return gpw == 1 ? launch_t16_gemv<1>(a, s) : gpw == 2 ? launch_t16_gemv<2>(a, s)
                                                            : launch_t16_gemv<4>(a, s);
  }
  DenseStreamArgs sa;
  size_t slds = 0;
  bool sz2 = false;
  if (stream_shape(M, sh, bits, sa.ss, slds, sz2)) {
    sa.a = a;
    // the K-split form also holds the waves' partial tiles in LDS
    const bool ks_fits = slds + stream_ks_bytes(1) <= (size_t)kMaxLds;
    stream_split(items, sa.ss.tiles, sa.ss.nchunk, ks_fits, sa.wpi, sa.tpw, sa.ks);
    if (sa.ks) slds += stream_ks_bytes(1);
    return launch_stream(sa, items, bits, sz2, slds, s);
  }
  const size_t lds = gemv_lds_bytes(sh, T);
  GLQ_CHECK(lds <= (size_t)kMaxLds, "M*K too large for the GEMV path (needs %zu bytes of LDS)",
            lds);
  if (bits == 2) {
    if (T == 1) return launch_dense<2, 1>(a, lds, s);
    if (T == 2) return launch_dense<2, 2>(a, lds, s);
    return launch_dense<2, 4>(a, lds, s);
  }
  if (T == 1) return launch_dense<4, 1>(a, lds, s);
  if (T == 2) return launch_dense<4, 2>(a, lds, s);
  return launch_dense<4, 4>(a, lds, s);
}

// ---------------------------------------------------------------------------
// Allocation-free form: the x*U partials live in a file-scope device array
// (one copy per GPU, held until the process ends) instead of a caller's
// workspace.  Host code never passes the array's name to a kernel: its
// device address is looked up once per device with hipGetSymbolAddress and
// kept here.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = 4ll << 20;  // 4 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::once_flag g_scratch_once[kMaxDevices];
static hipError_t g_scratch_rc[kMaxDevices];

// Device address of `scratch` on the current device (looked up on the first
// call for that device).
static int scratch_ptr(void** out) {
  int dev = -1;
  GLQ_HIP(hipGetDevice(&dev));
  GLQ_CHECK(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_rc[dev] == hipSuccess ? p : nullptr;
  });
  if (g_scratch_rc[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr) {
    set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
              hipGetErrorString(g_scratch_rc[dev]));
    return GLQ_ERR_HIP;
  }
  *out = g_scratch_ptr[dev];
  return GLQ_OK;
}

}  // namespace glq

using namespace glq;

extern "C" {

int64_t glq_gemv_noalloc_max_scratch_bytes(void) { return kScratchBytes; }

int glq_gemv_lora_noalloc(const void* x, int64_t M, int64_t K, int64_t N,
                          const int32_t* codes, int bits, const void* scales,
                          const void* zeros, int64_t group, int sym, const void* U,
                          const void* SV, int64_t rank, const void* xU, const void* bias,
                          void* y, void* stream) {
  clear_error();
  GLQ_CHECK(M >= 0 && K >= 0 && N >= 0 && rank >= 0, "negative size");
  const bool partials = SV != nullptr && rank > 0 && xU == nullptr && M > 0 && N > 0;
  const int64_t need = partials ? gemv_workspace_need(1, M, K, rank) : 0;
  GLQ_CHECK(need <= kScratchBytes,
            "x*U partials need %lld bytes, above the %lld-byte static scratch of the "
            "allocation-free entry point (use glq_gemv_lora with a workspace)",
            (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (partials) {
    int rc = scratch_ptr(&ws);
    if (rc) return rc;
  }
  return gemv_impl(1, x, 0, M, K, N, codes, 0, bits, scales, zeros, 0, group, sym,
                   U, 0, SV, 0, rank, xU, 0, bias, 0, y, 0, ws, need, stream);
}

int64_t glq_gemv_workspace_bytes(int64_t items, int64_t M, int64_t K, int64_t N,
                                 int64_t rank) {
  (void)N;
  if (items < 0 || M < 0 || K < 0 || rank < 0) return -1;
  return gemv_workspace_need(items, M, K, rank);
}

int glq_gemv_lora(const void* x, int64_t M, int64_t K, int64_t N,
                  const int32_t* codes, int bits, const void* scales,
                  const void* zeros, int64_t group, int sym, const void* U,
                  const void* SV, int64_t rank, const void* xU, const void* bias,
                  void* y, void* workspace, int64_t workspace_bytes_given,
                  void* stream) {
  return gemv_impl(1, x, 0, M, K, N, codes, 0, bits, scales, zeros, 0, group, sym,
                   U, 0, SV, 0, rank, xU, 0, bias, 0, y, 0, workspace,
                   workspace_bytes_given, stream);
}

int glq_gemv_lora_batched(int64_t items, const void* x, int64_t x_stride,
                          int64_t M, int64_t K, int64_t N, const int32_t* codes,
                          int64_t codes_stride, int bits, const void* scales,
                          const void* zeros, int64_t sz_stride, int64_t group,
                          int sym, const void* U, int64_t u_stride,
                          const void* SV, int64_t sv_stride, int64_t rank,
                          const void* xU, int64_t xu_stride, const void* bias,
                          int64_t bias_stride, void* y, int64_t y_stride,
                          void* workspace, int64_t workspace_bytes_given,
                          void* stream) {
  return gemv_impl(items, x, x_stride, M, K, N, codes, codes_stride, bits, scales,
                   zeros, sz_stride, group, sym, U, u_stride, SV, sv_stride, rank,
                   xU, xu_stride, bias, bias_stride, y, y_stride, workspace,
                   workspace_bytes_given, stream);
}

int glq_gemv_lora_clustered(int64_t items, const void* x, int64_t x_stride, int64_t M,
                            int64_t K, int64_t N, const int32_t* codes, int64_t codes_stride,
                            int bits, const void* scales, const void* zeros, int64_t sz_stride,
                            int64_t group, int sym, const void* U, int64_t u_stride,
                            const int32_t* u_index, int64_t n_u, const void* xU,
                            int64_t xu_stride, const void* SV, int64_t sv_stride, int64_t rank,
                            const void* bias, int64_t bias_stride, void* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes_given, void* stream) {
  clear_error();
  GLQ_CHECK(u_index != nullptr && n_u >= 1, "u_index and n_u >= 1 required");
  GLQ_CHECK(U != nullptr || xU != nullptr, "U or xU required");
  GLQ_CHECK(xU == nullptr || xu_stride >= M * rank, "xu_stride must cover M x rank");
  return gemv_impl(items, x, x_stride, M, K, N, codes, codes_stride, bits, scales, zeros,
                   sz_stride, group, sym, xU ? nullptr : U, u_stride, SV, sv_stride, rank, xU,
                   xu_stride, bias, bias_stride, y, y_stride, workspace, workspace_bytes_given,
                   stream, u_index, n_u);
}

int glq_gemv_lora_parts(int64_t items, const void* x, int64_t x_stride, int64_t M, int64_t K,
                        int64_t N, const int32_t* codes, int64_t codes_stride, int bits,
                        const void* scales, const void* zeros, int64_t sz_stride, int64_t group,
                        int sym, const void* SV, int64_t sv_stride, int64_t rank,
                        const float* parts, int64_t P, const int32_t* u_index, int64_t n_u,
                        const void* bias, int64_t bias_stride, void* y, int64_t y_stride,
                        void* stream) {
  clear_error();
  GLQ_CHECK(SV != nullptr && rank > 0 && parts != nullptr && P >= 1,
            "SV, rank > 0, parts and P >= 1 required");
  GLQ_CHECK(((uintptr_t)parts & 3) == 0, "parts must be 4-byte aligned");
  GLQ_CHECK(u_index == nullptr || n_u >= 1, "u_index needs n_u >= 1");
  return gemv_impl(items, x, x_stride, M, K, N, codes, codes_stride, bits, scales, zeros,
                   sz_stride, group, sym, nullptr, 0, SV, sv_stride, rank, nullptr, 0, bias,
                   bias_stride, y, y_stride, nullptr, 0, stream, u_index, n_u, parts, P);
}

int64_t glq_lowrank_workspace_bytes(int64_t items, int64_t M, int64_t K, int64_t rank) {
  if (items < 0 || M < 0 || K < 0 || rank < 0) return -1;
  return workspace_need(items, M, K, rank);
}

int glq_lowrank_xu_batched(int64_t items, const void* x, int64_t x_stride, int64_t M, int64_t K,
                           const void* U, int64_t u_stride, int64_t rank, void* xu,
                           int64_t xu_stride, void* workspace, int64_t workspace_bytes_given,
                           void* stream) {
  clear_error();
  GLQ_CHECK(items >= 0 && M >= 0 && K >= 0 && rank >= 0, "negative size");
  if (items == 0 || M == 0 || rank == 0) return GLQ_OK;
  GLQ_CHECK(M <= 16, "takes 1 <= M <= 16 rows (got M=%lld)", (long long)M);
  GLQ_CHECK(K > 0 && K < (1ll << 24), "bad K=%lld", (long long)K);
  GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
            (long long)rank);
  GLQ_CHECK(x && U && xu, "null data pointer");
  GLQ_CHECK(((uintptr_t)U & 15) == 0 && (items == 1 || u_stride % 8 == 0),
            "U must be 16-byte aligned");
  const int64_t need = workspace_need(items, M, K, rank);
  GLQ_CHECK(workspace != nullptr && workspace_bytes_given >= need,
            "workspace of %lld bytes needed (got %lld)", (long long)need,
            (long long)workspace_bytes_given);
  DenseArgs a = {};
  a.u = (const __half*)U;
  a.u_es = u_stride;
  a.x = (const __half*)x;
  a.x_es = x_stride;
  a.apart = (const float*)workspace;
  a.items = (int)items;
  a.M = (int)M;
  a.P = (int)lowrank_slices(K);
  a.sh.K = (int)K;
  a.sh.rank = (int)rank;
  a.sh.rpad = (int)align_up(rank, 32);
  GLQ_CHECK(items * a.P < (1ll << 31), "too many workgroups");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(items * a.P));
  if (M == 1) lowrank_partial_kernel<1><<<grid, dim3(256), 0, s>>>(a);
  else if (M == 2) lowrank_partial_kernel<2><<<grid, dim3(256), 0, s>>>(a);
  else lowrank_partial_kernel<4><<<grid, dim3(256), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("lowrank_partial_kernel");
  const int64_t n = items * M * rank;
  lowrank_finalize_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(
      a.apart, a.items, a.P, a.M, (int)rank, a.sh.rpad, (__half*)xu, xu_stride);
  GLQ_LAUNCH_CHECK("lowrank_finalize_kernel");
  return GLQ_OK;
}

int glq_lowrank_xu_routed(int64_t picks, const void* x, int64_t K, const void* U, int64_t u_rows,
                          int64_t rank, const int32_t* sel, int64_t experts,
                          const int32_t* cluster_of, void* xu, void* workspace,
                          int64_t workspace_bytes_given, void* stream) {
  clear_error();
  GLQ_CHECK(picks >= 0 && K >= 0 && rank >= 0 && u_rows >= 1 && experts >= 1, "bad size");
  if (picks == 0 || rank == 0) return GLQ_OK;
  GLQ_CHECK(K > 0 && K < (1ll << 24), "bad K=%lld", (long long)K);
  GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
            (long long)rank);
  GLQ_CHECK(x && U && xu && sel && cluster_of, "null pointer");
  GLQ_CHECK(((uintptr_t)U & 15) == 0, "U must be 16-byte aligned");
  const int64_t need = workspace_need(picks, 1, K, rank);
  GLQ_CHECK(workspace != nullptr && workspace_bytes_given >= need,
            "workspace of %lld bytes needed (got %lld)", (long long)need,
            (long long)workspace_bytes_given);
  DenseArgs a = {};
  a.u = (const __half*)U;
  a.u_es = K * rank;
  a.x = (const __half*)x;
  a.x_es = K;
  a.apart = (const float*)workspace;
  a.items = (int)picks;
  a.M = 1;
  a.P = (int)lowrank_slices(K);
  a.sh.K = (int)K;
  a.sh.rank = (int)rank;
  a.sh.rpad = (int)align_up(rank, 32);
  a.usel = sel;
  a.ucl = cluster_of;
  a.nsel = (int)std::min<int64_t>(experts, 1 << 30);
  a.nu = (int)std::min<int64_t>(u_rows, 1 << 30);
  GLQ_CHECK(picks * a.P < (1ll << 31), "too many workgroups");
  hipStream_t s = (hipStream_t)stream;
  lowrank_partial_kernel<1><<<dim3((unsigned)(picks * a.P)), dim3(256), 0, s>>>(a);
  GLQ_LAUNCH_CHECK("lowrank_partial_kernel");
  const int64_t n = picks * rank;
  lowrank_finalize_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(
      a.apart, a.items, a.P, 1, (int)rank, a.sh.rpad, (__half*)xu, rank);
  GLQ_LAUNCH_CHECK("lowrank_finalize_kernel");
  return GLQ_OK;
}

}  // extern "C"
