// Decoder-layer pieces of the model-level decode step that sit around the
// GLoRCQ projections and the MoE step: RMSNorm (optionally fused with the
// residual add before it), the per-head q/k RMSNorm + rotary embedding +
// static-KV-cache write of one decode token, and single-query grouped-query
// attention over the static cache.  Each replaces a chain of 5-10 small
// framework kernels per use with one launch, with the framework's rounding
// points kept (fp16 results where the framework rounds to fp16, fp32 inside).

#include <hip/hip_fp16.h>

#include "glq_gemv_core.h"
#include "glq_handoff.h"
#include "glq_internal.h"

namespace glq {
namespace {

constexpr int kDecThreads = 256;
constexpr int kHeadDim = 128;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Sum (or max) over the 256 threads of a block; every thread gets the result.
template <bool MAX>
__device__ inline float block_reduce(float v, float* red) {
  v = MAX ? wave_max(v) : wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return MAX ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))
             : (red[0] + red[1]) + (red[2] + red[3]);
}

// fp16 x fp16 -> fp16 as the framework's elementwise ops compute it (fp32
// product, one rounding).
__device__ inline _Float16 hmul(_Float16 a, _Float16 b) { return (_Float16)((float)a * (float)b); }

// ---------------------------------------------------------------------------
// One token row's partial of a = x U over R <= 32 NI rows of U, with the U
// loads issued before x exists (a launch that normalizes or merges the row
// first): thread t holds columns jb + 8 (t & 7) .. + 8 of rows (t >> 3) +
// 32 i; rows past R and columns past rank read as zero.  Then dot() sums
// x[k] U[k][jb + j] over the rows (fp32; per thread over its rows, then the
// 32 row groups in order through LDS) and returns the sum of column jb + j
// to thread j < 64.  Every thread of the 256 calls both.
// ---------------------------------------------------------------------------
constexpr int kURowsRed = 32 * 64;  // LDS floats of URows::dot

template <int NI>
struct URows {
  f16x8 u[NI];
  __device__ void issue(const __half* U, int rank, int R, int jb) {
    const int c = jb + 8 * (threadIdx.x & 7), r0 = threadIdx.x >> 3;
    asm volatile("" ::: "memory");  // after the memory operations issued before
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = r0 + 32 * i;
      u[i] = (row < R && c < rank) ? *(const f16x8*)(U + (int64_t)row * rank + c) : f16x8{};
    }
    // compiler memory barriers on both sides keep the loads where they are
    // issued (the compiler would otherwise move them next to their first use,
    // or ahead of loads the caller needs first); they wait for nothing
    asm volatile("" ::: "memory");
  }
  // x must be complete in LDS (a barrier after its writes) before the call.
  __device__ float dot(const __half* x /* LDS, R values */, int R,
                       float* red /* LDS, kURowsRed floats */) const {
    const int r0 = threadIdx.x >> 3;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int row = r0 + 32 * i;
      const float xv = row < R ? __half2float(x[row]) : 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[c] = fmaf(xv, (float)u[i][c], acc[c]);
    }
    __syncthreads();  // red may still be read from a previous call
    float* mine = red + r0 * 64 + 8 * (threadIdx.x & 7);
    *(float4*)mine = float4{acc[0], acc[1], acc[2], acc[3]};
    *(float4*)(mine + 4) = float4{acc[4], acc[5], acc[6], acc[7]};
    __syncthreads();
    float v = 0.f;
    if (threadIdx.x < 64) {
#pragma unroll 8
      for (int q = 0; q < 32; ++q) v += red[q * 64 + threadIdx.x];
    }
    return v;
  }
};

// ---------------------------------------------------------------------------
// RMSNorm over rows of D fp16 values (Qwen3MoeRMSNorm.forward):
//   y   = x (+ residual, fp16 add)            -> residual_out when fused
//   out = fp16(w * fp16(y * rsqrt(mean(y^2) + eps)))
// One block per row; each thread holds up to kNormIters 8-wide pieces.
// ---------------------------------------------------------------------------
constexpr int kNormIters = 4;  // D <= 256 * 8 * 4 = 8192

// The row pass of the RMSNorm, shared by every kernel that normalizes a row
// (256 threads, the same order of sums everywhere, so the same bits): thread
// tid takes 8-wide pieces tid + 256 it of the row into y (x, or fp16(x +
// residual)) and every thread gets r = rsqrt(mean(y^2) + eps).
__device__ inline float rms_row(const __half* x, const __half* res, int64_t row, int D, float eps,
                                f16x8 (&y)[kNormIters], float* red) {
  const f16x8* xr = (const f16x8*)(x + row * D);
  const f16x8* rr = res ? (const f16x8*)(res + row * D) : nullptr;
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < kNormIters; ++it) {
    const int i = threadIdx.x + it * kDecThreads;  // 8-wide piece index
    if (i * 8 < D) {
      f16x8 v = xr[i];
      if (rr) {
        const f16x8 r = rr[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (_Float16)((float)v[e] + (float)r[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (float)v[e] * (float)v[e];
      y[it] = v;
    }
  }
  const float total = block_reduce<false>(ss, red);
  return rsqrtf(total / (float)D + eps);
}

// out = fp16(w * fp16(y * r)) of one 8-wide piece.
__device__ inline f16x8 rms_piece(const f16x8& y, const __half* w, int i, float r) {
  const f16x8 wv = ((const f16x8*)w)[i];
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = hmul(wv[e], (_Float16)((float)y[e] * r));
  return o;
}

__global__ __launch_bounds__(kDecThreads) void rmsnorm_kernel(
    const __half* __restrict__ x, const __half* __restrict__ res, const __half* __restrict__ w,
    __half* __restrict__ out, __half* __restrict__ res_out, int D, float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  f16x8 y[kNormIters];
  const float r = rms_row(x, res, row, D, eps, y, red);
#pragma unroll
  for (int it = 0; it < kNormIters; ++it) {
    const int i = threadIdx.x + it * kDecThreads;
    if (i * 8 < D) {
      if (res) ((f16x8*)(res_out + row * D))[i] = y[it];
      ((f16x8*)(out + row * D))[i] = rms_piece(y[it], w, i, r);
    }
  }
}

// ---------------------------------------------------------------------------
// RMSNorm of M <= 16 rows and, in the same launch, the fp32 partials of
// out U_u for n_u matrices U_u (D x rank): the x U of the projections that
// read the normalized rows (q, k and v of a decoder layer), which sum the
// partials in slice order as they load a (glq_gemv_lora_parts).  Workgroup
// (u, s) normalizes every row (rms_row: the bits of rmsnorm_kernel), keeps
// its K slice s (kLowrankRows values of each row) in LDS -- and, for u = 0,
// writes that slice of out (and of the fused residual sum) -- then writes the
// slice's partial of out U_u to parts[u][s].
// ---------------------------------------------------------------------------
struct RxArgs {
  const __half *x, *res, *w;
  __half *out, *res_out;
  const __half* U;
  int64_t u_stride;  // halves between U matrices
  float* part;       // (n_u, S, M, rpad)
  int M, D, S, rank, rpad;
  float eps;
};

constexpr int kRxMaxRows = 16;
constexpr size_t kRxLds = (size_t)kRxMaxRows * kLowrankRows * 2   // the rows' slices (fp16)
                          + kURowsRed * 4                         // partial sums
                          + (size_t)16 * kLowrankRows * 2         // lowrank_partial's x slice
                          + (size_t)64 * kLowrankUtStride * 2;    // U block, transposed

// MC = 0: up to kRxPfRows rows, the slice's U loads issued before the
// norms (URows); MC = 4: 3..16 rows by MFMA tiles (lowrank_partial).
constexpr int kRxPfRows = 3;

template <int MC>
__global__ __launch_bounds__(kDecThreads) void rmsnorm_xu_kernel(RxArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  __half* xn = (__half*)smem;                               // [M][kLowrankRows]
  float* red = (float*)(xn + kRxMaxRows * kLowrankRows);    // kURowsRed (>= 4*4*64)
  __half* xl = (__half*)(red + kURowsRed);                  // 16 x kLowrankRows
  __half* ut = xl + 16 * kLowrankRows;                      // 64 x kLowrankUtStride
  __shared__ float red4[4];
  const int u = blockIdx.x / g.S, s = blockIdx.x - u * g.S;
  const int k0 = s * kLowrankRows, kl = min(kLowrankRows, g.D - k0);
  const int p0 = k0 / 8, p1 = p0 + kl / 8;  // the slice's 8-wide pieces
  const __half* Us = g.U + u * g.u_stride + (int64_t)k0 * g.rank;  // the slice's rows
  URows<kLowrankRows / 32> ur;
  if constexpr (MC == 0) ur.issue(Us, g.rank, kl, 0);
  for (int m = 0; m < g.M; ++m) {
    f16x8 y[kNormIters];
    const float r = rms_row(g.x, g.res, m, g.D, g.eps, y, red4);
#pragma unroll
    for (int it = 0; it < kNormIters; ++it) {
      const int i = threadIdx.x + it * kDecThreads;
      if (i >= p0 && i < p1) {
        const f16x8 o = rms_piece(y[it], g.w, i, r);
        *(f16x8*)(xn + m * kLowrankRows + 8 * (i - p0)) = o;
        if (u == 0) {
          ((f16x8*)(g.out + (int64_t)m * g.D))[i] = o;
          if (g.res) ((f16x8*)(g.res_out + (int64_t)m * g.D))[i] = y[it];
        }
      }
    }
  }
  __syncthreads();
  float* mine = g.part + ((int64_t)u * g.S + s) * g.M * g.rpad;
  if constexpr (MC == 0) {
    for (int jb = 0; jb < g.rpad; jb += 64) {
      if (jb > 0) ur.issue(Us, g.rank, kl, jb);
      for (int m = 0; m < g.M; ++m) {
        const float v = ur.dot(xn + m * kLowrankRows, kl, red);
        if (threadIdx.x < 64 && jb + threadIdx.x < g.rpad) mine[m * g.rpad + jb + threadIdx.x] = v;
      }
    }
  } else {
    // rows of the slice from LDS, indexed as lowrank_partial reads them
    // (xrow(m) + k for k in [k0, k0 + kl))
    auto xrow = [&](int m) { return xn + m * kLowrankRows - k0; };
    lowrank_partial<MC>(xrow, g.M, g.D, g.rank, g.rpad, g.U + u * g.u_stride, s, mine, red, xl,
                        (int)threadIdx.x, ut);
  }
}

// ---------------------------------------------------------------------------
// One decode token per batch row: q/k head RMSNorm (weights qw / kw over the
// 128 head dims), rotary embedding q' = q cos + rotate_half(q) sin with every
// product and the sum rounded to fp16 (apply_rotary_pos_emb), k' and v
// written to the static cache at position *pos; q' to q_out (B, Hq, 128)
// (NaN when *pos is outside the cache).
// One wave per head: heads [0, Hq) are q, [Hq, Hq + Hk) k, then Hk of v.
// Lane l holds dims 2l, 2l + 1; rotate_half pairs lane l with lane l ^ 32.
// ---------------------------------------------------------------------------
struct QkArgs {
  const __half *q, *k, *v;  // rows of q_stride / kv_stride values per token
  int64_t q_stride, kv_stride;
  int q_item;  // > 0: q item-major, [Hq*128 / q_item][B][q_item] (a batched GEMV's output)
  const __half *qw, *kw;
  const __half *cos, *sin;  // (B or 1, 128)
  int64_t cs_stride;        // 0 when one row serves every token
  __half* q_out;
  __half *k_cache, *v_cache;  // (B, Hk, max_len, 128)
  const int64_t* pos;         // write position (device)
  int* len_out;               // *pos + 1, for the attention launch
  int B, Hq, Hk, max_len;
  float eps;
};

__global__ __launch_bounds__(kDecThreads) void qk_norm_rope_kernel(QkArgs a) {
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.x * (kDecThreads / 64) + (threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int64_t p = *a.pos;
  if (head == 0 && b == 0 && lane == 0) *a.len_out = (int)(p + 1);
  if (head >= a.Hq + 2 * a.Hk) return;
  const bool in_cache = p >= 0 && p < a.max_len;
  const int kind = head < a.Hq ? 0 : (head < a.Hq + a.Hk ? 1 : 2);
  const int h = kind == 0 ? head : (kind == 1 ? head - a.Hq : head - a.Hq - a.Hk);
  const int hc = h * kHeadDim;  // the head's first column
  const __half* src =
      kind != 0 ? (kind == 1 ? a.k : a.v) + b * a.kv_stride + hc
      : a.q_item > 0 ? a.q + ((int64_t)(hc / a.q_item) * a.B + b) * a.q_item + hc % a.q_item
                     : a.q + b * a.q_stride + hc;
  const f16x2 x = ((const f16x2*)src)[lane];
  const int64_t crow = (((int64_t)b * a.Hk + h) * a.max_len + (in_cache ? p : 0)) * kHeadDim;
  if (kind == 2) {
    if (in_cache) ((f16x2*)(a.v_cache + crow))[lane] = x;
    return;
  }
  const float f0 = (float)x[0], f1 = (float)x[1];
  const float r = rsqrtf(wave_sum(f0 * f0 + f1 * f1) / (float)kHeadDim + a.eps);
  const f16x2 wv = ((const f16x2*)(kind == 0 ? a.qw : a.kw))[lane];
  f16x2 n;
  n[0] = hmul(wv[0], (_Float16)(f0 * r));
  n[1] = hmul(wv[1], (_Float16)(f1 * r));
  // partner dims (2l + 64 for l < 32, 2l - 64 otherwise)
  const uint32_t nb = __builtin_bit_cast(uint32_t, n);
  const uint32_t pb = (uint32_t)__shfl_xor((int)nb, 32);
  f16x2 rot = __builtin_bit_cast(f16x2, pb);
  if (lane < 32) rot = -rot;
  const f16x2 c = ((const f16x2*)(a.cos + b * a.cs_stride))[lane];
  const f16x2 s = ((const f16x2*)(a.sin + b * a.cs_stride))[lane];
  f16x2 o;
#pragma unroll
  for (int e = 0; e < 2; ++e) o[e] = (_Float16)((float)hmul(n[e], c[e]) + (float)hmul(rot[e], s[e]));
  if (kind == 0) {
    // a position past the static cache attends without this token: q' goes
    // out as NaN so the step's output shows it (transformers' StaticLayer
    // raises on the out-of-range cache write instead)
    if (!in_cache) o = f16x2{(_Float16)__builtin_nanf(""), (_Float16)__builtin_nanf("")};
    ((f16x2*)(a.q_out + ((int64_t)b * a.Hq + h) * kHeadDim))[lane] = o;
  } else if (in_cache)
    ((f16x2*)(a.k_cache + crow))[lane] = o;
}

// ---------------------------------------------------------------------------
// Single-query attention of token b's q heads of KV group g over cache
// positions [0, L), L = *len (clamped to [1, max_len]), split over blocks of
// kAttnChunk positions (flash-decoding):
//   out = sum_p softmax_p(scale * q . k_p) v_p        (fp32, fp16 result)
// Block (split, g, b) stages its K and V rows and the group's rep <= 8 q rows
// in LDS (every load in flight at once), scores (position, head) pairs with
// v_dot2 on fp16 pairs, forms per-head max m, sum l and l-weighted V rows o,
// and writes (m, l, o) to the workspace.  The last block of (b, g) to arrive
// (an arrival counter, incremented after a device-scope fence) merges the
// splits -- M = max m_s, out = sum o_s e^(m_s - M) / sum l_s e^(m_s - M) --
// and zeroes the counter for the next call; the last block of (0, 0) also
// advances *advance (the cache's fill counter) by one.
// ---------------------------------------------------------------------------
constexpr int kAttnChunk = 128;
constexpr int kAttnMaxRep = 8;
constexpr int kKStride = kHeadDim + 8;  // LDS row of K (halves), 16-byte aligned
constexpr int kPartStride = kHeadDim + 4;  // m, l, 2 pad, o: rows 16-byte aligned

struct AttnArgs {
  const __half* q;  // (B, Hq, 128)
  const __half *k_cache, *v_cache;
  const int* len;
  int64_t* advance;
  __half* out;     // (B, Hq * 128)
  float* part;     // [B][Hq][nsplit][kPartStride]: m, l, -, -, o[128]
  unsigned* count; // [B][Hk], zero between calls
  int B, Hq, Hk, max_len, nsplit;
  float scale;
  // XU form: the fp32 partials of out U of each token (the o projection's
  // x U), one per KV group, summed in group order by the projection
  const __half* U;  // (Hq * 128, rank)
  float* xpart;     // [Hk][B][rpad]
  int rank, rpad;
};

constexpr size_t kAttnLds = 2 * kAttnMaxRep * kHeadDim          // q rows
                            + 2 * kAttnChunk * kKStride          // K rows
                            + 2 * kAttnChunk * kHeadDim          // V rows
                            + 4 * kAttnMaxRep * kAttnChunk + 16;  // weights, flag

template <bool XU>
__global__ __launch_bounds__(kDecThreads) void decode_attention_kernel(AttnArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __half* qs = (__half*)smem;
  __half* ks = qs + kAttnMaxRep * kHeadDim;
  __half* vs = ks + kAttnChunk * kKStride;
  float* ps = (float*)(vs + kAttnChunk * kHeadDim);
  int* flag = (int*)(ps + kAttnMaxRep * kAttnChunk);
  const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int rep = a.Hq / a.Hk;
  const int L = min(max(*a.len, 1), a.max_len);
  const int c0 = split * kAttnChunk, n = max(0, min(kAttnChunk, L - c0));
  const int64_t base = ((int64_t)b * a.Hk + g) * a.max_len * kHeadDim + (int64_t)c0 * kHeadDim;
  // stage: 16-byte pieces, 16 per row; K and V rows [0, n), q rows [0, rep).
  // Every load is unconditional (rows past n re-read row n - 1, the rows past
  // n in LDS are never read), so all 16 go out before the first wait.
  if (n > 0) {
    constexpr int NJ = kAttnChunk * 16 / kDecThreads;  // 16-byte pieces per thread
    f16x8 kb[NJ], vb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int idx = j * kDecThreads + tid, r = min(idx >> 4, n - 1), c = idx & 15;
      kb[j] = ((const f16x8*)(a.k_cache + base))[r * 16 + c];
      vb[j] = ((const f16x8*)(a.v_cache + base))[r * 16 + c];
    }
    if (tid < rep * 16)
      ((f16x8*)qs)[tid] = ((const f16x8*)(a.q + ((int64_t)b * a.Hq + g * rep) * kHeadDim))[tid];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int idx = j * kDecThreads + tid, r = idx >> 4, c = idx & 15;
      *(f16x8*)(ks + r * kKStride + 8 * c) = kb[j];
      ((f16x8*)vs)[idx] = vb[j];
    }
  }
  __syncthreads();
  // scores: position p = tid % chunk, heads h = tid / chunk, + 256 / chunk, ...
  {
    const int p = tid & (kAttnChunk - 1);
    for (int h = tid / kAttnChunk; h < rep; h += kDecThreads / kAttnChunk) {
      float s = -__builtin_inff();
      if (p < n) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const f16x8 kv = *(const f16x8*)(ks + p * kKStride + 8 * j);
          const f16x8 qv = *(const f16x8*)(qs + h * kHeadDim + 8 * j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f16x2 k2 = {kv[2 * e], kv[2 * e + 1]}, q2 = {qv[2 * e], qv[2 * e + 1]};
            if (e & 1)
              s1 = __builtin_amdgcn_fdot2(q2, k2, s1, false);
            else
              s0 = __builtin_amdgcn_fdot2(q2, k2, s0, false);
          }
        }
        s = (s0 + s1) * a.scale;
      }
      ps[h * kAttnChunk + p] = s;
    }
  }
  __syncthreads();
  // per head (32 lanes each): chunk max and sum, weights in place
  const int h = tid >> 5, l32 = tid & 31;
  float m = -__builtin_inff(), l = 0.f;
  if (h < rep) {
    float* row = ps + h * kAttnChunk;
#pragma unroll
    for (int i = 0; i < kAttnChunk / 32; ++i) m = fmaxf(m, row[l32 + 32 * i]);
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (n > 0) {
#pragma unroll
      for (int i = 0; i < kAttnChunk / 32; ++i) {
        const int p = l32 + 32 * i;
        const float e = p < n ? expf(row[p] - m) : 0.f;
        row[p] = e;
        l += e;
      }
    }
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) l += __shfl_xor(l, o);
  }
  __syncthreads();
  // o_h[4 l32 .. +4] = sum_p w[h][p] v[p][..]
  float* my = a.part + (((int64_t)b * a.Hq + g * rep + h) * a.nsplit + split) * kPartStride;
  if (h < rep) {
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    const float* row = ps + h * kAttnChunk;
#pragma unroll 8
    for (int p = 0; p < n; ++p) {
      const float w = row[p];
      const uint2 vv = *(const uint2*)(vs + p * kHeadDim + 4 * l32);
      const f16x2 va = __builtin_bit_cast(f16x2, vv.x), vb2 = __builtin_bit_cast(f16x2, vv.y);
      o0 += w * (float)va[0];
      o1 += w * (float)va[1];
      o2 += w * (float)vb2[0];
      o3 += w * (float)vb2[1];
    }
    if (l32 == 0) {
      handoff_put(my, m);
      handoff_put(my + 1, l);
    }
    handoff_put(my + 4 + 4 * l32, o0);
    handoff_put(my + 5 + 4 * l32, o1);
    handoff_put(my + 6 + 4 * l32, o2);
    handoff_put(my + 7 + 4 * l32, o3);
  }
  // arrival (glq_handoff.h); the last block of (b, g) merges the splits
  if (!handoff_arrive(a.count + b * a.Hk + g, (unsigned)a.nsplit, flag)) return;
  // The other blocks' partials through coherent loads, up to 8 splits' worth
  // in flight at once, merged online (running max M, sums rescaled when M
  // grows).  Every thread loads (threads past rep read head rep - 1's and
  // drop them), so that in the XU form the group's rows of U -- rows
  // [g R, g R + R) -- go out right after the first 8 splits' loads: the merge
  // waits for its own loads only and the U rows arrive behind it.
  const int R = rep * kHeadDim;
  URows<kAttnMaxRep * kHeadDim / 32> ur;
  const float* ph =
      a.part + ((int64_t)b * a.Hq + g * rep + min(h, rep - 1)) * a.nsplit * kPartStride;
  float M = -__builtin_inff(), den = 0.f, r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
  auto merge8 = [&](int s0, bool first) {
    float ms[8], ls[8];
    float4 os[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s2 = min(s0 + j, a.nsplit - 1);
      const float* pp = ph + s2 * kPartStride;
      ms[j] = handoff_get(pp);
      ls[j] = handoff_get(pp + 1);
      os[j] = float4{handoff_get(pp + 4 + 4 * l32), handoff_get(pp + 5 + 4 * l32),
                     handoff_get(pp + 6 + 4 * l32), handoff_get(pp + 7 + 4 * l32)};
    }
    if constexpr (XU) {
      if (first) ur.issue(a.U + (int64_t)g * R * a.rank, a.rank, R, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (s0 + j >= a.nsplit || ms[j] == -__builtin_inff()) continue;  // none / empty split
      const float Mn = fmaxf(M, ms[j]);
      const float fo = expf(M - Mn), fn = expf(ms[j] - Mn);  // M = -inf: fo = 0
      den = den * fo + ls[j] * fn;
      r0 = r0 * fo + os[j].x * fn;
      r1 = r1 * fo + os[j].y * fn;
      r2 = r2 * fo + os[j].z * fn;
      r3 = r3 * fo + os[j].w * fn;
      M = Mn;
    }
  };
  merge8(0, true);
  for (int s0 = 8; s0 < a.nsplit; s0 += 8) merge8(s0, false);
  if (h < rep) {
    const float inv = 1.f / den;
    f16x2 oa = {(_Float16)(r0 * inv), (_Float16)(r1 * inv)};
    f16x2 ob = {(_Float16)(r2 * inv), (_Float16)(r3 * inv)};
    __half* dst = a.out + (int64_t)b * a.Hq * kHeadDim + (int64_t)(g * rep + h) * kHeadDim;
    const uint2 o4 = uint2{__builtin_bit_cast(uint32_t, oa), __builtin_bit_cast(uint32_t, ob)};
    *(uint2*)(dst + 4 * l32) = o4;
    if constexpr (XU) *(uint2*)((__half*)ks + h * kHeadDim + 4 * l32) = o4;  // K rows are dead
  }
  if constexpr (XU) {
    // the group's partial of out U (fp32), read by the next launch
    const __half* xo = (const __half*)ks;
    float* red = (float*)((__half*)ks + kAttnMaxRep * kHeadDim);  // kURowsRed floats
    float* mine = a.xpart + ((int64_t)g * a.B + b) * a.rpad;
    __syncthreads();  // the merged rows are in xo
    for (int jb = 0; jb < a.rpad; jb += 64) {
      if (jb > 0) ur.issue(a.U + (int64_t)g * R * a.rank, a.rank, R, jb);
      const float v = ur.dot(xo, R, red);
      if (tid < 64 && jb + tid < a.rpad) mine[jb + tid] = v;
    }
  }
  if (tid == 0) {
    handoff_reset(a.count + b * a.Hk + g);
    if (a.advance && b == 0 && g == 0) *a.advance += 1;
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
bool al4(const void* p) { return ((uintptr_t)p & 3) == 0; }

}  // namespace
}  // namespace glq

extern "C" int glq_rmsnorm(const void* x, const void* residual, const void* weight, int64_t rows,
                           int64_t dim, float eps, void* out, void* residual_out, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(rows >= 0 && dim > 0, "rows must be >= 0 and dim > 0");
  GLQ_CHECK(dim % 8 == 0 && dim <= kDecThreads * 8 * kNormIters,
            "dim must be a multiple of 8 and <= %d (got %lld)", kDecThreads * 8 * kNormIters,
            (long long)dim);
  GLQ_CHECK(rows < (1ll << 31), "rows must be < 2^31");
  if (rows == 0) return GLQ_OK;
  GLQ_CHECK(x && weight && out && al16(x) && al16(weight) && al16(out),
            "x, weight, out must be non-null and 16-byte aligned");
  GLQ_CHECK(!residual || (residual_out && al16(residual) && al16(residual_out)),
            "a residual needs a 16-byte aligned residual_out");
  rmsnorm_kernel<<<dim3((unsigned)rows), dim3(kDecThreads), 0, (hipStream_t)stream>>>(
      (const __half*)x, (const __half*)residual, (const __half*)weight, (__half*)out,
      (__half*)residual_out, (int)dim, eps);
  GLQ_LAUNCH_CHECK("rmsnorm_kernel");
  return GLQ_OK;
}

extern "C" int glq_rmsnorm_xu(const void* x, const void* residual, const void* weight,
                              int64_t rows, int64_t dim, float eps, void* out,
                              void* residual_out, const void* U, int64_t u_stride, int64_t n_u,
                              int64_t rank, float* parts, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(rows >= 0 && dim > 0, "rows must be >= 0 and dim > 0");
  GLQ_CHECK(rows <= kRxMaxRows, "rows must be <= %d (got %lld)", kRxMaxRows, (long long)rows);
  GLQ_CHECK(dim % 8 == 0 && dim <= kDecThreads * 8 * kNormIters,
            "dim must be a multiple of 8 and <= %d (got %lld)", kDecThreads * 8 * kNormIters,
            (long long)dim);
  GLQ_CHECK(n_u >= 1 && n_u <= 65535, "n_u must be in [1, 65535]");
  GLQ_CHECK(rank > 0 && rank <= 1024 && rank % 8 == 0,
            "rank must be a multiple of 8 in [8, 1024]");
  GLQ_CHECK(u_stride >= dim * rank || n_u == 1, "u_stride must cover a (dim, rank) matrix");
  if (rows == 0) return GLQ_OK;
  GLQ_CHECK(x && weight && out && U && parts && al16(x) && al16(weight) && al16(out) &&
                al16(U) && (n_u == 1 || u_stride % 8 == 0) && ((uintptr_t)parts & 3) == 0,
            "x, weight, out, U must be non-null and 16-byte aligned, parts non-null");
  GLQ_CHECK(!residual || (residual_out && al16(residual) && al16(residual_out)),
            "a residual needs a 16-byte aligned residual_out");
  RxArgs g;
  g.x = (const __half*)x; g.res = (const __half*)residual; g.w = (const __half*)weight;
  g.out = (__half*)out; g.res_out = (__half*)residual_out;
  g.U = (const __half*)U; g.u_stride = u_stride;
  g.part = parts;
  g.M = (int)rows; g.D = (int)dim; g.S = (int)((dim + kLowrankRows - 1) / kLowrankRows);
  g.rank = (int)rank; g.rpad = (int)align_up(rank, 32); g.eps = eps;
  const dim3 grid((unsigned)(n_u * g.S));
  if (rows > kRxPfRows) {
    static size_t attr = 64 * 1024;
    int rc = set_lds_limit(rmsnorm_xu_kernel<4>, kRxLds, attr);
    if (rc) return rc;
    rmsnorm_xu_kernel<4><<<grid, dim3(kDecThreads), kRxLds, (hipStream_t)stream>>>(g);
  } else {
    static size_t attr = 64 * 1024;
    int rc = set_lds_limit(rmsnorm_xu_kernel<0>, kRxLds, attr);
    if (rc) return rc;
    rmsnorm_xu_kernel<0><<<grid, dim3(kDecThreads), kRxLds, (hipStream_t)stream>>>(g);
  }
  GLQ_LAUNCH_CHECK("rmsnorm_xu_kernel");
  return GLQ_OK;
}

extern "C" int glq_qk_norm_rope(const void* q, const void* k, const void* v, int64_t tokens,
                                int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                int64_t q_stride, int64_t q_item_rows, int64_t kv_stride,
                                const void* q_norm_w,
                                const void* k_norm_w, float eps, const void* cos, const void* sin,
                                int64_t cs_stride, void* q_out, void* k_cache, void* v_cache,
                                int64_t max_len, const int64_t* pos, int32_t* len_out,
                                void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(head_dim == kHeadDim, "head_dim must be %d (got %lld)", kHeadDim,
            (long long)head_dim);
  GLQ_CHECK(tokens >= 0 && tokens <= 65535, "tokens must be in [0, 65535]");
  GLQ_CHECK(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && q_heads <= 1024,
            "q_heads must be a positive multiple of kv_heads (<= 1024)");
  GLQ_CHECK(max_len > 0 && max_len < (1ll << 31), "max_len must be in [1, 2^31)");
  GLQ_CHECK(q_stride >= q_heads * head_dim && kv_stride >= kv_heads * head_dim &&
                q_stride % 2 == 0 && kv_stride % 2 == 0 && cs_stride % 2 == 0 && cs_stride >= 0,
            "row strides must cover the heads and be even");
  GLQ_CHECK(q_item_rows >= 0 && q_item_rows % head_dim == 0 &&
                (q_item_rows == 0 || (q_heads * head_dim) % q_item_rows == 0),
            "q_item_rows must be 0 or a multiple of head_dim dividing q_heads * head_dim");
  if (tokens == 0) return GLQ_OK;
  GLQ_CHECK(q && k && v && q_norm_w && k_norm_w && cos && sin && q_out && k_cache && v_cache &&
                pos && len_out,
            "null pointer argument");
  GLQ_CHECK(al4(q) && al4(k) && al4(v) && al4(q_norm_w) && al4(k_norm_w) && al4(cos) &&
                al4(sin) && al4(q_out) && al4(k_cache) && al4(v_cache) && al4(len_out) &&
                ((uintptr_t)pos & 7) == 0,
            "tensor arguments must be 4-byte aligned (pos 8-byte)");
  QkArgs a;
  a.q = (const __half*)q; a.k = (const __half*)k; a.v = (const __half*)v;
  a.q_stride = q_stride; a.kv_stride = kv_stride; a.q_item = (int)q_item_rows;
  a.qw = (const __half*)q_norm_w; a.kw = (const __half*)k_norm_w;
  a.cos = (const __half*)cos; a.sin = (const __half*)sin; a.cs_stride = cs_stride;
  a.q_out = (__half*)q_out; a.k_cache = (__half*)k_cache; a.v_cache = (__half*)v_cache;
  a.pos = pos; a.len_out = len_out;
  a.B = (int)tokens; a.Hq = (int)q_heads; a.Hk = (int)kv_heads; a.max_len = (int)max_len;
  a.eps = eps;
  const int heads = a.Hq + 2 * a.Hk, per = kDecThreads / 64;
  qk_norm_rope_kernel<<<dim3((unsigned)((heads + per - 1) / per), (unsigned)tokens),
                        dim3(kDecThreads), 0, (hipStream_t)stream>>>(a);
  GLQ_LAUNCH_CHECK("qk_norm_rope_kernel");
  return GLQ_OK;
}

extern "C" int64_t glq_decode_attention_workspace_bytes(int64_t tokens, int64_t q_heads,
                                                      int64_t kv_heads, int64_t max_len) {
  using namespace glq;
  if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || max_len <= 0) return -1;
  const int64_t nsplit = (max_len + kAttnChunk - 1) / kAttnChunk;
  const int64_t part = align_up(4 * tokens * q_heads * nsplit * kPartStride, 256);
  return part + align_up(4 * tokens * kv_heads, 256);
}

static int attention_launch(const void* q, const void* k_cache, const void* v_cache,
                            int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t max_len, const int32_t* len, float scale, int64_t* advance,
                            void* out, const void* U, int64_t rank, float* parts,
                            void* workspace, int64_t workspace_bytes, void* stream);

extern "C" int glq_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                                    int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                    int64_t head_dim, int64_t max_len, const int32_t* len,
                                    float scale, int64_t* advance, void* out, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  glq::clear_error();
  return attention_launch(q, k_cache, v_cache, tokens, q_heads, kv_heads, head_dim, max_len, len,
                          scale, advance, out, nullptr, 0, nullptr, workspace, workspace_bytes,
                          stream);
}

extern "C" int glq_decode_attention_xu(const void* q, const void* k_cache, const void* v_cache,
                                       int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                       int64_t head_dim, int64_t max_len, const int32_t* len,
                                       float scale, int64_t* advance, void* out, const void* U,
                                       int64_t rank, float* parts, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(U && parts && rank > 0 && rank <= 1024, "U, parts and 0 < rank <= 1024 required");
  GLQ_CHECK(al16(U) && al4(parts) && rank % 8 == 0,
            "U must be 16-byte aligned, parts 4-byte, rank a multiple of 8");
  return attention_launch(q, k_cache, v_cache, tokens, q_heads, kv_heads, head_dim, max_len, len,
                          scale, advance, out, U, rank, parts, workspace, workspace_bytes,
                          stream);
}

static int attention_launch(const void* q, const void* k_cache, const void* v_cache,
                            int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t max_len, const int32_t* len, float scale, int64_t* advance,
                            void* out, const void* U, int64_t rank, float* parts,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace glq;
  static size_t attr = 64 * 1024, attr_xu = 64 * 1024;
  GLQ_CHECK(head_dim == kHeadDim, "head_dim must be %d (got %lld)", kHeadDim,
            (long long)head_dim);
  GLQ_CHECK(tokens >= 0 && tokens <= 65535, "tokens must be in [0, 65535]");
  GLQ_CHECK(q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 &&
                q_heads / kv_heads <= kAttnMaxRep && kv_heads <= 65535,
            "q_heads must be a multiple of kv_heads with at most %d q heads per KV head",
            kAttnMaxRep);
  GLQ_CHECK(max_len > 0 && max_len <= (1ll << 24), "max_len must be in [1, 2^24]");
  if (tokens == 0) return GLQ_OK;
  const int64_t need = glq_decode_attention_workspace_bytes(tokens, q_heads, kv_heads, max_len);
  GLQ_CHECK(workspace && workspace_bytes >= need,
            "workspace of %lld bytes needed (got %lld); its counters must start zero",
            (long long)need, (long long)workspace_bytes);
  GLQ_CHECK(q && k_cache && v_cache && len && out, "null pointer argument");
  GLQ_CHECK(al16(q) && al16(k_cache) && al16(v_cache) && al4(len) && al16(out) &&
                ((uintptr_t)workspace & 255) == 0 && (!advance || ((uintptr_t)advance & 7) == 0),
            "q, caches and out must be 16-byte aligned, len 4-byte, workspace 256-byte, "
            "advance 8-byte");
  AttnArgs a;
  a.q = (const __half*)q; a.k_cache = (const __half*)k_cache; a.v_cache = (const __half*)v_cache;
  a.len = len; a.advance = advance; a.out = (__half*)out;
  a.B = (int)tokens; a.Hq = (int)q_heads; a.Hk = (int)kv_heads; a.max_len = (int)max_len;
  a.nsplit = (int)((max_len + kAttnChunk - 1) / kAttnChunk);
  a.scale = scale;
  a.part = (float*)workspace;
  a.count = (unsigned*)((char*)workspace +
                        align_up(4 * tokens * q_heads * (int64_t)a.nsplit * kPartStride, 256));
  a.U = (const __half*)U;
  a.xpart = parts;
  a.rank = (int)rank;
  a.rpad = (int)align_up(rank, 32);
  const dim3 grid((unsigned)a.nsplit, (unsigned)kv_heads, (unsigned)tokens);
  if (U) {
    int rc = set_lds_limit(decode_attention_kernel<true>, kAttnLds, attr_xu);
    if (rc) return rc;
    decode_attention_kernel<true><<<grid, dim3(kDecThreads), kAttnLds, (hipStream_t)stream>>>(a);
  } else {
    int rc = set_lds_limit(decode_attention_kernel<false>, kAttnLds, attr);
    if (rc) return rc;
    decode_attention_kernel<false><<<grid, dim3(kDecThreads), kAttnLds, (hipStream_t)stream>>>(a);
  }
  GLQ_LAUNCH_CHECK("decode_attention_kernel");
  return GLQ_OK;
}
