// Fused dequant-GEMV + low-rank correction for decode (1 <= M <= 16), gfx950.
//
//   y[m,n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) x[m,k]
//          + sum_j a[m,j] SV[n,j] + bias[n],          a = fp16(x U)
//
// Reference semantics: GLoRCQLinear.forward (inference/quantized_linear.py:
// 286-355) = gptq dequant-matmul (inference/kernels/__init__.py:284-346,
// kernels/gptq_matmul.cu:42-98) + LoRA `y + (x @ U) @ SV.T`.
//
// Design (MI355X-first, not a translation of the CUDA kernel):
//  * One launch does everything.  A workgroup takes a job ticket from an
//    atomic counter.  The first `items*P` tickets are low-rank producers: each
//    computes a K-slice partial of a = x U (U rows streamed with 16-byte loads,
//    partials reduced across lanes with wave shuffles and across waves in LDS)
//    and publishes it with an agent-scope release.  Every later ticket is a
//    consumer tile of 16*T output rows.  A consumer streams packed codes and
//    only waits for its item's producers in the epilogue; producers always
//    hold smaller tickets, so they are resident and the wait always ends (and
//    is bounded anyway: past a spin limit it sets the workspace error word).
//    The last workgroup to exit zeroes the counters for the next launch.
//  * Codes are decoded in registers straight into fp16 MFMA operands with one
//    v_and_or per two codes: code bits land in the fp16 mantissa under an
//    exponent chosen per bit position, so each operand is (2^e + q) exactly.
//    The 2^e bias is removed once per 128-code chunk with a precomputed
//    sum_k 2^e(k) x[m,k]; zero-points likewise with sum_k x[m,k]; the group
//    scale multiplies the chunk's fp32 MFMA result.  No per-weight dequant.
//  * v_mfma_f32_16x16x32_f16: A = 16 weight rows x 32 codes, B = 32 codes x
//    16 tokens (rows m >= M read as zero), fp32 accumulate.  Lane group
//    kb = lane/16 owns 32 contiguous codes of every 128-code chunk, loaded as
//    one 8-byte (2-bit) or 16-byte (4-bit) vector per row; x is staged once
//    per workgroup in LDS in the matching permuted order.
//  * The 4 waves of a workgroup split K; partial tiles are summed in LDS, then
//    the correction a SV^T is two more MFMAs per tile on the same accumulator.

#include <hip/hip_fp16.h>
#include <stdlib.h>

#include "glq_internal.h"

namespace glq {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct GemvArgs {
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
  const __half* xu;
  int64_t xu_es;
  int items, M, K, N, G, group, rank, sym;
  int P;        // low-rank producer jobs per item (0: none)
  int ks;       // U rows per producer job
  int tiles;    // consumer jobs per item
  int kw;       // int32 words per weight row
  int rpad;     // rank rounded up to 32
  int kp;       // codes per K-phase staged in LDS (multiple of group)
  int xstride;  // halves per token row of staged x in LDS (kp + 8)
  int apad;     // halves per token row of staged a in LDS
  unsigned* ctr;
  float* apart;  // (items, P, M, rpad)
  int spin_limit;
};

// Dynamic LDS layout of a consumer workgroup (byte offsets, 16-byte aligned).
struct LdsLayout {
  int xs, xsum, xbias, s, z, red, a, total;
};

__host__ __device__ inline int al16(int v) { return (v + 15) & ~15; }

__host__ __device__ inline LdsLayout lds_layout(int M, int K, int G, int T, int xstride,
                                                int apad) {
  const int nch = K >> 7;
  LdsLayout L;
  int o = 0;
  L.xs = o;    o += al16(M * xstride * 2);
  L.xsum = o;  o += al16(M * nch * 4);
  L.xbias = o; o += al16(M * nch * 4);
  L.s = o;     o += al16(G * 16 * T * 4);
  L.z = o;     o += al16(G * 16 * T * 4);
  L.red = o;   o += 4 * T * 64 * 16;
  L.a = o;     o += al16(M * apad * 2);
  L.total = o;
  return L;
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

// ---------------------------------------------------------------------------
// Low-rank producer: apart[item][p][m][j] = sum_{k in slice p} x[m,k] U[k,j]
// ---------------------------------------------------------------------------
__device__ void gemv_producer(const GemvArgs& a, int item, int p,
                              float* red /* 4*4*64 floats of LDS */) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j8 = tid & 7, kr = tid >> 3;  // kr in 0..31
  const int k0 = p * a.ks;
  const int k1 = min(a.K, k0 + a.ks);
  const __half* U = a.u + (int64_t)item * a.u_es;
  const __half* X = a.x + (int64_t)item * a.x_es;
  float* out = a.apart + ((int64_t)item * a.P + p) * a.M * a.rpad;
  for (int jb = 0; jb < a.rpad; jb += 64) {
    const int j = jb + 8 * j8;
    const bool jv = j < a.rank;
    for (int mb = 0; mb < a.M; mb += 4) {
      float acc[4][8];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[mm][c] = 0.f;
      for (int k = k0 + kr; k < k1; k += 32) {
        f16x8 u = {};
        if (jv) u = *(const f16x8*)(U + (int64_t)k * a.rank + j);
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
          if (mb + mm < a.M) {
            const float xv = __half2float(X[(int64_t)(mb + mm) * a.K + k]);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[mm][c] += xv * (float)u[c];
          }
        }
      }
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
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
        for (int mm = 0; mm < 4; ++mm)
#pragma unroll
          for (int c = 0; c < 8; ++c)
            red[(wave * 4 + mm) * 64 + 8 * lane + c] = acc[mm][c];
      }
      __syncthreads();
      {
        const int mm = tid >> 6, jj = tid & 63;
        if (mb + mm < a.M && jb + jj < a.rpad) {
          const float s = red[(0 * 4 + mm) * 64 + jj] + red[(1 * 4 + mm) * 64 + jj] +
                          red[(2 * 4 + mm) * 64 + jj] + red[(3 * 4 + mm) * 64 + jj];
          out[(int64_t)(mb + mm) * a.rpad + jb + jj] = s;
        }
      }
      __syncthreads();
    }
  }
  // Publish: every thread's stores are released at agent scope before the
  // done counter moves.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0)
    __hip_atomic_fetch_add(a.ctr + kCtrDone + item, 1u, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Consumer: 16*T output rows of one item.
// ---------------------------------------------------------------------------
template <int BITS, int T>
__device__ void gemv_consumer(const GemvArgs& a, int item, int tile,
                              unsigned char* smem) {
  constexpr int R = 16 * T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kb = lane >> 4;
  const int M = a.M, K = a.K, N = a.N, G = a.G;
  const int KP = a.kp;        // codes per K-phase (multiple of the group size)
  const int ncp = KP >> 7;    // 128-code chunks per phase
  const int cpg = a.group >> 7;  // chunks per quantization group
  const int gp = KP / a.group;   // groups per phase
  const int r0 = tile * R;

  const LdsLayout L = lds_layout(M, KP, gp, T, a.xstride, a.apad);
  __half* xs = (__half*)(smem + L.xs);      // M x xstride, permuted x of the phase
  float* xsum = (float*)(smem + L.xsum);    // M x ncp
  float* xbias = (float*)(smem + L.xbias);  // M x ncp
  float* s_l = (float*)(smem + L.s);        // gp x R scales
  float* z_l = (float*)(smem + L.z);        // gp x R zero-points
  f32x4* red = (f32x4*)(smem + L.red);      // 4 x T x 64 partial tiles
  __half* a_l = (__half*)(smem + L.a);      // M x apad low-rank factor a

  const __half* X = a.x + (int64_t)item * a.x_es;
  const __half* S = a.scales + (int64_t)item * a.sz_es;
  const __half* Z = a.zeros + (int64_t)item * a.sz_es;
  const uint32_t* C = a.codes + (int64_t)item * a.codes_es;
  const uint32_t xor_mask = a.sym ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  const bool mv = li < M;
  int64_t roff[T];
#pragma unroll
  for (int t = 0; t < T; ++t)
    roff[t] = (int64_t)min(r0 + t * 16 + li, N - 1) * a.kw + kb * BITS;
  f32x4 yacc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) yacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += KP) {
    const int kl = min(KP, K - k0);  // codes in this phase
    const int nchl = kl >> 7;
    // ---- stage x (permuted to operand order) and its per-chunk sums ----
    {
      const int nb = kl >> 4;  // 16-code blocks per token row in this phase
      const int total = M * nb;
      for (int base = 0; base < total; base += 256) {
        const int idx = base + tid;
        const bool v = idx < total;
        float s = 0.f, sb = 0.f;
        int m = 0, blk = 0;
        if (v) {
          m = idx / nb;
          blk = idx - m * nb;
          const f16x8* src = (const f16x8*)(X + (int64_t)m * K + k0 + blk * 16);
          f16x8 in0 = src[0], in1 = src[1];
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
            sb += code_bias<BITS>(pos) * f;
          }
          f16x8 o0, o1;
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            o0[c] = o[c];
            o1[c] = o[8 + c];
          }
          f16x8* dst = (f16x8*)(xs + (int64_t)m * a.xstride + blk * 16);
          dst[0] = o0;
          dst[1] = o1;
        }
        // 8 consecutive blocks form one 128-code chunk (nb % 8 == 0).
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        sb += __shfl_xor(sb, 1);
        sb += __shfl_xor(sb, 2);
        sb += __shfl_xor(sb, 4);
        if (v && (idx & 7) == 0) {
          xsum[m * ncp + (blk >> 3)] = s;
          xbias[m * ncp + (blk >> 3)] = sb;
        }
      }
    }
    // ---- stage this phase's scales / zero-points, transposed to [g][row] ----
    {
      const int g0 = k0 / a.group;
      const int gl = kl / a.group;
      const float zsym = (float)(1 << (BITS - 1));
      for (int idx = tid; idx < R * gl; idx += 256) {
        const int row = idx / gl, g = idx - row * gl;
        const int n = min(r0 + row, N - 1);
        s_l[g * R + row] = __half2float(S[(int64_t)n * G + g0 + g]);
        z_l[g * R + row] = a.sym ? zsym : __half2float(Z[(int64_t)n * G + g0 + g]);
      }
    }
    __syncthreads();

    // ---- main loop: this wave's share of the phase's chunks ----
    const int c_begin = (wave * nchl) >> 2, c_end = ((wave + 1) * nchl) >> 2;
    const int cg0 = k0 >> 7;  // global index of the phase's first chunk
    for (int ch = c_begin; ch < c_end; ++ch) {
      uint32_t wv[T][BITS];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const uint32_t* p = C + roff[t] + (cg0 + ch) * (4 * BITS);
        if constexpr (BITS == 2) {
          const u32x2 q = *(const u32x2*)p;
          wv[t][0] = q.x;
          wv[t][1] = q.y;
        } else {
          const u32x4 q = *(const u32x4*)p;
          wv[t][0] = q.x;
          wv[t][1] = q.y;
          wv[t][2] = q.z;
          wv[t][3] = q.w;
        }
      }
      f16x8 bx[4];
      float c1 = 0.f, c2 = 0.f;
      if (mv) {
        const f16x8* xp = (const f16x8*)(xs + (int64_t)li * a.xstride + ch * 128 + kb * 32);
#pragma unroll
        for (int j = 0; j < 4; ++j) bx[j] = xp[j];
        c1 = xbias[li * ncp + ch];
        c2 = xsum[li * ncp + ch];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) bx[j] = f16x8{};
      }
      const int g = ch / cpg;  // group index within the phase
#pragma unroll
      for (int t = 0; t < T; ++t) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if constexpr (BITS == 2) {
          f16x8 s0, s1, s2, s3;
          decode2(wv[t][0] ^ xor_mask, s0, s1);
          decode2(wv[t][1] ^ xor_mask, s2, s3);
          acc = mfma_16x16x32(s0, bx[0], acc);
          acc = mfma_16x16x32(s1, bx[1], acc);
          acc = mfma_16x16x32(s2, bx[2], acc);
          acc = mfma_16x16x32(s3, bx[3], acc);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc = mfma_16x16x32(decode4(wv[t][j] ^ xor_mask), bx[j], acc);
        }
        const f32x4 sc = *(const f32x4*)(s_l + g * R + t * 16 + 4 * kb);
        const f32x4 zc = *(const f32x4*)(z_l + g * R + t * 16 + 4 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          yacc[t][i] += sc[i] * ((acc[i] - c1) - zc[i] * c2);
      }
    }
    __syncthreads();  // the next phase overwrites the staged x / scales
  }

  // ---- sum the 4 waves' K-partials ----
#pragma unroll
  for (int t = 0; t < T; ++t) red[(wave * T + t) * 64 + lane] = yacc[t];

  // ---- low-rank factor a (M x rank) into LDS ----
  const bool lora = a.rank > 0 && a.sv != nullptr;
  if (lora && a.xu == nullptr && tid == 0) {
    int it = 0;
    while (__hip_atomic_load(a.ctr + kCtrDone + item, __ATOMIC_ACQUIRE,
                             __HIP_MEMORY_SCOPE_AGENT) < (unsigned)a.P) {
      if (++it > a.spin_limit) {
        __hip_atomic_store(a.ctr + kCtrError, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  if (lora) {
    if (a.xu == nullptr) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const float* ap = a.apart + (int64_t)item * a.P * M * a.rpad;
      for (int idx = tid; idx < M * a.rpad; idx += 256) {
        float s = 0.f;
        for (int p = 0; p < a.P; ++p) s += ap[(int64_t)p * M * a.rpad + idx];
        const int m = idx / a.rpad, j = idx - m * a.rpad;
        a_l[m * a.apad + j] = __float2half(s);
      }
    } else {
      const __half* xu = a.xu + (int64_t)item * a.xu_es;
      for (int idx = tid; idx < M * a.rpad; idx += 256) {
        const int m = idx / a.rpad, j = idx - m * a.rpad;
        a_l[m * a.apad + j] = j < a.rank ? xu[(int64_t)m * a.rank + j] : __float2half(0.f);
      }
    }
  }
  __syncthreads();

  // ---- epilogue: wave w finishes tiles t = w, w+4, ... ----
  for (int t = wave; t < T; t += 4) {
    f32x4 y = red[(0 * T + t) * 64 + lane];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const f32x4 o = red[(w * T + t) * 64 + lane];
      y += o;
    }
    if (lora) {
      const int rowA = min(r0 + t * 16 + li, N - 1);
      const __half* svr = a.sv + (int64_t)item * a.sv_es + (int64_t)rowA * a.rank;
      for (int s = 0; s < a.rpad; s += 32) {
        const int j = s + 8 * kb;
        f16x8 av = {}, bv = {};
        if (j < a.rank) av = *(const f16x8*)(svr + j);
        if (mv) bv = *(const f16x8*)(a_l + li * a.apad + j);
        y = mfma_16x16x32(av, bv, y);
      }
    }
    if (mv) {
      __half* Y = a.y + (int64_t)item * a.y_es + (int64_t)li * N;
      const __half* B = a.bias ? a.bias + (int64_t)item * a.bias_es : nullptr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = r0 + t * 16 + 4 * kb + i;
        if (n < N) {
          float v = y[i];
          if (B) v += __half2float(B[n]);
          Y[n] = __float2half(v);
        }
      }
    }
  }
}

template <int BITS, int T>
__global__ __launch_bounds__(256) void gemv_lora_kernel(GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_job;
  __shared__ int s_last;
  const int tid = threadIdx.x;
  if (tid == 0)
    s_job = (int)__hip_atomic_fetch_add(a.ctr + kCtrTicket, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int job = s_job;
  const int nprod = a.items * a.P;
  if (job < nprod) {
    gemv_producer(a, job / a.P, job - (job / a.P) * a.P, (float*)smem);
  } else if (job < nprod + a.items * a.tiles) {
    const int c = job - nprod;
    gemv_consumer<BITS, T>(a, c / a.tiles, c - (c / a.tiles) * a.tiles, smem);
  }
  // Exit protocol: the last workgroup resets the counters for the next launch.
  __syncthreads();
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(a.ctr + kCtrExit, 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == gridDim.x - 1;
  }
  __syncthreads();
  if (s_last) {
    for (int i = tid; i < a.items; i += 256)
      __hip_atomic_store(a.ctr + kCtrDone + i, 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(a.ctr + kCtrTicket, 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctr + kCtrExit, 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kProducerRows = 256;  // U rows per producer job
constexpr int kMaxLds = 160 * 1024;

static int64_t producer_jobs(int64_t K) { return (K + kProducerRows - 1) / kProducerRows; }

static int64_t apart_offset(int64_t items) {
  return align_up(4 * (kCtrDone + items), 256);
}

static int64_t workspace_bytes(int64_t items, int64_t M, int64_t K, int64_t rank) {
  const int64_t rpad = align_up(rank, 32);
  const int64_t P = rank > 0 ? producer_jobs(K) : 0;
  return apart_offset(items) + align_up(items * P * M * rpad * 4, 256);
}

static size_t lds_bytes(int M, int KP, int group, int T, int apad) {
  return (size_t)lds_layout(M, KP, KP / group, T, KP + 8, apad).total;
}

// Codes per K-phase: the whole K when x fits the staging budget, else the
// largest multiple of the group size that does.
constexpr int kXStageBudget = 40 * 1024;
static int64_t phase_len(int64_t M, int64_t K, int64_t group) {
  int64_t kp = (kXStageBudget / (2 * M) - 8) / group * group;
  if (kp < group) kp = group;
  return kp >= K ? K : kp;
}

template <int BITS, int T>
static int launch_t(const GemvArgs& a, int grid, size_t lds, hipStream_t s) {
  // Opt in to more than 64 KB of dynamic LDS only when a launch needs it.
  static size_t attr_bytes = 64 * 1024;
  if (lds > attr_bytes) {
    GLQ_HIP(hipFuncSetAttribute((const void*)gemv_lora_kernel<BITS, T>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_bytes = lds;
  }
  gemv_lora_kernel<BITS, T><<<dim3(grid), dim3(256), lds, s>>>(a);
  GLQ_LAUNCH_CHECK("gemv_lora_kernel");
  return GLQ_OK;
}

static int pick_tiles(int64_t items, int64_t N) {
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

static int gemv_impl(int64_t items, const void* x, int64_t x_stride, int64_t M,
                     int64_t K, int64_t N, const int32_t* codes,
                     int64_t codes_stride, int bits, const void* scales,
                     const void* zeros, int64_t sz_stride, int64_t group, int sym,
                     const void* U, int64_t u_stride, const void* SV,
                     int64_t sv_stride, int64_t rank, const void* xU,
                     int64_t xu_stride, const void* bias, int64_t bias_stride,
                     void* y, int64_t y_stride, void* workspace,
                     int64_t workspace_bytes_given, void* stream) {
  clear_error();
  GLQ_CHECK(items >= 0 && M >= 0 && K >= 0 && N >= 0, "negative size");
  if (items == 0 || M == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(bits == 2 || bits == 4, "bits must be 2 or 4 (got %d)", bits);
  GLQ_CHECK(M <= 16, "GEMV path takes 1 <= M <= 16 rows (got M=%lld)", (long long)M);
  GLQ_CHECK(K > 0 && K % 128 == 0, "K=%lld must be a positive multiple of 128", (long long)K);
  GLQ_CHECK(group > 0 && group % 128 == 0 && K % group == 0,
            "group=%lld must be a multiple of 128 dividing K=%lld", (long long)group,
            (long long)K);
  GLQ_CHECK(N < (1ll << 30) && K < (1ll << 24), "shape too large");
  GLQ_CHECK(x && codes && scales && y && (sym || zeros), "null data pointer");
  const bool lora = SV != nullptr && rank > 0;
  if (lora) {
    GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
              (long long)rank);
    GLQ_CHECK(U != nullptr || xU != nullptr, "LoRA needs U or a precomputed xU");
  }
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x) && al16(codes) && (!lora || al16(SV)) && (!lora || !U || al16(U)),
            "x, codes, U and SV must be 16-byte aligned");
  GLQ_CHECK(items == 1 || (x_stride % 8 == 0 && codes_stride % 4 == 0 &&
                           (!lora || sv_stride % 8 == 0) && (!lora || !U || u_stride % 8 == 0)),
            "item strides must keep 16-byte alignment");
  const int64_t G = K / group;
  const int64_t P = (lora && xU == nullptr) ? producer_jobs(K) : 0;
  const int64_t need = workspace_bytes(items, M, K, lora ? rank : 0);
  GLQ_CHECK(workspace != nullptr && workspace_bytes_given >= need,
            "workspace of %lld bytes needed (got %lld)", (long long)need,
            (long long)workspace_bytes_given);
  GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");

  const int T = pick_tiles(items, N);
  GemvArgs a;
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
  a.items = (int)items;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.G = (int)G;
  a.group = (int)group;
  a.rank = lora ? (int)rank : 0;
  a.sym = sym ? 1 : 0;
  a.P = (int)P;
  a.ks = kProducerRows;
  a.tiles = (int)((N + 16 * T - 1) / (16 * T));
  a.kw = (int)(K * bits / 32);
  a.rpad = (int)align_up(a.rank, 32);
  a.kp = (int)phase_len(M, K, group);
  a.xstride = a.kp + 8;
  a.apad = a.rpad + 8;
  a.ctr = (unsigned*)workspace;
  a.apart = (float*)((char*)workspace + apart_offset(items));
  a.spin_limit = 1 << 20;

  const size_t lds = lds_bytes(a.M, a.kp, a.group, T, a.apad);
  GLQ_CHECK(lds <= (size_t)kMaxLds,
            "M*K too large for the GEMV path (needs %zu bytes of LDS)", lds);
  const int64_t grid = items * P + items * a.tiles;
  GLQ_CHECK(grid < (1ll << 31), "too many workgroups");
  hipStream_t s = (hipStream_t)stream;
  if (bits == 2) {
    if (T == 1) return launch_t<2, 1>(a, (int)grid, lds, s);
    if (T == 2) return launch_t<2, 2>(a, (int)grid, lds, s);
    return launch_t<2, 4>(a, (int)grid, lds, s);
  }
  if (T == 1) return launch_t<4, 1>(a, (int)grid, lds, s);
  if (T == 2) return launch_t<4, 2>(a, (int)grid, lds, s);
  return launch_t<4, 4>(a, (int)grid, lds, s);
}

}  // namespace glq

using namespace glq;

extern "C" {

int64_t glq_gemv_workspace_bytes(int64_t items, int64_t M, int64_t K, int64_t N,
                                 int64_t rank) {
  (void)N;
  if (items < 0 || M < 0 || K < 0 || rank < 0) return -1;
  return workspace_bytes(items, M, K, rank);
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

}  // extern "C"
