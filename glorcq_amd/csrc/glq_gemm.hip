// Prefill: fused dequant GEMM + low-rank correction for M > 16 tokens
// (the reference's gptq_dequant_gemm_kernel, inference/kernels/gptq_matmul.cu:
// 111-213, used for B > 4, plus the LoRA tail of GLoRCQLinear.forward,
// inference/quantized_linear.py:338-349).
//
//   y[m][n] = sum_g s[n][g] * sum_{k in g} x[m][k] (q[n][k] - z[n][g])
//             + (a SV^T)[m][n] + bias[n],     a = fp16(x U)
//
// gemm_dq_kernel: a workgroup owns a tile of 64 tokens x 64 weight rows; wave
// w computes rows 16w..16w+15 for all 64 tokens (four 16x16 MFMA tiles), so
// each decoded code feeds four MFMAs.  K advances in chunks of 256 codes (two
// groups): the x chunk of the 64 tokens is staged in LDS (double-buffered,
// permuted into the decode order, with per-group sums c1 = sum(operand
// bias * x) and c2 = sum(x)); a wave's codes, scales and zero-points go
// straight to registers, one chunk ahead.  Codes decode exactly into fp16
// 2^e + q (glq_gemv_core.h: decode2/decode4); each group's MFMA sum is
// corrected and scaled in fp32:
//   y += s_g * ((acc_g - c1_g) - z_g * c2_g).
// MFMA k-steps stay inside one group, so all 16 MFMA token rows carry tokens
// (no half-empty operands as in the GEMV's two-groups-per-step layout).
// Epilogue: y += a SV^T (MFMA, a from the x U launch), + bias, fp16 store.
#include <algorithm>

#include "glq_gemv_core.h"

namespace glq {

constexpr int kGemmBM = 64;    // tokens per workgroup tile
constexpr int kGemmBN = 64;    // weight rows per workgroup tile (16 per wave)
constexpr int kGemmKC = 256;   // codes per K chunk (two groups of 128)
constexpr int kGemmXS = kGemmKC + 8;  // halves per staged token row

struct GemmArgs {
  const __half* x;          // (M, K)
  const uint32_t* codes;    // (N, K*b/32)
  const __half* scales;     // (N, G)
  const __half* zeros;      // (N, G) (unused with sym)
  const __half* a;          // (M, rank) fp16 x U, or null
  const __half* sv;         // (N, rank)
  const __half* bias;       // (N,) or null
  __half* y;                // (M, N)
  int M, K, N, G, kw, rank;
};

struct GemmLds {
  int xs, xc, total;  // xs: [2][BM][XS] halves; xc: [2][group 2][c1,c2][half 2][BM] floats
};
__host__ __device__ inline GemmLds gemm_lds() {
  GemmLds L;
  L.xs = 0;
  L.xc = 2 * kGemmBM * kGemmXS * 2;
  L.total = L.xc + 2 * 2 * 2 * 2 * kGemmBM * 4;
  return L;
}

// Staging assignment: thread -> (token m, group gg, half hh) of a chunk: 64
// codes = 8 f16x8 loads.
template <int BITS>
struct GemmStage {
  f16x8 v[8];
  __device__ __forceinline__ void load(const GemmArgs& g, int m0, int k0, int tid) {
    const int m = m0 + (tid >> 2), gg = (tid >> 1) & 1, hh = tid & 1;
    const int kb = k0 + 128 * gg + 64 * hh;
    const bool ok = m < g.M && kb < g.K;
    const __half* src = g.x + (int64_t)(ok ? m : 0) * g.K + (ok ? kb : 0);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = ok ? *(const f16x8*)(src + 8 * u) : f16x8{};
  }
  __device__ __forceinline__ void store(__half* xs, float* xc, int tid) const {
    const int m = tid >> 2, gg = (tid >> 1) & 1, hh = tid & 1;
    float s = 0.f, sb = 0.f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {  // four 16-code blocks
      const f16x8 a = v[2 * blk], b = v[2 * blk + 1];
      f16x8 o0, o1;
      if constexpr (BITS == 2) {  // one word = 16 codes: order 0,8,1,9,..  (perm_src<2>)
        o0 = __builtin_shufflevector(a, b, 0, 8, 1, 9, 2, 10, 3, 11);
        o1 = __builtin_shufflevector(a, b, 4, 12, 5, 13, 6, 14, 7, 15);
        // operand biases (code_bias<2>): pairs (k, k+8) share 1024,256,64,16,4,1024,256,64
        const float p[8] = {(float)a[0] + (float)b[0], (float)a[1] + (float)b[1],
                            (float)a[2] + (float)b[2], (float)a[3] + (float)b[3],
                            (float)a[4] + (float)b[4], (float)a[5] + (float)b[5],
                            (float)a[6] + (float)b[6], (float)a[7] + (float)b[7]};
        sb += 1024.f * (p[0] + p[5]) + 256.f * (p[1] + p[6]) + 64.f * (p[2] + p[7]) +
              16.f * p[3] + 4.f * p[4];
#pragma unroll
        for (int c = 0; c < 8; ++c) s += p[c];
      } else {  // one word = 8 codes: order 0,4,1,5,..  per word (perm_src<4>)
        o0 = __builtin_shufflevector(a, a, 0, 4, 1, 5, 2, 6, 3, 7);
        o1 = __builtin_shufflevector(b, b, 0, 4, 1, 5, 2, 6, 3, 7);
        // operand biases (code_bias<4>): codes 0-3 of a word 1024, codes 4-7 64... per
        // decode4: positions (0,1),(4,5) -> 1024 hold codes {0,4},{2,6}; (2,3),(6,7) -> 64
        // hold codes {1,5},{3,7}
        const float e = (float)a[0] + (float)a[4] + (float)a[2] + (float)a[6] + (float)b[0] +
                        (float)b[4] + (float)b[2] + (float)b[6];
        const float o = (float)a[1] + (float)a[5] + (float)a[3] + (float)a[7] + (float)b[1] +
                        (float)b[5] + (float)b[3] + (float)b[7];
        sb += 1024.f * e + 64.f * o;
        s += e + o;
      }
      f16x8* dst = (f16x8*)(xs + m * kGemmXS + 128 * gg + 64 * hh + 16 * blk);
      dst[0] = o0;
      dst[1] = o1;
    }
    xc[((gg * 2 + 0) * 2 + hh) * kGemmBM + m] = sb;  // c1 half-sum
    xc[((gg * 2 + 1) * 2 + hh) * kGemmBM + m] = s;   // c2 half-sum
  }
};

// One wave's codes, scales and zero-points for one chunk (two groups).
template <int BITS>
struct GemmCodes {
  uint32_t w[2][BITS == 2 ? 2 : 4];
  float s[2], z[2];
  __device__ __forceinline__ void load(const GemmArgs& g, int row, int chunk, int kb, bool sym) {
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int grp = 2 * chunk + gg;
      const bool gv = grp < g.G;
      const int gc = gv ? grp : g.G - 1;
      const uint32_t* base = g.codes + (int64_t)row * g.kw;
      if constexpr (BITS == 2) {  // words 2kb, 2kb+1 of the group's 8
        const u32x2 q = *(const u32x2*)(base + 8 * gc + 2 * kb);
        w[gg][0] = q.x;
        w[gg][1] = q.y;
      } else {  // words 4kb..4kb+3 of the group's 16
        const u32x4 q = *(const u32x4*)(base + 16 * gc + 4 * kb);
        w[gg][0] = q.x;
        w[gg][1] = q.y;
        w[gg][2] = q.z;
        w[gg][3] = q.w;
      }
      const float sc = __half2float(g.scales[(int64_t)row * g.G + gc]);
      s[gg] = gv ? sc : 0.f;
      z[gg] = sym ? (float)(1 << (BITS - 1)) : __half2float(g.zeros[(int64_t)row * g.G + gc]);
    }
  }
};

template <int BITS, bool SYM>
__global__ __launch_bounds__(256, 2) void gemm_dq_kernel(GemmArgs g) {
  extern __shared__ __align__(16) unsigned char smem[];
  const GemmLds L = gemm_lds();
  __half* xs0 = (__half*)(smem + L.xs);
  float* xc0 = (float*)(smem + L.xc);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * kGemmBN, m0 = blockIdx.y * kGemmBM;
  const int row = min(n0 + 16 * wave + li, g.N - 1);
  const int nch = (g.K + kGemmKC - 1) / kGemmKC;
  constexpr uint32_t xor_mask = SYM ? (BITS == 2 ? 0xAAAAAAAAu : 0x88888888u) : 0u;
  const DecodeConsts dk = DecodeConsts::make();

  f32x4 y[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) y[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  GemmStage<BITS> st;
  GemmCodes<BITS> cur, nxt;
  st.load(g, m0, 0, tid);
  cur.load(g, row, 0, kb, SYM);
  st.store(xs0, xc0, tid);
  __syncthreads();

  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < nch;
    if (more) {  // next chunk in flight while this one computes
      st.load(g, m0, (c + 1) * kGemmKC, tid);
      nxt.load(g, row, c + 1, kb, SYM);
    }
    const __half* xs = xs0 + buf * kGemmBM * kGemmXS;
    const float* xc = xc0 + buf * 2 * 2 * 2 * kGemmBM;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      f16x8 bop[4];  // B operands of the group's four MFMA k-steps
      if constexpr (BITS == 2) {
        decode2(cur.w[gg][0] ^ xor_mask, bop[0], bop[1], dk);
        decode2(cur.w[gg][1] ^ xor_mask, bop[2], bop[3], dk);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) bop[j] = decode4(cur.w[gg][j] ^ xor_mask, dk);
      }
      const float sc = cur.s[gg], zc = cur.z[gg];
      const float* c1a = xc + ((gg * 2 + 0) * 2 + 0) * kGemmBM;
      const float* c1b = xc + ((gg * 2 + 0) * 2 + 1) * kGemmBM;
      const float* c2a = xc + ((gg * 2 + 1) * 2 + 0) * kGemmBM;
      const float* c2b = xc + ((gg * 2 + 1) * 2 + 1) * kGemmBM;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const __half* xr = xs + (16 * t + li) * kGemmXS + 128 * gg;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // k-slot kb of step j: 2-bit word 2kb + j/2, half j%2; 4-bit word 4kb + j
          const int off = BITS == 2 ? 16 * (2 * kb + (j >> 1)) + 8 * (j & 1) : 8 * (4 * kb + j);
          acc = mfma_16x16x32(*(const f16x8*)(xr + off), bop[j], acc);
        }
        const int mt = 16 * t + 4 * kb;  // this lane's first token of the tile
        const f32x4 c1 = *(const f32x4*)(c1a + mt) + *(const f32x4*)(c1b + mt);
        const f32x4 c2 = *(const f32x4*)(c2a + mt) + *(const f32x4*)(c2b + mt);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[t][i] += sc * ((acc[i] - c1[i]) - zc * c2[i]);
      }
    }
    if (more) {
      st.store(xs0 + (buf ^ 1) * kGemmBM * kGemmXS, xc0 + (buf ^ 1) * 2 * 2 * 2 * kGemmBM, tid);
      cur = nxt;
    }
    __syncthreads();
  }

  // ---- epilogue: y += a SV^T, + bias, store ----
  if (g.a) {
    for (int j0 = 0; j0 < g.rank; j0 += 32) {
      const int jk = j0 + 8 * kb;
      const bool jv = jk < g.rank;
      const f16x8 bv = jv ? *(const f16x8*)(g.sv + (int64_t)row * g.rank + jk) : f16x8{};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int m = m0 + 16 * t + li;
        const f16x8 av = (jv && m < g.M) ? *(const f16x8*)(g.a + (int64_t)m * g.rank + jk)
                                         : f16x8{};
        y[t] = mfma_16x16x32(av, bv, y[t]);
      }
    }
  }
  const int n = n0 + 16 * wave + li;
  if (n < g.N) {
    const float bn = g.bias ? __half2float(g.bias[n]) : 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * t + 4 * kb + i;
        if (m < g.M) g.y[(int64_t)m * g.N + n] = __float2half(y[t][i] + bn);
      }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

template <int BITS, bool SYM>
int launch_gemm(const GemmArgs& g, hipStream_t s) {
  static size_t attr = 64 * 1024;
  const size_t lds = (size_t)gemm_lds().total;
  int rc = set_lds_limit(gemm_dq_kernel<BITS, SYM>, lds, attr);
  if (rc) return rc;
  const dim3 grid((unsigned)((g.N + kGemmBN - 1) / kGemmBN),
                  (unsigned)((g.M + kGemmBM - 1) / kGemmBM));
  gemm_dq_kernel<BITS, SYM><<<grid, dim3(256), lds, s>>>(g);
  GLQ_LAUNCH_CHECK("gemm_dq_kernel");
  return GLQ_OK;
}

// x U for the GEMM path: the batched low-rank entry point over 16-token
// blocks of x (U shared: stride 0); a lands at the end of the workspace.
int64_t gemm_workspace_need(int64_t M, int64_t K, int64_t rank) {
  if (rank <= 0) return 0;
  const int64_t full = M / 16, tail = M % 16;
  int64_t need = glq_lowrank_workspace_bytes(full > 0 ? full : 1, 16, K, rank);
  if (tail) need = std::max(need, glq_lowrank_workspace_bytes(1, tail, K, rank));
  return align_up(need, 256) + align_up(M * rank * 2, 256);
}

}  // namespace
}  // namespace glq

extern "C" int64_t glq_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank) {
  (void)N;
  if (M <= 0 || K <= 0) return 0;
  return glq::gemm_workspace_need(M, K, rank);
}

extern "C" int glq_gemm_lora(const void* x, int64_t M, int64_t K, int64_t N,
                             const int32_t* codes, int bits, const void* scales,
                             const void* zeros, int64_t group, int sym, const void* U,
                             const void* SV, int64_t rank, const void* xU, const void* bias,
                             void* y, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace glq;
  clear_error();
  GLQ_CHECK(M >= 0 && K >= 0 && N >= 0, "negative size");
  if (M == 0 || N == 0) return GLQ_OK;
  GLQ_CHECK(bits == 2 || bits == 4, "bits must be 2 or 4 (got %d)", bits);
  GLQ_CHECK(group == 128, "the GEMM path takes group 128 (got %lld)", (long long)group);
  GLQ_CHECK(K > 0 && K % 128 == 0 && K < (1 << 24), "K=%lld must be a positive multiple of 128",
            (long long)K);
  GLQ_CHECK(N < (1ll << 30) && M < (1ll << 31) / 2, "shape too large");
  GLQ_CHECK(x && codes && scales && y && (sym || zeros), "null data pointer");
  const bool lora = SV != nullptr && rank > 0;
  if (lora) {
    GLQ_CHECK(rank % 8 == 0 && rank <= 512, "rank=%lld must be a multiple of 8, <= 512",
              (long long)rank);
    GLQ_CHECK(U != nullptr || xU != nullptr, "LoRA needs U or a precomputed xU");
  }
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  GLQ_CHECK(al16(x) && al16(codes) && (!lora || al16(SV)) && (!xU || al16(xU)) &&
                (!U || al16(U)),
            "x, codes, U, SV and xU must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const __half* a = nullptr;
  if (lora) {
    if (xU) {
      a = (const __half*)xU;
    } else {
      const int64_t need = gemm_workspace_need(M, K, rank);
      GLQ_CHECK(workspace != nullptr && workspace_bytes >= need,
                "workspace of %lld bytes needed (got %lld)", (long long)need,
                (long long)workspace_bytes);
      GLQ_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
      const int64_t part = need - align_up(M * rank * 2, 256);
      __half* abuf = (__half*)((char*)workspace + part);
      const int64_t full = M / 16, tail = M % 16;
      if (full > 0) {
        int rc = glq_lowrank_xu_batched(full, x, 16 * K, 16, K, U, 0, rank, abuf, 16 * rank,
                                        workspace, part, stream);
        if (rc) return rc;
      }
      if (tail) {
        int rc = glq_lowrank_xu_batched(1, (const __half*)x + full * 16 * K, 0, tail, K, U, 0,
                                        rank, abuf + full * 16 * rank, 0, workspace, part,
                                        stream);
        if (rc) return rc;
      }
      a = abuf;
    }
  }
  GemmArgs g;
  g.x = (const __half*)x;
  g.codes = (const uint32_t*)codes;
  g.scales = (const __half*)scales;
  g.zeros = (const __half*)zeros;
  g.a = a;
  g.sv = lora ? (const __half*)SV : nullptr;
  g.bias = (const __half*)bias;
  g.y = (__half*)y;
  g.M = (int)M;
  g.K = (int)K;
  g.N = (int)N;
  g.G = (int)(K / 128);
  g.kw = (int)(K * bits / 32);
  g.rank = lora ? (int)rank : 0;
  if (bits == 2) return sym ? launch_gemm<2, true>(g, s) : launch_gemm<2, false>(g, s);
  return sym ? launch_gemm<4, true>(g, s) : launch_gemm<4, false>(g, s);
}
