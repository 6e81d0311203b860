// Prefill entry point glq_gemm_lora: argument checks, then the grouped
// dequant-to-fp16 MFMA GEMM of glq_prefill.hip in its dense form (one
// "expert", token rows in order):
//   launch 1  pf_lowrank_kernel   a = fp16(x U), only when U is given (rank
//   (+ finalize)                  <= 128; larger ranks take
//                                 glq_lowrank_xu_batched first)
//   launch 2  pf_gemm_kernel      y = fp16(x W^T + a SV^T + bias) over tiles
//                                 sized to the problem, x read as given
// Reference: gptq_dequant_gemm_kernel (inference/kernels/gptq_matmul.cu:
// 111-213, used for B > 4) and the LoRA tail of GLoRCQLinear.forward
// (inference/quantized_linear.py:338-349).
#include <hip/hip_fp16.h>

#include <algorithm>

#include "glq_internal.h"

namespace glq {
int pf_dense_gemm(const void* x, int64_t M, int64_t K, int64_t N, const int32_t* codes,
                  int bits, const void* scales, const void* zeros, int sym, const void* U,
                  const void* SV, int64_t rank, const void* xU, const void* bias, void* y,
                  void* workspace, int64_t workspace_bytes, hipStream_t s);
int64_t pf_gemm_prefill_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank,
                                        int bits);
}  // namespace glq

namespace {
// ranks above this take the low-rank entry point before the GEMM
constexpr int64_t kInLaunchRank = 128;

int64_t lowrank_block_ws(int64_t M, int64_t K, int64_t rank) {
  const int64_t full = M / 16, tail = M % 16;
  int64_t need = glq_lowrank_workspace_bytes(full > 0 ? full : 1, 16, K, rank);
  if (tail) need = std::max(need, glq_lowrank_workspace_bytes(1, tail, K, rank));
  return glq::align_up(need, 256) + glq::align_up(M * rank * 2, 256);
}
}  // namespace

// Enough for either code width (the plan's token tile depends on it).
extern "C" int64_t glq_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  if (rank < 0) return -1;
  const int64_t pf = std::max(glq::pf_gemm_prefill_workspace_bytes(M, K, N, rank, 2),
                              glq::pf_gemm_prefill_workspace_bytes(M, K, N, rank, 4));
  if (rank > kInLaunchRank) return pf + lowrank_block_ws(M, K, rank);
  return pf;
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
  GLQ_CHECK(sym >= 0 && sym <= 2, "sym must be 0, 1 or 2 (got %d)", sym);
  GLQ_CHECK(group == 128, "the GEMM path takes group 128 (got %lld)", (long long)group);
  GLQ_CHECK(K > 0 && K % 128 == 0 && K < (1 << 24), "K=%lld must be a positive multiple of 128",
            (long long)K);
  GLQ_CHECK(N < (1ll << 30) && M < (1ll << 31) / 2 && M * K < (1ll << 31), "shape too large");
  GLQ_CHECK(x && codes && scales && y && (sym == 1 || zeros), "null data pointer");
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
  GLQ_CHECK(workspace != nullptr && ((uintptr_t)workspace & 255) == 0,
            "a 256-byte aligned workspace of glq_gemm_workspace_bytes is required");
  const int64_t need = glq_gemm_workspace_bytes(M, K, N, lora && !xU ? rank : 0);
  GLQ_CHECK(workspace_bytes >= need, "workspace of %lld bytes needed (got %lld)",
            (long long)need, (long long)workspace_bytes);
  hipStream_t s = (hipStream_t)stream;
  const void* a = xU;
  if (lora && !xU && rank > kInLaunchRank) {
    // a = fp16(x U) by the low-rank entry point (16-row blocks), past the
    // prefill workspace
    char* xw = (char*)workspace + std::max(glq::pf_gemm_prefill_workspace_bytes(M, K, N, rank, 2),
                                           glq::pf_gemm_prefill_workspace_bytes(M, K, N, rank, 4));
    const int64_t xneed = lowrank_block_ws(M, K, rank);
    const int64_t pbytes = xneed - align_up(M * rank * 2, 256);
    __half* abuf = (__half*)(xw + pbytes);
    const int64_t full = M / 16, tail = M % 16;
    if (full > 0) {
      int rc = glq_lowrank_xu_batched(full, x, 16 * K, 16, K, U, 0, rank, abuf, 16 * rank, xw,
                                      pbytes, stream);
      if (rc) return rc;
    }
    if (tail) {
      int rc = glq_lowrank_xu_batched(1, (const __half*)x + full * 16 * K, 0, tail, K, U, 0,
                                      rank, abuf + full * 16 * rank, 0, xw, pbytes, stream);
      if (rc) return rc;
    }
    a = abuf;
  }
  return pf_dense_gemm(x, M, K, N, codes, bits, scales, zeros, sym, a ? nullptr : U,
                       lora ? SV : nullptr, lora ? rank : 0, a, bias, y, workspace,
                       workspace_bytes, s);
}
