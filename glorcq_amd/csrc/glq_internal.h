// Internal helpers shared by the HIP translation units of libglorcq_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/glorcq_hip.h"

namespace glq {

// Per-thread message of the last failed entry point.
void set_error(const char* fmt, ...);
void clear_error();

}  // namespace glq

// Argument check: records the message and returns GLQ_ERR_INVALID from the
// enclosing C entry point (the analogue of TORCH_CHECK in the reference host
// code, inference/kernels/gptq_matmul.cu:232-267).
#define GLQ_CHECK(cond, ...)            \
  do {                                  \
    if (!(cond)) {                      \
      glq::set_error(__VA_ARGS__);      \
      return GLQ_ERR_INVALID;           \
    }                                   \
  } while (0)

// HIP call check.
#define GLQ_HIP(call)                                                       \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess) {                                                 \
      glq::set_error("%s failed: %s", #call, hipGetErrorString(e_));        \
      return GLQ_ERR_HIP;                                                   \
    }                                                                       \
  } while (0)

// Launch check after every kernel launch (the reference has none).
#define GLQ_LAUNCH_CHECK(name)                                              \
  do {                                                                      \
    hipError_t e_ = hipGetLastError();                                      \
    if (e_ != hipSuccess) {                                                 \
      glq::set_error("launch of %s failed: %s", name, hipGetErrorString(e_)); \
      return GLQ_ERR_HIP;                                                   \
    }                                                                       \
  } while (0)

namespace glq {
inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// MoE decode steps of at most this many tokens take the lane path
// (glq_moe_lane.hip) when their shapes fit it; both entry points return -1 /
// an error when it does not.
constexpr int kMoeLaneMaxB = 16;
// Both MoE decode paths start their workspace tables at kMoeWsHeader bytes.
// The header holds arrival counters, zero between steps: word 0 (the
// many-token router), bytes 64 .. 255 (the lane path's per-token router
// counters), bytes 1024 .. 2559 and 2560 .. 4095 (the lane path's token-tile
// row-block counters of the shared gate/up and the shared down), bytes 4096
// .. 8191 (the lane path's (token, row block) combine counters).
constexpr int64_t kMoeWsHeader = 8192;
constexpr int kMoeCombineCnt = 1024;
constexpr int kMoeT16MaxRB = 384;  // row blocks a token-tile role may count
int64_t moe_lane_workspace_bytes(const glq_moe_params* p);
int moe_lane_decode(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                    hipStream_t s);

// Raises a kernel's dynamic-LDS limit to `lds` bytes once (attr_bytes caches
// the limit already set for that kernel).
template <class KernelFn>
int set_lds_limit(KernelFn fn, size_t lds, size_t& attr_bytes) {
  if (lds > attr_bytes) {
    GLQ_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds));
    attr_bytes = lds;
  }
  return GLQ_OK;
}
}  // namespace glq
