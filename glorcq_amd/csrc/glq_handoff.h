// Data handed between the workgroups of one launch (split-K partials, router
// logits) and the arrival counters that tell the last workgroup it may read
// them.
//
// gfx950 has one L2 per XCD, and those L2s are not coherent with each other
// for plain stores: a device-scope fence (__threadfence()) writes back and
// invalidates the whole L2 of the XCD, which costs microseconds when many
// workgroups arrive at once.  Instead the handed-over data goes out as
// agent-scope atomic stores (global_store ... sc1: coherent across the L2s)
// and comes back as agent-scope atomic loads; each workgroup waits for its
// own stores to complete (s_waitcnt vmcnt(0)) before one thread bumps the
// counter with an agent-scope atomic add, so every store of a workgroup that
// has arrived is visible to the workgroup that reads the counter's last value.
// Data read by later launches needs none of this (kernel boundaries are
// device-scope release/acquire points).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace glq {

template <class T>
__device__ __forceinline__ void handoff_put(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T handoff_get(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread of the workgroup calls it after its handoff_put stores; returns
// (to every thread) whether this workgroup is the n-th and last to arrive on
// *cnt, which the last one must leave at zero (handoff_reset) once it has
// read the others' data.  `flag` is an int in LDS.
__device__ __forceinline__ bool handoff_arrive(unsigned* cnt, unsigned n, int* flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
  __syncthreads();
  return *flag != 0;
}
__device__ __forceinline__ void handoff_reset(unsigned* cnt) {
  __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// p[0] + p[stride] + ... + p[(n-1) stride] of data handed over inside the
// launch (agent-scope loads), in that order, loads in batches of 8 (the
// order and the zeros of sum_strided, glq_gemv_core.h).
__device__ __forceinline__ float sum_strided_coh(const float* p, int64_t stride, int n) {
  float s = 0.f;
  for (int q0 = 0; q0 < n; q0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = q0 + u < n ? handoff_get(p + (int64_t)(q0 + u) * stride) : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  return s;
}

}  // namespace glq
