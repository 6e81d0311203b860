// Routing keys shared by the MoE decode paths (glq_moe.hip, glq_moe_lane.hip).
#pragma once

#include <hip/hip_fp16.h>
#include <stdint.h>

namespace glq {

// Routing keys: the order (logit descending, expert index ascending) as one
// unsigned compare.  The fp16 logit's bits map to an order-preserving 16-bit
// value (negative: all bits flipped; positive: sign bit set; -0 taken as +0),
// above 0xFFFF - e.  moe_key_logit inverts it.
__device__ __forceinline__ uint32_t moe_key(uint32_t bits, int e) {  // bits: the fp16 pattern
  uint32_t u = bits & 0xFFFFu;
  if (u == 0x8000u) u = 0u;
  u = (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
  return (u << 16) | (uint32_t)(0xFFFF - e);
}
__device__ __forceinline__ float moe_key_logit(uint32_t k) {
  uint32_t u = k >> 16;
  u = (u & 0x8000u) ? (u & 0x7FFFu) : (~u & 0xFFFFu);
  return __half2float(__ushort_as_half((unsigned short)u));
}

}  // namespace glq
