// Packed-code codec kernels: pack, unpack and exact fp16 dequantization, plus
// the library's error state and workspace utilities.
//
// Bit layout (the reference's LSB-first convention, inference/kernels/
// __init__.py:113-118 and inference/quantized_linear.py:115-146, widened from
// uint8 to int32 words): code k of row n is bits [b*(k%cpw), b*(k%cpw)+b) of
// word n*(K/cpw) + k/cpw, cpw = 32/b codes per word.

#include <hip/hip_fp16.h>
#include <string.h>

#include "glq_internal.h"

namespace glq {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

// One thread per packed word: emits cpw codes.
template <int BITS>
__global__ void unpack_kernel(const uint32_t* __restrict__ codes, int64_t words,
                              int sym, int32_t* __restrict__ out) {
  constexpr int CPW = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= words) return;
  uint32_t v = codes[w];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    int32_t q = (int32_t)((v >> (BITS * c)) & MASK);
    if (sym == 1 && q >= (1 << (BITS - 1))) q -= (1 << BITS);  // two's complement
    if (sym == 2) q -= (1 << (BITS - 1));                       // stored offset by 2^(b-1)
    out[w * CPW + c] = q;
  }
}

// One thread per packed word: emits cpw fp16 weights, each rounded exactly as
// the reference's fp16 dequant loop does: fp16(fp16(q - z) * s) (sym: q * s;
// sym == 2: q is the stored code minus 2^(b-1)).
template <int BITS>
__global__ void dequant_kernel(const uint32_t* __restrict__ codes, int64_t N,
                               int64_t K, const __half* __restrict__ scales,
                               const __half* __restrict__ zeros, int64_t group,
                               int sym, __half* __restrict__ W) {
  constexpr int CPW = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t kw = K / CPW;
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= N * kw) return;
  const int64_t n = w / kw;
  const int64_t k0 = (w % kw) * CPW;
  const int64_t G = K / group;
  uint32_t v = codes[w];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const int64_t k = k0 + c;
    const int64_t g = k / group;
    int32_t q = (int32_t)((v >> (BITS * c)) & MASK);
    __half s = scales[n * G + g];
    __half wq;
    if (sym == 1) {
      if (q >= (1 << (BITS - 1))) q -= (1 << BITS);
      wq = __hmul(__int2half_rn(q), s);
    } else {
      if (sym == 2) q -= (1 << (BITS - 1));
      wq = __hmul(__hsub(__int2half_rn(q), zeros[n * G + g]), s);
    }
    W[n * K + k] = wq;
  }
}

// One thread per output word.
template <int BITS>
__global__ void pack_kernel(const int32_t* __restrict__ q, int64_t words,
                            uint32_t* __restrict__ codes) {
  constexpr int CPW = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= words) return;
  uint32_t v = 0;
#pragma unroll
  for (int c = 0; c < CPW; ++c)
    v |= ((uint32_t)q[w * CPW + c] & MASK) << (BITS * c);
  codes[w] = v;
}

}  // namespace glq

using namespace glq;

// LoRA factor dequantization (load time): out[r][c] = fp16((q / maxval) * scale)
// in fp32, maxval = 2^(nbits-1) - 1, q from an int8 container or from int4
// nibbles packing row pairs (row 2i in the low nibble of byte row i, row 2i+1
// in the high nibble, value - 7); scale per column (cols,) or per row
// (rows, 1).  The reference's _dequant_intN / _unpack_int4
// (inference/model_builder.py:69-80, cross_layer_share.py:584-649) followed
// by .half(): the same fp32 operations in the same order, so the result is
// bit-identical.  One thread per output element.
__global__ void dequant_factor_kernel(const int8_t* __restrict__ q8,
                                      const uint8_t* __restrict__ q4, int64_t rows,
                                      int64_t cols, const __half* __restrict__ scale,
                                      int per_row, float maxval, __half* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  const int64_t r = i / cols, c = i - r * cols;
  int qv;
  if (q4) {
    const uint8_t b = q4[(r >> 1) * cols + c];
    qv = (int)((r & 1) ? (b >> 4) : (b & 0xf)) - 7;
  } else {
    qv = q8[i];
  }
  const float sc = __half2float(scale[per_row ? r : c]);
  out[i] = __float2half_rn(((float)qv / maxval) * sc);
}

static int check_codec_shape(int64_t N, int64_t K, int bits) {
  GLQ_CHECK(bits == 2 || bits == 4, "bits must be 2 or 4 (got %d)", bits);
  GLQ_CHECK(N >= 0 && K >= 0, "negative shape N=%lld K=%lld", (long long)N,
            (long long)K);
  GLQ_CHECK(K % (32 / bits) == 0,
            "K=%lld must be a multiple of %d for %d-bit codes", (long long)K,
            32 / bits, bits);
  return GLQ_OK;
}

extern "C" {

int glq_version(void) { return 100; }

const char* glq_last_error(void) { return g_err; }

int glq_unpack_codes(const int32_t* codes, int64_t N, int64_t K, int bits,
                     int sym, int32_t* out, void* stream) {
  clear_error();
  int rc = check_codec_shape(N, K, bits);
  if (rc) return rc;
  GLQ_CHECK(sym >= 0 && sym <= 2, "sym must be 0, 1 or 2 (got %d)", sym);
  const int64_t words = N * K / (32 / bits);
  if (words == 0) return GLQ_OK;
  GLQ_CHECK(codes && out, "null pointer");
  const int bs = 256;
  const dim3 grid((unsigned)((words + bs - 1) / bs));
  hipStream_t s = (hipStream_t)stream;
  if (bits == 2)
    unpack_kernel<2><<<grid, bs, 0, s>>>((const uint32_t*)codes, words, sym, out);
  else
    unpack_kernel<4><<<grid, bs, 0, s>>>((const uint32_t*)codes, words, sym, out);
  GLQ_LAUNCH_CHECK("unpack_kernel");
  return GLQ_OK;
}

int glq_dequant_weight(const int32_t* codes, int64_t N, int64_t K, int bits,
                       const void* scales, const void* zeros, int64_t group,
                       int sym, void* W, void* stream) {
  clear_error();
  int rc = check_codec_shape(N, K, bits);
  if (rc) return rc;
  GLQ_CHECK(group > 0 && K % group == 0,
            "K=%lld must be a multiple of group=%lld", (long long)K,
            (long long)group);
  GLQ_CHECK(sym >= 0 && sym <= 2, "sym must be 0, 1 or 2 (got %d)", sym);
  const int64_t words = N * K / (32 / bits);
  if (words == 0) return GLQ_OK;
  GLQ_CHECK(codes && scales && W && (sym == 1 || zeros), "null pointer");
  const int bs = 256;
  const dim3 grid((unsigned)((words + bs - 1) / bs));
  hipStream_t s = (hipStream_t)stream;
  if (bits == 2)
    dequant_kernel<2><<<grid, bs, 0, s>>>((const uint32_t*)codes, N, K,
                                          (const __half*)scales,
                                          (const __half*)zeros, group, sym,
                                          (__half*)W);
  else
    dequant_kernel<4><<<grid, bs, 0, s>>>((const uint32_t*)codes, N, K,
                                          (const __half*)scales,
                                          (const __half*)zeros, group, sym,
                                          (__half*)W);
  GLQ_LAUNCH_CHECK("dequant_kernel");
  return GLQ_OK;
}

int glq_pack_codes(const int32_t* q, int64_t N, int64_t K, int bits,
                   int32_t* codes, void* stream) {
  clear_error();
  int rc = check_codec_shape(N, K, bits);
  if (rc) return rc;
  const int64_t words = N * K / (32 / bits);
  if (words == 0) return GLQ_OK;
  GLQ_CHECK(q && codes, "null pointer");
  const int bs = 256;
  const dim3 grid((unsigned)((words + bs - 1) / bs));
  hipStream_t s = (hipStream_t)stream;
  if (bits == 2)
    pack_kernel<2><<<grid, bs, 0, s>>>(q, words, (uint32_t*)codes);
  else
    pack_kernel<4><<<grid, bs, 0, s>>>(q, words, (uint32_t*)codes);
  GLQ_LAUNCH_CHECK("pack_kernel");
  return GLQ_OK;
}

int glq_dequant_factor(const void* q, int int4_packed, int64_t rows, int64_t cols,
                       const void* scale, int scale_per_row, int nbits, void* out,
                       void* stream) {
  clear_error();
  GLQ_CHECK(rows >= 0 && cols >= 0, "negative shape");
  GLQ_CHECK(nbits >= 2 && nbits <= 8, "nbits must be 2..8 (got %d)", nbits);
  GLQ_CHECK(!int4_packed || nbits == 4, "int4-packed factors have nbits = 4");
  if (rows == 0 || cols == 0) return GLQ_OK;
  GLQ_CHECK(q && scale && out, "null pointer");
  GLQ_CHECK(rows * cols < (1ll << 40), "factor too large");
  const int bs = 256;
  const int64_t n = rows * cols;
  const dim3 grid((unsigned)((n + bs - 1) / bs));
  const float maxval = (float)((1 << (nbits - 1)) - 1);
  dequant_factor_kernel<<<grid, bs, 0, (hipStream_t)stream>>>(
      int4_packed ? nullptr : (const int8_t*)q, int4_packed ? (const uint8_t*)q : nullptr, rows,
      cols, (const __half*)scale, scale_per_row ? 1 : 0, maxval, (__half*)out);
  GLQ_LAUNCH_CHECK("dequant_factor_kernel");
  return GLQ_OK;
}

}  // extern "C"
