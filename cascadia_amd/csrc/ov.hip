// ov.hip -- the OpenVINO CascadiaInt4Gemv format at the boundary
// (cascadia-ov-genai-shim/cpp/gemv_offload.cpp:150-340, 623-638).
//
// That op's weights are packed two per byte, element 0 in the low nibble,
// each nibble a two's-complement int4: q = (x ^ 8) - 8.  The crate's nibble is
// offset binary, q = x' - 8, so x' = x ^ 8: one XOR of 0x88 per byte turns an
// OV matrix into the crate layout (same products, bit for bit), done once when
// the weights are uploaded; every kernel of this library then runs it.  Its
// scales are f16 [n, k / group], the crate layout of f16 scales.  The op takes
// and returns f16 or f32 activations: the f16 side is converted here.
#include "int4_common.hpp"
#include "ov.hpp"

namespace cai4 {

namespace {

__global__ __launch_bounds__(256) void ov_xor_kernel(const uint32_t *src, size_t n_words,
                                                     uint32_t *dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_words) dst[i] = src[i] ^ 0x88888888u;
}

__global__ __launch_bounds__(256) void ov_xor_tail_kernel(const uint8_t *src, size_t from,
                                                          size_t n, uint8_t *dst) {
  const size_t i = from + threadIdx.x;
  if (i < n) dst[i] = src[i] ^ 0x88u;
}

__global__ __launch_bounds__(256) void f16_to_f32_kernel(const uint16_t *src, size_t n,
                                                         float *dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = (float)__builtin_bit_cast(_Float16, src[i]);
}

__global__ __launch_bounds__(256) void f32_to_f16_kernel(const float *src, size_t n,
                                                         uint16_t *dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = __builtin_bit_cast(uint16_t, (_Float16)src[i]);
}

}  // namespace

hipError_t ov_to_crate(const uint8_t *src, size_t n_bytes, uint8_t *dst, hipStream_t st) {
  const size_t words = n_bytes / 4;
  if (words)
    hipLaunchKernelGGL(ov_xor_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                       reinterpret_cast<const uint32_t *>(src), words,
                       reinterpret_cast<uint32_t *>(dst));
  if (n_bytes % 4)
    hipLaunchKernelGGL(ov_xor_tail_kernel, dim3(1), dim3(256), 0, st, src, words * 4, n_bytes,
                       dst);
  return hipGetLastError();
}

hipError_t f16_to_f32(const uint16_t *src, size_t n, float *dst, hipStream_t st) {
  if (n)
    hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src,
                       n, dst);
  return hipGetLastError();
}

hipError_t f32_to_f16(const float *src, size_t n, uint16_t *dst, hipStream_t st) {
  if (n)
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src,
                       n, dst);
  return hipGetLastError();
}

}  // namespace cai4
