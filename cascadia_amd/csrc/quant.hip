// quant.hip -- load-time INT4 quantiser on the GPU: bf16 weights [N, K] ->
// packed nibbles [N, K/2] + bf16 group scales [N, K/G], as the crate's
// quantize_int4_group (crates/cascadia-int4-gemm/src/shell_int4.rs:148-212,
// fixed G = 32 there; any G that is a multiple of 32 dividing K here).
//
// Per group: max|w| (NaNs never win the comparison), scale = max / 7 (1e-10
// for an all-zero group), stored as bf16 by the crate's rounding
// (shell_int4.rs:214-220: bits + 0x7FFF + lsb, no NaN branch); then
// q = clamp(round(w * (1 / scale_bf16)), -8, 7) with round half away from
// zero, and nibble q + 8 (column 2i low, 2i+1 high).  The divisions are
// IEEE-rounded and the product is not fused with anything, so the bytes match
// the crate bit for bit.  A NaN weight becomes q = 0 (Rust's `as i32` of NaN),
// nibble 8.
//
// One thread per group: it reads its group's 16-byte chunks twice (the max,
// then the codes; the second pass hits the cache) and writes four bytes (eight
// nibbles) per chunk.  Load-time work: the bytes move once, well inside a
// millisecond for a config 1 expert.
#include <math.h>

#include "int4_common.hpp"
#include "quant.hpp"

namespace cai4 {

namespace {

__global__ __launch_bounds__(256) void quantize_group_kernel(const uint16_t *w, int N, int K,
                                                             int G, uint8_t *packed,
                                                             uint16_t *scales) {
  const int ng = K / G;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)N * ng) return;
  const long r = gid / ng;
  const int g = (int)(gid - r * ng);
  const uint16_t *src = w + r * K + (long)g * G;
  float mx = 0.0f;
  for (int c = 0; c < G; c += 8) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t *>(src + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a0 = fabsf(bf16_to_f32(v[e] & 0xFFFFu)), a1 = fabsf(bf16_to_f32(v[e] >> 16));
      if (a0 > mx) mx = a0;  // shell_int4.rs:167-170 (a NaN never compares greater)
      if (a1 > mx) mx = a1;
    }
  }
  const float scale = mx == 0.0f ? 1.0e-10f : __fdiv_rn(mx, 7.0f);
  const uint32_t b = fbits(scale);
  const uint32_t sb = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;  // shell_int4.rs:214-220
  scales[r * ng + g] = (uint16_t)sb;
  const float inv = __fdiv_rn(1.0f, bf16_to_f32(sb));
  uint8_t *dst = packed + (r * K + (long)g * G) / 2;
  for (int c = 0; c < G; c += 8) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t *>(src + c);
    uint32_t out = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t bits = (j & 1) ? v[j >> 1] >> 16 : v[j >> 1] & 0xFFFFu;
      const float qf = roundf(__fmul_rn(bf16_to_f32(bits), inv));  // half away from zero
      const int q = qf != qf ? 0 : (int)fminf(fmaxf(qf, -8.0f), 7.0f);
      out |= (uint32_t)((q + 8) & 0x0F) << (4 * j);  // column c + j: byte j / 2, nibble j & 1
    }
    *reinterpret_cast<uint32_t *>(dst + c / 2) = out;
  }
}

}  // namespace

hipError_t quantize_group(const uint16_t *w_bf16, int N, int K, int G, uint8_t *packed,
                          uint16_t *scale_bits, hipStream_t st) {
  const long groups = (long)N * (K / G);
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_group_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                     st, w_bf16, N, K, G, packed, scale_bits);
  return hipGetLastError();
}

}  // namespace cai4
