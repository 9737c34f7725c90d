// quant.hpp -- load-time INT4 quantiser (bf16 weights -> crate layout).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cai4 {

// w_bf16 [N, K] (16-byte aligned), G a multiple of 32 dividing K; packed
// [N, K/2] nibbles, scale_bits [N, K/G] bf16.
hipError_t quantize_group(const uint16_t *w_bf16, int N, int K, int G, uint8_t *packed,
                          uint16_t *scale_bits, hipStream_t st);

}  // namespace cai4
