// ov.hpp -- the OpenVINO CascadiaInt4Gemv weight format
// (cascadia-ov-genai-shim/cpp/gemv_offload.cpp): conversions at the boundary.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

// Two's-complement nibbles ((x ^ 8) - 8) -> the crate's offset nibbles
// (x' - 8 with x' = x ^ 8): every byte XOR 0x88; dst may equal src.
hipError_t ov_to_crate(const uint8_t *src, size_t n_bytes, uint8_t *dst, hipStream_t st);

// f16 bits -> f32 (exact), and f32 -> f16 bits (round to nearest even), n elements.
hipError_t f16_to_f32(const uint16_t *src, size_t n, float *dst, hipStream_t st);
hipError_t f32_to_f16(const float *src, size_t n, uint16_t *dst, hipStream_t st);

}  // namespace cai4
