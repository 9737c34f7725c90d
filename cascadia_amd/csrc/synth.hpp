// synth.hpp -- synthetic data generators and the debug dequantiser.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

hipError_t fill_synthetic(int kind, uint64_t seed, uint64_t stream_id, size_t n, double p0,
                          double p1, int dtype, void *out, hipStream_t st);
hipError_t debug_dequant(const uint8_t *packed, const uint8_t *scale_bits, int N, int K, int G,
                         int sdt, float *w, hipStream_t st);

}  // namespace cai4
