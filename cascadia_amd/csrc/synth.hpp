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
// XOR of every 32-bit word of buf[0 .. bytes) folded into sink[1024] (see
// stream_read_kernel): the benchmark's streaming-read ceiling.
hipError_t stream_read(const void *buf, size_t bytes, uint32_t *sink, hipStream_t st);

}  // namespace cai4
