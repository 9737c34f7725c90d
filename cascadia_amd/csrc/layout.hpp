// layout.hpp -- the MFMA-tiled device layout of an INT4 matrix.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

// Tiled blocks of a matrix with groups of G columns hold their dwords
// transposed across the four 16-lane rows (layout.hip) when G is not a
// multiple of 128: each 32-column MFMA step then reads whole groups as stored.
__host__ __device__ inline bool tiled_xposed(int G) { return G % 128 != 0; }

void tiled_sizes(int N, int K, int G, size_t *packed_bytes, size_t *scale_bytes);
hipError_t tile_weights(const uint8_t *packed, const uint8_t *scale_bits, int N, int K, int G,
                        uint8_t *packed_tiled, uint8_t *scale_tiled, hipStream_t st);

}  // namespace cai4
