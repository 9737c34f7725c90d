// layout.hip -- the MFMA-tiled device layout of an INT4 matrix.
//
// The crate's row-major layout (format.rs:3-17) makes one wave instruction of
// the decode GEMM touch 16 rows x 64 bytes, 2 KB apart, and a row's next 64
// bytes arrive much later -- poor DRAM page locality.  The tiled layout stores
// each (16-row tile T, 128-column k-block kb) as one contiguous 1 KB block in
// MFMA lane order, so every wave streams sequentially:
//
//   packed_tiled[(T*KB + kb)*1024 + 16*l .. +16]
//       = swz(packed[16*T + (l & 15)][kb*64 + 16*(l >> 4) .. +16])  (l = lane 0..63)
//   scale_tiled[(T*NG + g)*16 + r] = scale[16*T + r][g]             (u16)
//
// with KB = ceil(K/128), NG = K/G, rows past N and bytes past K/2 zero.
// swz re-orders the 8 nibbles of each dword: the crate's byte b holds columns
// 2b (low) and 2b+1 (high); the tiled byte b holds columns b (low) and b+4
// (high), so that the MFMA decode (two masks, one shift, four byte permutes)
// yields the dword's 8 columns in natural order and the activations need no
// re-ordering.  The nibble codes and scale bits are moved, never changed, so
// every kernel computes bit-identical results from either layout.
//
// Groups of fewer than 128 columns (G not a multiple of 128): every 32-column
// MFMA step must cover whole groups, so its lanes' dwords must be the block's
// columns 32 s .. 32 s + 31.  Those blocks are stored with the dwords
// transposed across the four 16-lane rows -- dword s of lane row c is dword c
// of lane row s above:
//
//   packed_tiled[(T*KB + kb)*1024 + 16*l + 4*s .. +4]
//       = swz(packed[16*T + (l & 15)][kb*64 + 16*s + 4*(l >> 4) .. +4])
//
// -- so the kernels load a step's fragment as stored (the transpose, four
// lane permutes per fragment, was otherwise paid in every k-loop).
#include "int4_common.hpp"
#include "layout.hpp"

namespace cai4 {

void tiled_sizes(int N, int K, int G, size_t *packed_bytes, size_t *scale_bytes) {
  const size_t tiles = (size_t)(N + 15) / 16, kb = (size_t)(K + 127) / 128;
  *packed_bytes = tiles * kb * 1024;
  *scale_bytes = tiles * (size_t)(K / G) * 16 * 2;
}

CAI4_DEV uint32_t swizzle_dword(uint32_t d) {
  uint32_t r = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) r |= ((d >> (4 * e)) & 0xFu) << (8 * e);
#pragma unroll
  for (int e = 4; e < 8; ++e) r |= ((d >> (4 * e)) & 0xFu) << (8 * (e - 4) + 4);
  return r;
}

__global__ void tile_packed_kernel(const uint8_t *__restrict__ packed, int N, int K, int xposed,
                                   uint8_t *__restrict__ out) {
  const size_t kbt = (size_t)(K + 127) / 128;
  const size_t total = (size_t)((N + 15) / 16) * kbt * 64;  // 16-byte chunks
  const size_t row_bytes = (size_t)K / 2;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t l = i & 63, blk = i >> 6;
    const size_t T = blk / kbt, kb = blk % kbt;
    const size_t r = 16 * T + (l & 15);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (r < (size_t)N) {
      const uint8_t *row = packed + r * row_bytes;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        // untransposed: dword s of the lane's own 16 bytes; transposed: dword
        // (lane row) of lane row s's 16 bytes.  row_bytes is a multiple of 16:
        // a 16-byte part is wholly inside the row or past it.
        const size_t part = kb * 64 + 16 * (xposed ? (size_t)s : (l >> 4));
        const size_t dw = xposed ? (l >> 4) : (size_t)s;
        if (part < row_bytes)
          w[s] = swizzle_dword(*reinterpret_cast<const uint32_t *>(row + part + 4 * dw));
      }
    }
    reinterpret_cast<u32x4_t *>(out)[i] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

__global__ void tile_scales_kernel(const uint16_t *__restrict__ scales, int N, int NG,
                                   uint16_t *__restrict__ out) {
  const size_t total = (size_t)((N + 15) / 16) * NG * 16;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t rr = i & 15, tg = i >> 4;
    const size_t T = tg / NG, g = tg % NG;
    const size_t r = 16 * T + rr;
    out[i] = r < (size_t)N ? scales[r * NG + g] : (uint16_t)0;
  }
}

hipError_t tile_weights(const uint8_t *packed, const uint8_t *scale_bits, int N, int K, int G,
                        uint8_t *packed_tiled, uint8_t *scale_tiled, hipStream_t st) {
  const size_t chunks = (size_t)((N + 15) / 16) * ((K + 127) / 128) * 64;
  size_t grid = (chunks + 255) / 256;
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(tile_packed_kernel, dim3(grid), dim3(256), 0, st, packed, N, K,
                     tiled_xposed(G) ? 1 : 0, packed_tiled);
  if (hipError_t e = hipGetLastError()) return e;
  const size_t ns = (size_t)((N + 15) / 16) * (K / G) * 16;
  grid = (ns + 255) / 256;
  if (grid > 16384) grid = 16384;
  hipLaunchKernelGGL(tile_scales_kernel, dim3(grid), dim3(256), 0, st,
                     reinterpret_cast<const uint16_t *>(scale_bits), N, K / G,
                     reinterpret_cast<uint16_t *>(scale_tiled));
  return hipGetLastError();
}

}  // namespace cai4
