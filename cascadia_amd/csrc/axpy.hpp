// axpy.hpp -- the AXPY form of the sparse down projection (ffn_axpy.rs).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

// down [H, I] (crate layout, groups of G along I, scales bf16 or f16) ->
// transposed [I, H] with groups of 32 along H and bf16 scales
// (ffn_axpy.rs:342-440, bit-identical).
hipError_t transpose_requantize(const uint8_t *src, const uint8_t *src_scale_bits, int H, int I,
                                int G, int sdt, uint8_t *dst, uint8_t *dst_scale_bits,
                                hipStream_t st);

struct AxpyPlan {
  int slices, per_slice;
  size_t partial_bytes;
};
AxpyPlan axpy_plan(int H, int n_active);

// y[H] += sum over a < n_active of scalars[active[a]] * W_t[active[a], :]
// (ffn_axpy.rs:82-160); ids >= I are skipped; partial:
// axpy_plan(H, n_active).partial_bytes.
hipError_t axpy_active(const uint8_t *pt, const uint8_t *st_bits, const float *scalars,
                       const uint32_t *active, int n_active, int H, int I, float *partial,
                       float *y, hipStream_t st);

}  // namespace cai4
