// prefill.hpp -- INT4 weight-only GEMM for many tokens (M >= 64).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

// The prefill kernel handles MFMA-tiled weights with K and G multiples of 128.
bool prefill_supported(int M, int N, int K, int G, int tiled);

// Device workspace prefill_gemm needs (256-byte aligned): per-row seeds, and
// f32 partial sums when K is split across workgroups.
size_t prefill_workspace_bytes(int M, int N, int K, int num_cus);

// y[M, N] = x[M, K] (bf16) * W^T, f32 accumulation; bf16 (RNE) or f32 output.
hipError_t prefill_gemm(const uint8_t *w, const uint8_t *s, const uint16_t *x, void *y, int M,
                        int N, int K, int G, int sdt, int out_f32, void *ws, int num_cus,
                        hipStream_t st);

}  // namespace cai4
