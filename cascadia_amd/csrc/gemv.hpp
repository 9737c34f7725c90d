// gemv.hpp -- one-token INT4 GEMV over MFMA-tiled weights (decode shape).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "skinny.hpp"

namespace cai4 {

// kw waves per workgroup (one 16-row tile or gate/up tile pair), kpw k-blocks each.
struct GemvPlan {
  int kw, kpw;
};

// MFMA-tiled weights, G a multiple of 128 dividing K; epilogues f32, bf16, SwiGLU
// (f32 or hi/lo); the plan's LDS within one CU's.  Dense: M = 1, activation
// modes A_BF16 / A_XF32 / A_HILO.  Grouped (a.chunks): chunks of one row
// (chunk_rows = 1), max_chunks of them, modes A_GATHER / A_HILO.
bool gemv_supported(const SkinnyArgs &a, int amode, int epi, int num_cus, int chunk_rows = 0,
                    int max_chunks = 0);
GemvPlan gemv_plan(int N, int K, int num_cus);
hipError_t gemv_launch(const SkinnyArgs &a, int amode, int epi, int num_cus, int max_chunks,
                       hipStream_t st);

}  // namespace cai4
