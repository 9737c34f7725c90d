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

// M = 1, MFMA-tiled weights, G a multiple of 128 dividing K, not grouped; activation
// modes A_BF16 / A_XF32 / A_HILO; epilogues f32, bf16, SwiGLU (f32 or hi/lo); the
// plan's LDS within one CU's.
bool gemv_supported(const SkinnyArgs &a, int amode, int epi, int num_cus);
GemvPlan gemv_plan(int N, int K, int num_cus);
hipError_t gemv_launch(const SkinnyArgs &a, int amode, int epi, int num_cus, hipStream_t st);

}  // namespace cai4
