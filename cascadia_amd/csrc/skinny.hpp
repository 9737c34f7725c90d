// skinny.hpp -- host-visible interface of the decode-regime INT4 GEMM.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

enum Epilogue { EPI_F32 = 0, EPI_SWIGLU = 1, EPI_BF16 = 2 };

struct SkinnyArgs {
  const uint8_t *w0;  // packed [N, K/2]           (gate for EPI_SWIGLU)
  const uint8_t *w1;  // packed [N, K/2] up matrix (EPI_SWIGLU only)
  const uint8_t *s0;  // scales u16 [N, K/G]
  const uint8_t *s1;
  const void *x;      // activations [M, ldx]: bf16 bits or f32
  void *out;          // [M, ldo]: f32 (EPI_F32, EPI_SWIGLU) or bf16 bits (EPI_BF16)
  int N, K, G, M, ldx, ldo, sdt;
};

struct SkinnyPlan {
  int nt, mt, waves, row_blocks, m_chunks;
  size_t lds_bytes;
};

SkinnyPlan skinny_plan(int N, int K, int M, bool xf32, int epi, int num_cus);
hipError_t skinny_launch(const SkinnyArgs &a, const SkinnyPlan &p, bool xf32, int epi,
                         hipStream_t st);

}  // namespace cai4
