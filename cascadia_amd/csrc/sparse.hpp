// sparse.hpp -- launchers of the activation-sparse expert FFN pieces
// (ffn_sparsity.rs:131-179, 187-348, 499-537).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cai4 {

// Per token t (grid T): sg[t] = SiLU(gate[t]) (the stable form when sparse),
// act[t][0..cnt[t]) = the active lanes ascending, inter[t][i] = 0 for every
// inactive lane; counts_out (nullable) receives cnt.  thr == nullptr: the
// global tau; else one threshold per lane.  I lanes per token.
hipError_t sparse_mask(const float *gate, int T, int I, float tau, const float *thr, float *sg,
                       uint32_t *act, uint32_t *cnt, uint32_t *counts_out, float *inter,
                       hipStream_t st);

// inter[t][r] = sg[t][r] * (W_up[r, :] . x[t]) for r in act[t][0..cnt[t]);
// weights [I, K] in the crate (tiled = 0) or MFMA-tiled layout.
hipError_t rows_subset_up(const uint8_t *w, const uint8_t *s, int I, int K, int G, int sdt,
                          int tiled, const void *x, bool x_f32, int T, const uint32_t *act,
                          const uint32_t *cnt, const float *sg, float *inter, hipStream_t st);

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st);

}  // namespace cai4
