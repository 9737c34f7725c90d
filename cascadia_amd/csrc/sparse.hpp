// sparse.hpp -- launchers of the activation-sparse expert FFN pieces
// (ffn_sparsity.rs:131-179, 187-348, 499-537).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cai4 {

// Between the gate and down GEMMs, per token t: sg = stable SiLU(gate), the
// token's max |sg| and per-channel flag in cells[2t], [2t + 1] (cleared
// here), then inter[t][r] = silu_r * (W_up[r, :] . x[t]) for every active
// lane r and 0 for the rest; weights [I, K] in the crate (tiled = 0) or
// MFMA-tiled layout.  thr == nullptr: the global tau; else one threshold per
// lane.  counts_out (nullable) receives each token's active-lane count.
// plain_silu: the AXPY form's g / (1 + e^-g) instead of the stable SiLU.
hipError_t sparse_ffn_mid(const uint8_t *w, const uint8_t *s, int I, int K, int G, int sdt,
                          int tiled, const void *x, bool x_f32, int T, const float *gate,
                          float tau, const float *thr, float *sg, uint32_t *cells, float *inter,
                          uint32_t *counts_out, hipStream_t st, bool plain_silu = false);

// After sparse_ffn_mid: each token's active lanes in ascending order into
// active[t * I ..] and their count into counts[t].
hipError_t sparse_compact(const float *gate, int I, int T, float tau, const float *thr,
                          const float *sg, const uint32_t *cells, uint32_t *active,
                          uint32_t *counts, hipStream_t st);

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st);

}  // namespace cai4
