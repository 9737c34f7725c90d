// sparse.hpp -- launchers of the activation-sparse expert FFN pieces
// (ffn_sparsity.rs:131-179, 499-537, 638-740; ffn_axpy.rs:82-160).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cai4 {

// Intermediate lanes per mask workgroup (a "group": one lane per thread).
constexpr int kSparseGroup = 256;
// Output columns per AXPY workgroup.
constexpr int kSparseAxCols = 512;

inline int sparse_groups(int I) { return (I + kSparseGroup - 1) / kSparseGroup; }
// Max-|silu| slots per token: one per 16-row tile when the one-token GEMV's
// epilogue writes them (gemv), else one per 256 lanes (sparse_slots).
inline int sparse_slots_per_token(int I, bool gemv) { return gemv ? (I + 15) / 16 : (I + 255) / 256; }

// The slots of a gate [T, I] computed by another GEMM: slots[t][b] = max
// |silu| over lanes [256 b, 256 b + 256) (bits; NaN counts as 0) | (any
// thr > 0 there) << 31.  stable: build_active_mask_mode's SiLU, else the plain one.
hipError_t sparse_slots(const float *gate, int I, int T, const float *thr, bool stable,
                        uint32_t *slots, hipStream_t st);

struct SparseMaskArgs {
  const float *gate, *up;  // [T, I] f32 each
  const uint32_t *slots;   // [T, n_slots]
  const float *thr;        // [I] per-channel thresholds, or null: tau
  float tau;
  int n_slots, I, H;
  uint32_t *cnt;           // [T, n_groups] active lanes per group
  // GEMV form: the intermediate [T, I], silu * up on active lanes, else 0
  float *inter;
  // AXPY form: the transposed down (dt [I, H / 2] bytes, dt_s bf16
  // [I, H / 32]) and the groups' partial output rows [tokens of the launch,
  // n_groups, H]; the launch covers tokens t0 ..
  const uint8_t *dt;
  const uint16_t *dt_s;
  float *partial;
  int t0;
};

// The GEMV form's mask and intermediate for T tokens (stable: the mask's
// SiLU is build_active_mask_mode's, else the plain one).
hipError_t sparse_mask(const SparseMaskArgs &a, int T, bool stable, hipStream_t st);

// The AXPY form for tokens t0 .. t0 + n_tokens - 1: the mask (plain SiLU),
// the transposed down's active rows into the groups' partial rows, then out
// rows t0 .. (overwritten) = their sum in group order and (counts not null)
// each token's active-lane count.
hipError_t sparse_axpy_ffn(const SparseMaskArgs &a, int n_tokens, float *out, uint32_t *counts,
                           hipStream_t st);

// counts[t] = the token's active-lane count (from the groups' counts).
hipError_t sparse_counts(const uint32_t *cnt, int n_groups, int T, uint32_t *counts,
                         hipStream_t st);

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st);

// ---- rows-subset GEMV (ffn_sparsity.rs:187-348) ----

// A matrix read one row at a time: packed / scale bits in the crate layout
// (tiled = 0) or the MFMA-tiled layout (tiled = 1, layout.hip).
struct RowsMatrix {
  const uint8_t *packed;
  const uint8_t *scales;  // u16 bits, bf16 (sdt 0) or fp16 (sdt 1)
  int N, K, G, sdt, tiled;
};

// y[r] = sum_c q[r, c] * scale[r, c / G] * x[c] for r in rows[0 .. n): x f32
// [K] (bf16 bits when x_bf16); rows >= N are skipped, every other y left
// untouched (a duplicate row writes the same value twice).  f32 arithmetic,
// x staged in LDS (K * 4 + K / 8 bytes) when that fits max_lds, else read
// from global memory.
hipError_t rows_subset(const RowsMatrix &w, const void *x, bool x_bf16, const uint32_t *rows,
                       int n, float *y, size_t max_lds, int num_cus, hipStream_t st);

// Intermediate lanes per workgroup of the fused rows-subset sparse kernels:
// 128, or 64 when 128-lane groups would leave CUs idle, down to 8 (GEMV form)
// or 16 (AXPY form) for small intermediates (subset_lanes).
constexpr int kSubsetGroup = 128;
int subset_lanes(int I, int num_cus, bool axpy);
inline bool subset_lanes_ok(int lanes) {
  return lanes == 8 || lanes == 16 || lanes == 32 || lanes == 64 || lanes == kSubsetGroup;
}
inline int subset_groups(int I, int lanes) { return (I + lanes - 1) / lanes; }
// The fused kernels stage one token's x (H f32 + H / 32 chunk sums) in LDS and
// hold the transposed down's H columns of a lane in registers: H a multiple of
// 32 up to 8192.
inline bool subset_supported(int H) { return H >= 32 && H % 32 == 0 && H <= 8192; }

// The activation-sparse FFN after its gate GEMV (gate rows + the max-|silu|
// slots), with the up projection computed only for the active lanes:
// workgroup (group of kSubsetGroup lanes, token) builds the mask, lists the
// active lanes in ascending order, and reads only their up rows.
struct SparseSubsetArgs {
  const float *gate;  // [T, I] f32
  const uint32_t *slots;
  int n_slots;
  const float *thr;  // [I] or null: tau
  float tau;
  RowsMatrix up;     // [I, H]
  const void *x;     // [T, H] f32, or bf16 bits when x_bf16
  int x_bf16;
  int I, H;
  int lanes;         // lanes per workgroup (group): subset_lanes(I, CUs, form)
  uint32_t *cnt;     // [T, subset_groups(I, lanes)] active lanes per group
  // GEMV form: inter [T, I] = silu * up on active lanes, else 0 (stable
  // SiLU, build_active_mask_mode's)
  float *inter;
  // AXPY form (plain SiLU): the transposed down (dt [I, H / 2] bytes, dt_s
  // bf16 [I, H / 32]) and the groups' partial output rows [launch tokens,
  // groups, H]; the launch covers tokens t0 ..
  const uint8_t *dt;
  const uint16_t *dt_s;
  float *partial;
  int t0;
};
hipError_t sparse_subset_mask(const SparseSubsetArgs &a, int T, hipStream_t st);
// The AXPY form for tokens t0 .. t0 + n_tokens - 1: out rows (overwritten) =
// the groups' partial rows added in group order; counts (may be null) each
// token's active-lane count.
// build_active_mask_mode (ffn_sparsity.rs:131-179) on one row of n gate
// values: silu_out = the stable SiLU of every lane; active_out[0 .. *n_active)
// = the lanes with |silu| >= cutoff * max|silu| in ascending order (cutoff =
// tau, or thresholds[i] when thresholds is not null), every lane when the max
// is 0 or the mode is dense (tau <= 0; no per-channel threshold > 0).  One
// workgroup.
hipError_t build_active_mask(const float *gate, int n, float tau, const float *thr, float *silu,
                             uint32_t *active, uint32_t *n_active, hipStream_t st);

// f32 <-> bf16 bits (format.rs:130-160): to bf16 by RNE with a quiet NaN,
// back exactly.
hipError_t f32_to_bf16_n(const float *x, uint16_t *out, size_t n, hipStream_t st);
hipError_t bf16_to_f32_n(const uint16_t *x, float *out, size_t n, hipStream_t st);

hipError_t sparse_subset_axpy(const SparseSubsetArgs &a, int n_tokens, float *out,
                              uint32_t *counts, hipStream_t st);

}  // namespace cai4
