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

}  // namespace cai4
