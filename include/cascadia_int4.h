/*
 * cascadia_int4.h -- C ABI of libcascadia_int4_hip.so, the MI355X (gfx950)
 * implementation of cascadia-int4-gemm's INT4 weight-only matmul path.
 *
 * Drop-in boundary.  Every entry point below replaces one function of the
 * reference crate (labscommunity/cascadia, crates/cascadia-int4-gemm) and
 * cites it.  Differences a caller must know:
 *   - Weight, activation and output pointers are DEVICE pointers (HBM).  The
 *     weights stay resident; nothing is copied per call.  The byte layout is
 *     the crate's, unchanged (src/format.rs:3-17, src/kernel.rs:3-13).
 *   - The crate hard-codes group 32 / bf16 scales (src/lib.rs:73); here the
 *     layout carries the group size G (a multiple of 32 dividing K) and the
 *     scale dtype (bf16 = the crate's, or fp16).
 *   - Length mismatches panic in the crate (assert_eq!, kernel.rs:39-43);
 *     here they return CASCADIA_INT4_ERR_ARG.  No abort or exception ever
 *     crosses this ABI.
 *   - Calls are enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and return without waiting; outputs are complete once the stream is
 *     synchronised (cascadia_int4_synchronize).  The crate's calls are
 *     synchronous; a caller that needs that calls cascadia_int4_synchronize.
 *   - A call over zero token rows (n_tokens == 0, n_active == 0,
 *     n_bytes == 0) reads and writes nothing and returns CASCADIA_INT4_OK;
 *     the buffers whose length is that count may then be NULL.  The exceptions follow the crate's asserts:
 *     the seq-major GEMMs (seq >= 1, kernel_avx512_multi.rs:80) and
 *     cascadia_int4_moe_forward return CASCADIA_INT4_ERR_ARG for zero rows.
 *   - Outputs are fully overwritten, as in the crate.  Calls are reentrant
 *     for distinct output buffers; a shared workspace (workspace == NULL, the
 *     library's own) makes concurrent calls on different streams race.
 *   - HIP graph capture: the library's own workspace grows by an allocation,
 *     which a capture cannot record; a call on a capturing stream that would
 *     grow it returns CASCADIA_INT4_ERR_ARG.  Callers that capture pass a
 *     workspace of the matching *_workspace_bytes size, or use
 *     cascadia_int4_expert_forward_noalloc, or warm the library's workspace
 *     with an eager call of the same shape first.  A growth never frees the
 *     buffer it replaces (the library keeps it until the process ends), so a
 *     graph captured on the smaller buffer stays valid after a later, larger
 *     eager call; it still shares that buffer with any eager call, so replays
 *     and eager calls that use the library's workspace must not overlap.
 */
#ifndef CASCADIA_INT4_H
#define CASCADIA_INT4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (c_ffi.rs returns 0 / -1 / -2 / -3 for its own calls). */
#define CASCADIA_INT4_OK 0
#define CASCADIA_INT4_ERR_NULL (-1)   /* a required pointer is NULL */
#define CASCADIA_INT4_ERR_ARG (-2)    /* shape / length / alignment invalid */
#define CASCADIA_INT4_ERR_DEVICE (-3) /* HIP runtime error, or I/O error on open */
#define CASCADIA_INT4_ERR_NOMEM (-4)  /* device allocation failed */

#define CASCADIA_INT4_SCALE_BF16 0u /* the crate's format (format.rs:16-17) */
#define CASCADIA_INT4_SCALE_F16 1u

/* Weight byte layouts.  CRATE is the crate's row-major layout, unchanged.
 * MFMA is the tiled device layout made by cascadia_int4_tile_weights: each
 * (16-row tile, 128-column k-block) is one contiguous 1 KB block in MFMA lane
 * order, so the decode kernels stream HBM sequentially; for groups narrower
 * than 128 columns the blocks hold their dwords transposed across the four
 * 16-lane rows, so a tiled copy is read with the group size it was made
 * for.  Same codes and scale bits, moved; results are bit-identical between
 * the two. */
#define CASCADIA_INT4_TILING_CRATE 0u
#define CASCADIA_INT4_TILING_MFMA 1u
/* Experts only (cascadia_int4_expert.tiling), for the activation-sparse
 * entry points, which read up one row at a time for the active lanes only:
 * gate and down MFMA-tiled, up in the crate layout (each row contiguous, so
 * an inactive row costs no bytes).  The other expert entry points refuse it
 * with CASCADIA_INT4_ERR_ARG. */
#define CASCADIA_INT4_TILING_MFMA_UP_ROWS 2u

/* Routing rules for the MoE entry point. */
#define CASCADIA_INT4_ROUTE_IDS 0u          /* caller supplies ids/weights */
#define CASCADIA_INT4_ROUTE_SIGMOID_BIAS 1u /* shell_int4.rs:588-620 / glm/gate.rs:24-62 */
#define CASCADIA_INT4_ROUTE_SOFTMAX_TOPK 2u /* softmax over the top-k logits */

/* One packed INT4 matrix: packed u8 [n_rows, k_cols/2] (byte i of a row =
 * column 2i in the low nibble, 2i+1 in the high nibble, q = nibble - 8) and
 * scale_bits u16 LE [n_rows, k_cols/group_size].  w = f32(q) * f32(scale). */
typedef struct cascadia_int4_layout {
  uint32_t n_rows;      /* N, output rows */
  uint32_t k_cols;      /* K, a multiple of group_size */
  uint32_t group_size;  /* G, a multiple of 32 (the crate: 32) */
  uint32_t scale_dtype; /* CASCADIA_INT4_SCALE_BF16 or _F16 */
  uint32_t tiling;      /* CASCADIA_INT4_TILING_CRATE or _MFMA */
} cascadia_int4_layout;

/* Byte sizes of the MFMA-tiled copy of a matrix (rows padded to 16, columns
 * to 128).  layout->tiling is ignored. */
int cascadia_int4_tiled_sizes(const cascadia_int4_layout *layout, size_t *packed_bytes,
                              size_t *scale_bytes);

/* Write the MFMA-tiled copy of a crate-layout matrix (done once, when the
 * weights are uploaded).  layout->tiling is ignored (the source is CRATE). */
int cascadia_int4_tile_weights(const cascadia_int4_layout *layout, const uint8_t *packed,
                               const uint8_t *scale_bits, uint8_t *packed_tiled,
                               uint8_t *scale_tiled, void *stream);

/* Library version string. */
const char *cascadia_int4_version(void);

/* Wait for all work enqueued on `stream`. */
int cascadia_int4_synchronize(void *stream);

/* The launch-plan overrides CASCADIA_INT4_* (tuning and tests only; every
 * default is measured) are read from the environment once per process, at the
 * first call that needs each; this makes the next calls read them again.  No
 * counterpart in the crate, which has no plan overrides. */
void cascadia_int4_reload_tuning(void);

/* y[r] = sum_c (nibble[r,c]-8) * scale[r, c/G] * x[c] for one f32 vector.
 * Replaces dequant_gemv_int4 (src/kernel.rs:31-71) and
 * dequant_gemv_int4_auto (src/kernel_avx512.rs:274-297).
 * x: f32 [k_cols], y: f32 [n_rows]. */
int cascadia_int4_dequant_gemv(const cascadia_int4_layout *layout, const uint8_t *packed,
                               const uint8_t *scale_bits, const float *x, float *y,
                               void *stream);

/* y[r] for the rows r listed in active_rows[0 .. n_active) only: the same
 * dot products as cascadia_int4_dequant_gemv, every other y left untouched
 * (the caller zeroes it when it needs defined values there; a row listed
 * twice is written twice with the same value).  Replaces
 * dequant_gemv_int4_rows_subset (src/ffn_sparsity.rs:187-243) and
 * dequant_gemv_int4_rows_subset_auto (:317-348).  Rows >= n_rows are skipped
 * (the crate's debug_assert).  Only the listed rows' bytes are read; in the
 * CRATE layout a row is contiguous, in the MFMA layout its bytes are spread
 * over 16-byte pieces of its tile.  x: f32 [k_cols], 16-byte aligned;
 * active_rows: u32 [n_active]; y: f32 [n_rows].  f32 arithmetic. */
int cascadia_int4_dequant_gemv_rows_subset(const cascadia_int4_layout *layout,
                                           const uint8_t *packed, const uint8_t *scale_bits,
                                           const float *x, float *y,
                                           const uint32_t *active_rows, uint32_t n_active,
                                           void *stream);

/* build_active_mask_mode (src/ffn_sparsity.rs:131-179; build_active_mask
 * :106-108 when thresholds is NULL, build_active_mask_per_channel :115-125
 * when it is not) on one row of n gate values: silu_out[i] = the stable SiLU
 * g >= 0 ? g / (1 + e^-g) : g e^g / (1 + e^g); active_out[0 .. *n_active_out)
 * = the lanes with |silu| >= cutoff * max|silu|, ascending (cutoff =
 * threshold, or thresholds[i]), or every lane when max|silu| is 0 or the mode
 * is dense (threshold <= 0 with thresholds NULL; no thresholds[i] > 0).
 * Device pointers: gate_out, silu_out f32 [n]; thresholds f32 [n] or NULL;
 * active_out u32 [n]; n_active_out u32 [1]. */
int cascadia_int4_build_active_mask(const float *gate_out, uint32_t n, float threshold,
                                    const float *thresholds, float *silu_out,
                                    uint32_t *active_out, uint32_t *n_active_out,
                                    void *stream);

/* f32 -> bf16 bits, round to nearest even with NaN kept quiet
 * (f32_to_bf16_bits, src/format.rs:151-160), and bf16 bits -> f32 exactly
 * (bf16_bits_to_f32, :130-135), over n device values. */
int cascadia_int4_f32_to_bf16(const float *x, size_t n, uint16_t *out_bf16, void *stream);
int cascadia_int4_bf16_to_f32(const uint16_t *x_bf16, size_t n, float *out, void *stream);

/* ys[t*n_rows + r] for t < seq, f32 activations xs [seq, k_cols].
 * Replaces dequant_gemm_int4_multi_auto (src/kernel_avx512_multi.rs:207-245)
 * and dequant_gemm_int4_multi_blocked_auto
 * (src/kernel_avx512_multi_blocked.rs:295-347); any seq >= 1. */
int cascadia_int4_dequant_gemm_multi(const cascadia_int4_layout *layout,
                                     const uint8_t *packed, const uint8_t *scale_bits,
                                     const float *xs, uint32_t seq, float *ys, void *stream);

/* As cascadia_int4_dequant_gemm_multi with bf16 activations (exact in the
 * MFMA): xs_bf16 [seq, k_cols] bf16 bits, ys f32 [seq, n_rows].  The crate
 * converts bf16 -> f32 before its GEMV (kernel.rs:89-93); same values. */
int cascadia_int4_dequant_gemm_bf16in(const cascadia_int4_layout *layout,
                                      const uint8_t *packed, const uint8_t *scale_bits,
                                      const uint16_t *xs_bf16, uint32_t seq, float *ys,
                                      void *stream);

/* Prefill GEMM, bf16 activations -> bf16 output (f32 accumulation, one RNE
 * rounding): ys_bf16[t*n_rows + r].  For seq > 64 the crate runs the
 * per-token GEMV loop (kernel_avx512_multi.rs:240-244); same contract. */
int cascadia_int4_gemm_bf16(const cascadia_int4_layout *layout, const uint8_t *packed,
                            const uint8_t *scale_bits, const uint16_t *xs_bf16, uint32_t seq,
                            uint16_t *ys_bf16, void *stream);

/* One expert's six weight slices (device pointers), as expert_forward takes
 * them (src/kernel.rs:75-84): gate/up are [inter, hidden], down is
 * [hidden, inter], each packed u8 + scale u16 in the layout above.  Packed
 * slices must be 16-byte aligned, scale slices 2-byte aligned. */
typedef struct cascadia_int4_expert {
  const uint8_t *gate_packed;
  const uint8_t *gate_scale;
  const uint8_t *up_packed;
  const uint8_t *up_scale;
  const uint8_t *down_packed;
  const uint8_t *down_scale;
  uint32_t tiling; /* CASCADIA_INT4_TILING_CRATE or _MFMA, for all six slices */
} cascadia_int4_expert;

/* Size in bytes of one flat expert blob: gate_p, gate_s, up_p, up_s, down_p,
 * down_s contiguous (format.rs:35-47 / ov_moe.rs:792-806, any dims/G). */
size_t cascadia_int4_expert_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size);

/* Fill *out with the six slices of a crate-layout flat expert blob at `flat`
 * (the slicing of ov_moe.rs:792-806 / format.rs:63-96); tiling = CRATE. */
int cascadia_int4_expert_from_flat(const uint8_t *flat, uint32_t hidden, uint32_t inter,
                                   uint32_t group_size, cascadia_int4_expert *out);

/* Bytes of the MFMA-tiled copy of one expert (six 256-byte-aligned
 * sections in the flat-blob order). */
size_t cascadia_int4_expert_tiled_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size);

/* Tile the six crate-layout slices of *src into the blob at dst (at least
 * cascadia_int4_expert_tiled_bytes, 256-byte aligned) and describe the
 * tiled slices in *out (tiling = MFMA). */
int cascadia_int4_tile_expert(uint32_t hidden, uint32_t inter, uint32_t group_size,
                              const cascadia_int4_expert *src, uint8_t *dst,
                              cascadia_int4_expert *out, void *stream);

/* Workspace bytes the expert / FFN entry points need for n_tokens rows on the
 * current device (the launch plan depends on its CU count); 0 on bad
 * arguments.  No counterpart in the crate, which allocates per call. */
size_t cascadia_int4_ffn_workspace_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t n_tokens);

/* expert_forward for n_tokens independent rows: out = bf16(W_d ·
 * (silu(W_g·x) ⊙ (W_u·x))) with x bf16, everything inside f32, one RNE
 * rounding of the output (src/kernel.rs:75-136; ffn_sparsity.rs:756 at
 * tau = 0).  x_bf16, out_bf16: [n_tokens, hidden] bf16 bits.  workspace:
 * >= cascadia_int4_ffn_workspace_bytes bytes, 16-byte aligned, or NULL to use
 * the library's per-device buffer.  Named _device because the crate's C FFI
 * already exports cascadia_int4_expert_forward for its safetensors-handle
 * call (c_ffi.rs:308-341, f32 in/out); that name stays reserved for it. */
int cascadia_int4_expert_forward_device(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                        uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                        const uint16_t *x_bf16, uint32_t n_tokens,
                                        uint16_t *out_bf16, void *workspace, void *stream);

/* cascadia_int4_expert_forward_device without a workspace argument and
 * without any allocation: no counterpart in the reference crate.  For callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The SwiGLU intermediate
 * and split-K partials live in a file-scope device array of
 * CASCADIA_INT4_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends;
 * a call whose cascadia_int4_ffn_workspace_bytes(hidden, inter, group_size,
 * n_tokens) exceeds it returns CASCADIA_INT4_ERR_ARG (config 1's Llama-3-8B
 * FFN fits up to 64 tokens).  Every call on one GPU shares that array, so
 * calls that overlap on one GPU (different streams, or threads) race;
 * serialise them.  Same kernels and results as the _device entry point. */
#define CASCADIA_INT4_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int cascadia_int4_expert_forward_noalloc(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t scale_dtype,
                                         const cascadia_int4_expert *expert,
                                         const uint16_t *x_bf16, uint32_t n_tokens,
                                         uint16_t *out_bf16, void *stream);

/* First half of the expert FFN: inter[t, i] = silu(W_g·x_t)[i] * (W_u·x_t)[i]
 * in f32 (kernel.rs:96-120; the batched gate/up + swiglu_mul of
 * shell_int4.rs:1112-1130).  x: [n_tokens, hidden], bf16 bits when x_is_f32
 * is 0, else f32.  inter_out: f32 [n_tokens, inter].  Only the gate/up
 * slices of *expert are read. */
int cascadia_int4_gate_up_silu(uint32_t hidden, uint32_t inter, uint32_t group_size,
                               uint32_t scale_dtype, const cascadia_int4_expert *expert,
                               const void *x, uint32_t x_is_f32, uint32_t n_tokens,
                               float *inter_out, void *stream);

/* The AXPY form of the sparse down projection (src/ffn_axpy.rs).
 * transpose_requantize_down (ffn_axpy.rs:342-440, load time): the down matrix
 * [hidden, inter] in the crate layout (groups of group_size along inter,
 * bf16 or fp16 scales; the crate: 32, bf16) -> packed_t [inter, hidden / 2]
 * (16-byte aligned) and bf16 scale_t [inter, hidden / 32], requantised in
 * groups of 32 along hidden exactly as the crate (scale = max|v| / 7, 1.0
 * for a zero group; codes round(v / scale) clamped to [-8, 7]).
 * dequant_axpy_active (ffn_axpy.rs:82-160): y[hidden] += sum over a <
 * n_active of scalars[active[a]] * dequant(packed_t[active[a], :]), only the
 * active rows read; ids >= inter are skipped.  All pointers device;
 * workspace >= cascadia_int4_axpy_workspace_bytes or NULL. */
int cascadia_int4_transpose_requantize_down(uint32_t hidden, uint32_t inter,
                                            uint32_t group_size, uint32_t scale_dtype,
                                            const uint8_t *packed, const uint8_t *scale_bits,
                                            uint8_t *packed_t, uint8_t *scale_t_bits,
                                            void *stream);
size_t cascadia_int4_axpy_workspace_bytes(uint32_t hidden, uint32_t n_active);
int cascadia_int4_dequant_axpy_active(const uint8_t *packed_t, const uint8_t *scale_t_bits,
                                      const float *scalars, const uint32_t *active,
                                      uint32_t n_active, uint32_t inter, uint32_t hidden,
                                      float *y, void *workspace, void *stream);

/* Activation-sparse expert FFN (src/ffn_sparsity.rs:438-538
 * ffn_forward_sparse_f32_mode, :756-867 expert_forward_sparse_mode; the
 * mask :131-179): gate in full, s = stable SiLU(gate), lanes with |s| >=
 * cutoff * max|s| active (cutoff = threshold, or thresholds[i] when
 * thresholds, device f32 [inter], is not NULL: SparsityMode::PerChannel), up
 * for the active rows only (the rows-subset GEMV: for hidden a multiple of 32
 * up to 8192 only those rows' bytes are read; a wider hidden reads up in
 * full), intermediate s * up on them and 0 elsewhere, down in full.
 * threshold <= 0 with thresholds NULL is the dense FFN
 * (cascadia_int4_ffn_forward_f32 / cascadia_int4_expert_forward_device), or,
 * for an expert in CASCADIA_INT4_TILING_MFMA_UP_ROWS, every lane active on
 * the sparse path.
 * Every token row is masked on its own; active_counts (device u32
 * [n_tokens], may be NULL) receives each row's active-lane count (the
 * crate's return value is count / inter).  _f32: x, out f32; _sparse: x, out
 * bf16 bits, out one RNE rounding of the f32 result.  workspace: >=
 * cascadia_int4_ffn_sparse_workspace_bytes, or NULL for the library's. */
size_t cascadia_int4_ffn_sparse_workspace_bytes(uint32_t hidden, uint32_t inter,
                                                uint32_t group_size, uint32_t n_tokens);
int cascadia_int4_ffn_forward_sparse_f32(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t scale_dtype,
                                         const cascadia_int4_expert *expert, const float *x,
                                         uint32_t n_tokens, float threshold,
                                         const float *thresholds, float *out,
                                         uint32_t *active_counts, void *workspace,
                                         void *stream);
int cascadia_int4_expert_forward_sparse(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                        uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                        const uint16_t *x_bf16, uint32_t n_tokens,
                                        float threshold, const float *thresholds,
                                        uint16_t *out_bf16, uint32_t *active_counts,
                                        void *workspace, void *stream);

/* The AXPY form of the activation-sparse FFN, f32 in / f32 out: replaces
 * ffn_forward_sparse_axpy_f32 / _per_channel / _mode
 * (src/ffn_sparsity.rs:569-740; called per routed expert by
 * crates/cascadia-engine-sparse-moe/src/runner.rs:1043, :1162).  gate in
 * full, s = g / (1 + e^-g), lanes with |s| >= cutoff * max|s| active (every
 * lane when max|s| is 0, threshold <= 0 with thresholds NULL, or every
 * per-channel threshold <= 0), up for the active rows only, inter = s * up
 * on them, then out = sum over the active lanes r (ascending) of inter[r] *
 * dequant(down_t[r, :]) -- the down matrix in the transposed layout of
 * cascadia_int4_transpose_requantize_down, given in expert->down_packed /
 * down_scale (as the crate passes down_packed_t / down_scale_t_bits in the
 * down slots); gate/up in expert->tiling (CRATE, MFMA, or MFMA_UP_ROWS:
 * gate tiled, up in the crate layout).  For hidden a multiple of 32 up to
 * 8192 the up rows and the transposed-down rows are read for the active lanes
 * only (one fused kernel per 128 lanes after the gate GEMV); a wider hidden
 * reads up in full.  The sum over the active lanes is added per 128-lane
 * group and the groups in order (deterministic; the crate adds them in one
 * ascending pass).  x, out: f32 [n_tokens, hidden]
 * (out fully overwritten); active_counts (device u32 [n_tokens], may be NULL)
 * receives each row's active-lane count (the crate returns count / inter).
 * workspace: >= cascadia_int4_ffn_sparse_axpy_workspace_bytes or NULL. */
size_t cascadia_int4_ffn_sparse_axpy_workspace_bytes(uint32_t hidden, uint32_t inter,
                                                     uint32_t group_size, uint32_t n_tokens);
int cascadia_int4_ffn_forward_sparse_axpy_f32(uint32_t hidden, uint32_t inter,
                                              uint32_t group_size, uint32_t scale_dtype,
                                              const cascadia_int4_expert *expert, const float *x,
                                              uint32_t n_tokens, float threshold,
                                              const float *thresholds, float *out,
                                              uint32_t *active_counts, void *workspace,
                                              void *stream);

/* Dense SwiGLU FFN, f32 in / f32 out, no rounding: ffn_forward_sparse_f32 at
 * tau = 0 (src/ffn_sparsity.rs:373-496), used for the shared expert
 * (shell_int4.rs:629).  x, out: [n_tokens, hidden] f32. */
int cascadia_int4_ffn_forward_f32(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                  uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                  const float *x, uint32_t n_tokens, float *out,
                                  void *workspace, void *stream);

/* ---- sparse-MoE layer (one pipeline stage on one GPU) ---- */

/* The routed experts of one layer, resident in HBM: expert e's blob starts at
 * experts + e * expert_stride and holds the six sections of an expert in the
 * crate's flat order (format.rs:35-47, tiling = CRATE) or of
 * cascadia_int4_tile_expert (tiling = MFMA).  experts and expert_stride must
 * be multiples of 256.  A shared expert (shell_int4.rs:629) is given by six
 * non-NULL pointers in `shared` (same tiling) and its intermediate size. */
typedef struct cascadia_int4_moe_layer {
  uint32_t hidden, inter, group_size, scale_dtype, tiling;
  uint32_t n_experts; /* <= 1024 */
  const uint8_t *experts;
  size_t expert_stride;
  cascadia_int4_expert shared; /* all pointers NULL: no shared expert */
  uint32_t shared_inter;
} cascadia_int4_moe_layer;

/* Routing of n_tokens tokens to top_k (<= 16) experts.
 *   ROUTE_SIGMOID_BIAS: s = sigmoid(logit); the top_k by s + bias (bias may be
 *     NULL), ties to the lower id; w = s / (sum s + 1e-20) * scale when
 *     normalize (K2.6 / GLM, shell_int4.rs:588-620, glm/gate.rs:24-62), else
 *     w = s * scale.
 *   ROUTE_SOFTMAX_TOPK: the top_k logits (ties to the lower id), w = softmax
 *     over them.
 *   ROUTE_IDS: ids / weights given, [n_tokens, top_k] int32 / f32.
 * Slots with w < threshold are skipped (runner.rs:1811). */
typedef struct cascadia_int4_routing {
  uint32_t mode, top_k;
  const float *logits; /* [n_tokens, n_experts] */
  const float *bias;   /* [n_experts] or NULL */
  float scale;
  uint32_t normalize;
  const int32_t *ids;
  const float *weights;
  float threshold;
} cascadia_int4_routing;

/* Workspace bytes of cascadia_int4_moe_forward on the current device. */
size_t cascadia_int4_moe_workspace_bytes(const cascadia_int4_moe_layer *layer, uint32_t top_k,
                                         uint32_t n_tokens);

/* One MoE layer for n_tokens tokens (runner.rs:1806-1832, batched):
 *   y_{t,k} = bf16 -> f32(expert_forward(bf16(x_t)))   for the routed slots
 *   out_t   = residual_t + shared(x_t) + sum_k w_{t,k} y_{t,k}   (f32, slot order)
 * with the shared expert f32 in / f32 out (ffn_forward_sparse_f32 at tau = 0).
 * x, residual (may be NULL: zero), out: f32 [n_tokens, hidden], 16-byte
 * aligned.  ids_out / weights_out (may be NULL) receive the routing,
 * [n_tokens, top_k].  All experts of all tokens run as two grouped GEMM
 * launches; nothing is synchronised with the host. */
int cascadia_int4_moe_forward(const cascadia_int4_moe_layer *layer,
                              const cascadia_int4_routing *routing, const float *x,
                              const float *residual, uint32_t n_tokens, float *out,
                              int32_t *ids_out, float *weights_out, void *workspace,
                              void *stream);

/* Dequantise to f32 [n_rows, k_cols] (bit-exact w = q*s; the kernel's own
 * decode path).  No crate counterpart; the parity check of the weights. */
int cascadia_int4_debug_dequant(const cascadia_int4_layout *layout, const uint8_t *packed,
                                const uint8_t *scale_bits, float *w_out, void *stream);

/* The crate's C handle API (src/c_ffi.rs:35-341), same names, signatures
 * and codes.  A source is a safetensors model directory
 * (model.safetensors.index.json + shards; expert tensors
 * language_model.model.layers.L.mlp.experts.E.{gate,up,down}_proj.weight_{packed,scale},
 * packed int32 = the crate's bytes, scales bf16 or f16), or a directory whose
 * manifest.json has "experts_format": "int4_bin" (flat expert files
 * experts/layer_LL/expert_EEE.bin, manifest.rs:137-142, groups of 32, bf16
 * scales, dims "hidden_size" / "expert_intermediate").  Experts are read
 * once, uploaded and tiled into HBM on first use (prewarm does that load, the
 * analogue of the crate's page-in) and stay resident in an LRU cache
 * (cascadia_int4_source_set_cache_limits) until evicted or destroy.
 * expert_forward is synchronous and takes host arrays of the model's hidden
 * size (the crate's HIDDEN = 7168): x f32 -> bf16 (RNE, NaN quiet), the
 * expert FFN, bf16 -> f32.  Codes: 0 OK; -1 null; -2 invalid UTF-8 path
 * (open) or an expert that cannot be read (prewarm / forward); -3 a
 * directory that cannot be opened, or a HIP failure.  A handle serialises
 * its calls. */
typedef struct CascadiaInt4Source CascadiaInt4Source;
int cascadia_int4_open_source(const char *model_dir, CascadiaInt4Source **out_handle);
void cascadia_int4_destroy_source(CascadiaInt4Source *handle);
int cascadia_int4_prewarm(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert);
int cascadia_int4_expert_forward(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert,
                                 const float *x_f32, float *out_f32);

/* A handle's expert cache (no counterpart in c_ffi.rs; the runner's
 * RunnerOptions.max_cached_experts and lru_stats, runner.rs:148-170,
 * 368-416).  Resident experts form an LRU bounded by max_experts and by
 * max_bytes of HBM (0 = unbounded; the defaults come from the environment
 * variables CASCADIA_INT4_MAX_CACHED_EXPERTS / CASCADIA_INT4_EXPERT_CACHE_BYTES
 * at open).  Lowering a limit evicts at once.  A device allocation that
 * fails evicts the least recently used experts and retries before a call
 * reports -3.  Codes: 0, -1 null handle, -3 HIP failure. */
int cascadia_int4_source_set_cache_limits(CascadiaInt4Source *handle, uint64_t max_experts,
                                          uint64_t max_bytes);
int cascadia_int4_source_cache_stats(CascadiaInt4Source *handle, uint64_t *cached,
                                     uint64_t *evictions, uint64_t *resident_bytes);

/* Expert prefetch: the runner's Prefetcher (runner.rs:282-360) over
 * prefetch_expert (safetensors_source.rs:308-330), which asks the OS to page
 * an expert in ahead of use.  Here the page-in goes all the way to HBM:
 * cascadia_int4_prefetch queues (layer, expert) for a background thread of
 * the handle (started by the first call) that reads the expert into pinned
 * host memory, uploads and tiles it on a stream of its own and adds it to the
 * expert cache (the LRU limits apply), so that a later prewarm or
 * expert_forward finds it resident.  The call never blocks: with 4096
 * requests queued it drops the request (the runner's try_submit); an expert
 * already resident or being loaded is skipped, and one that cannot be read is
 * left to load (and report its error) on first use.  prewarm / expert_forward
 * of an expert the thread is loading wait for that load rather than read it a
 * second time.  cascadia_int4_prefetch_wait returns once the queue is empty
 * and no load is in progress.  cascadia_int4_prefetch_stats: requests
 * queued, dropped, taken off the queue, and loaded into HBM by the thread.
 * destroy_source drops the queued requests and joins the thread.  Codes: 0,
 * -1 null handle. */
int cascadia_int4_prefetch(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert);
int cascadia_int4_prefetch_wait(CascadiaInt4Source *handle);
int cascadia_int4_prefetch_stats(CascadiaInt4Source *handle, uint64_t *submits, uint64_t *drops,
                                 uint64_t *processed, uint64_t *loaded);

/* ---- the OpenVINO CascadiaInt4Gemv format (crates/cascadia-ov-genai-shim/
 *      cpp/gemv_offload.cpp) ---- */

/* Convert that op's packed weights -- two per byte, element 0 in the low
 * nibble, each nibble a two's-complement int4, q = (x ^ 8) - 8
 * (gemv_offload.cpp:425-429, 630-632) -- to the crate's offset nibbles
 * (q = x' - 8): every byte XOR 0x88, so the products are unchanged bit for
 * bit.  Done once at upload; packed_crate may equal packed_ov.  Its f16
 * scales [n, k / group] are already the crate layout with
 * CASCADIA_INT4_SCALE_F16; tile the result with cascadia_int4_tile_weights as
 * any crate-layout matrix. */
int cascadia_int4_ov_to_crate(const uint8_t *packed_ov, size_t n_bytes, uint8_t *packed_crate,
                              void *stream);

/* One weight segment of the op (gemv_offload.cpp:334-341): n_rows output rows,
 * packed already converted by cascadia_int4_ov_to_crate (tiling CRATE, or
 * MFMA after cascadia_int4_tile_weights), f16 scales. */
typedef struct cascadia_int4_ov_segment {
  const uint8_t *packed;
  const uint8_t *scale_f16;
  uint32_t n_rows;
  uint32_t tiling;
} cascadia_int4_ov_segment;

/* The op's evaluate() (gemv_offload.cpp:413-660): out[r, :] = the segments'
 * GEMVs of activation row r, concatenated in segment order, for rows rows;
 * act f16 (act_f16 = 1) or f32 [rows, k_cols], out f16 (RNE) or f32
 * [rows, sum of n_rows]; any group size that is a multiple of 32 dividing
 * k_cols (the op: any even size).  f32 accumulation.  workspace: >=
 * cascadia_int4_ov_gemv_workspace_bytes (256-byte aligned) or NULL. */
size_t cascadia_int4_ov_gemv_workspace_bytes(const cascadia_int4_ov_segment *segs,
                                             uint32_t n_segs, uint32_t k_cols,
                                             uint32_t group_size, uint32_t rows);
int cascadia_int4_ov_gemv(const cascadia_int4_ov_segment *segs, uint32_t n_segs,
                          uint32_t k_cols, uint32_t group_size, const void *act,
                          uint32_t act_f16, uint32_t rows, void *out, uint32_t out_f16,
                          void *workspace, void *stream);

/* Load-time quantiser: bf16 weights [n_rows, k_cols] (device, 16-byte
 * aligned) -> packed nibbles [n_rows, k_cols/2] and bf16 group scales
 * [n_rows, k_cols/group_size], the crate layout.  Replaces
 * quantize_int4_group (src/shell_int4.rs:148-212: G = 32 there; here any
 * multiple of 32 dividing k_cols), bytes identical to it: scale =
 * bf16(max|w| / 7) (1e-10 for an all-zero group), q = clamp(round(w / scale),
 * -8, 7), nibble q + 8. */
int cascadia_int4_quantize_bf16(const uint16_t *w_bf16, uint32_t n_rows, uint32_t k_cols,
                                uint32_t group_size, uint8_t *packed, uint16_t *scale_bits,
                                void *stream);

/* Streaming read of bytes at buf (16-byte aligned, a multiple of 16): each
 * wave reads one contiguous 8 KB run with non-temporal 16-byte loads, the
 * access pattern of the decode GEMV's weight stream, without its arithmetic.
 * The XOR of every 32-bit word is folded into sink (device u32 [1024], zeroed
 * by the caller): the XOR of the 1024 words is the XOR of the data.  No
 * counterpart in the crate: the HBM read ceiling the benchmark reports beside
 * the decode kernels' rates. */
int cascadia_int4_stream_read(const void *buf, size_t bytes, uint32_t *sink, void *stream);

/* Seeded synthetic data, the same generator as the test oracle.
 * kind 0: bytes (uniform nibbles), n = byte count, out u8.
 * kind 1: scales fp16/bf16(|N(0,sigma)| + offset), n = count, out u16
 *         (p0 = sigma, p1 = offset, dtype = scale dtype).
 * kind 2: f32 N(0,1), out f32.   kind 3: bf16 N(0,1), out u16. */
int cascadia_int4_fill_synthetic(uint32_t kind, uint64_t seed, uint64_t stream_id, size_t n,
                                 double p0, double p1, uint32_t dtype, void *out,
                                 void *stream);

#ifdef __cplusplus
}
#endif
#endif /* CASCADIA_INT4_H */
