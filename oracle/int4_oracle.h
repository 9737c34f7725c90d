/*
 * int4_oracle.h -- CPU restatement of cascadia-int4-gemm's INT4 weight-only
 * matmul path (the parity oracle and the CPU baseline).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load, call or link this library, and
 * only as the checker / the timed CPU reference -- never as a product path.
 * The HIP library (cascadia_amd/) never links it and has no CPU fallback.
 *
 * Every function names the reference file:line it restates, relative to the
 * labscommunity/cascadia tree.  The crate hard-codes group 32 and bf16 scales
 * (crates/cascadia-int4-gemm/src/lib.rs:73, src/format.rs:16-17); these
 * functions take the group size G (a multiple of 32 dividing K) and the scale
 * dtype as parameters and reduce exactly to the crate's arithmetic at
 * G = 32 / bf16.
 *
 * Floating-point order matters: this file is compiled with
 * -ffp-contract=off so that every a*b+c the crate writes as two Rust ops
 * (Rust never contracts) stays two roundings here, and every explicit
 * _mm512_fmadd_ps of the crate is an explicit fmaf() here.
 */
#ifndef CASCADIA_INT4_ORACLE_H
#define CASCADIA_INT4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Scale dtypes (u16 little-endian per group). */
#define OR_SCALE_BF16 0 /* the crate's format (format.rs:16-17) */
#define OR_SCALE_F16 1  /* BASELINE configs' fp16 scales */

/* GEMV summation orders the crate ships. */
#define OR_ORDER_SCALAR 0 /* kernel.rs:31-71 (non-AVX-512 hosts) */
#define OR_ORDER_AVX512 1 /* kernel_avx512.rs:209-266 (AVX-512 hosts) */

/* Routing rules. */
#define OR_ROUTE_SIGMOID_BIAS 0 /* K2.6 noaux: shell_int4.rs:588-620, glm/gate.rs:24-62 */
#define OR_ROUTE_SOFTMAX_TOPK 1 /* softmax over the top-k logits (closed form) */

/* ---- scalar conversions (format.rs:128-160, half 2.7.1) ---- */
float or_bf16_to_f32(uint16_t bits);
uint16_t or_f32_to_bf16(float x);
float or_f16_to_f32(uint16_t bits);
uint16_t or_f32_to_f16(float x);
float or_scale_to_f32(uint16_t bits, int scale_dtype);

/* ---- layout helpers (format.rs:3-17, 98-126; kernel.rs:3-13) ---- */
size_t or_packed_bytes(size_t n_rows, size_t k_cols);
size_t or_scale_bytes(size_t n_rows, size_t k_cols, size_t group);
/* Flat per-expert file: gate_p, gate_s, up_p, up_s, down_p, down_s. */
size_t or_expert_bytes(size_t hidden, size_t inter, size_t group);
void or_expert_offsets(size_t hidden, size_t inter, size_t group, size_t off[6]);

/* Dequantise to f32 [n_rows, k_cols]: w = f32(nibble - 8) * f32(scale). */
void or_dequant(const uint8_t *packed, const uint8_t *scale_bits, size_t n_rows,
                size_t k_cols, size_t group, int scale_dtype, float *w_out);

/* ---- GEMV / multi-token GEMM ---- */
void or_gemv(const uint8_t *packed, const uint8_t *scale_bits, const float *x,
             size_t n_rows, size_t k_cols, size_t group, int scale_dtype, int order,
             float *y);
/* ys[t*n_rows + r] for t < seq (kernel_avx512_multi.rs:66-168, 207-245). */
void or_gemm_multi(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
                   size_t n_rows, size_t k_cols, size_t seq, size_t group,
                   int scale_dtype, int order, float *ys);
/* Rows-subset GEMV (ffn_sparsity.rs:187-348): only rows in `rows` written. */
void or_gemv_rows_subset(const uint8_t *packed, const uint8_t *scale_bits,
                         const float *x, size_t n_rows, size_t k_cols, size_t group,
                         int scale_dtype, int order, const uint32_t *rows,
                         size_t n_active, float *y);

/* ---- expert FFN ---- */
/* kernel.rs:75-136: bf16 in, f32 inside, bf16 out. */
void or_expert_forward(const uint16_t *x_bf16, size_t hidden, size_t inter, size_t group,
                       int scale_dtype, int order, const uint8_t *expert_flat,
                       uint16_t *out_bf16);
/* ffn_sparsity.rs:438-538: f32 in, f32 out; tau <= 0 is the dense branch. */
float or_ffn_forward_f32(const float *x, size_t hidden, size_t inter, size_t group,
                         int scale_dtype, int order, const uint8_t *expert_flat,
                         float tau, float *out);
/* ffn_sparsity.rs:756-867 (global tau): tau <= 0 delegates to or_expert_forward. */
float or_expert_forward_sparse(const uint16_t *x_bf16, size_t hidden, size_t inter,
                               size_t group, int scale_dtype, int order,
                               const uint8_t *expert_flat, float tau, uint16_t *out_bf16);
/* ffn_sparsity.rs:131-179: stable SiLU, mask |silu| >= tau*max; returns count. */
size_t or_build_active_mask(const float *gate_out, size_t n, float tau, float *silu_out,
                            uint32_t *active_out);
/* The *_mode variants take per-channel thresholds (SparsityMode::PerChannel,
 * ffn_sparsity.rs:85-90, 116-179, 407, 785); NULL selects the global tau. */
size_t or_build_active_mask_mode(const float *gate_out, size_t n, float tau,
                                 const float *thresholds, float *silu_out,
                                 uint32_t *active_out);
float or_ffn_forward_f32_mode(const float *x, size_t hidden, size_t inter, size_t group,
                              int scale_dtype, int order, const uint8_t *expert_flat,
                              float tau, const float *thresholds, float *out);
float or_expert_forward_sparse_mode(const uint16_t *x_bf16, size_t hidden, size_t inter,
                                    size_t group, int scale_dtype, int order,
                                    const uint8_t *expert_flat, float tau,
                                    const float *thresholds, uint16_t *out_bf16);

/* ffn_axpy.rs:342-440 (G = 32, bf16 scales both sides). */
void or_transpose_requantize_down(const uint8_t *src_packed, const uint8_t *src_scale_bits,
                                  size_t hidden, size_t inter, uint8_t *packed_t,
                                  uint8_t *scale_t_bits);
/* ffn_axpy.rs:82-160: y += sum_{r in active} scalars[r] * W_t[r, :]. */
void or_dequant_axpy_active(const uint8_t *packed_t, const uint8_t *scale_t_bits,
                            const float *scalars, const uint32_t *active, size_t n_active,
                            size_t inter, size_t hidden, float *y);
void or_ov_gemv(const uint8_t *packed, const uint16_t *scale_f16, const float *act, size_t n,
                size_t k, size_t gsize, float *out);
float or_ffn_forward_sparse_axpy_f32_mode(const float *x, size_t hidden, size_t inter,
                                          size_t group, int scale_dtype, int order,
                                          const uint8_t *gate_p, const uint8_t *gate_s,
                                          const uint8_t *up_p, const uint8_t *up_s,
                                          const uint8_t *down_pt, const uint8_t *down_st,
                                          float tau, const float *thresholds, float *out);

/* ---- routing ---- */
/* K2.6 / GLM rule: sigmoid, choose top-k by (sigmoid + bias) with ties to the
 * lower id, weights = sigmoid of the chosen, optionally renormalised (+1e-20),
 * then times `scale`.  bias may be NULL (all zero). */
void or_route_sigmoid_bias(const float *logits, const float *bias, size_t n_experts,
                           size_t top_k, float scale, int norm, int64_t *ids,
                           float *weights);
/* Softmax over the top-k logits (ties to the lower id). */
void or_route_softmax_topk(const float *logits, size_t n_experts, size_t top_k,
                           int64_t *ids, float *weights);

/* ---- MoE layer ---- */
/* runner.rs:1806-1832 / ov_moe.rs:670-681: per token, per slot in order,
 * skip w < threshold, y = bf16->f32(expert_forward(bf16(x_t))), moe += w*y.
 * experts: E flat expert blobs at experts_base + e*expert_stride. */
void or_moe_routed(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                   size_t group, int scale_dtype, int order, const uint8_t *experts_base,
                   size_t expert_stride, size_t n_experts, const int64_t *ids,
                   const float *weights, size_t top_k, float threshold, float *moe_out);
/* One stacked layer: h = x + shared(x) + moe(x)   (runner.rs:1831).
 * shared_flat may be NULL (no shared expert). */
void or_moe_layer(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                  size_t group, int scale_dtype, int order, const uint8_t *experts_base,
                  size_t expert_stride, size_t n_experts, const uint8_t *shared_flat,
                  size_t shared_inter, const int64_t *ids, const float *weights,
                  size_t top_k, float threshold, float *h_out);

/* ---- load-time quantiser (shell_int4.rs:148-212) ---- */
void or_quantize_int4_group(const uint16_t *w_bf16, size_t n_rows, size_t k_cols,
                            size_t group, uint8_t *packed, uint8_t *scale_bits);

/* ---- seeded synthetic generators (identical algorithm in the HIP lib) ---- */
uint64_t or_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx);
double or_rng_normal(uint64_t seed, uint64_t stream, uint64_t idx);
void or_fill_bytes(uint64_t seed, uint64_t stream, size_t n_bytes, uint8_t *out);
void or_fill_scales(uint64_t seed, uint64_t stream, size_t n, int scale_dtype,
                    double sigma, double offset, uint16_t *out);
void or_fill_normal_f32(uint64_t seed, uint64_t stream, size_t n, float *out);
void or_fill_normal_bf16(uint64_t seed, uint64_t stream, size_t n, uint16_t *out);

/* ---- CPU baseline (timed; OpenMP over rows, AVX-512 when present) ---- */
/* Returns the ISA used: 2 = AVX-512, 1 = AVX2, 0 = scalar. */
int or_cpu_isa(void);
int or_cpu_threads(void);
/* The crate's dispatch (kernel_avx512_multi.rs:207-245, _blocked.rs:295-347):
 * seq == 1 or seq > 64 -> per-token GEMV; 2..64 -> multi tile. */
void or_cpu_gemm(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
                 size_t n_rows, size_t k_cols, size_t seq, size_t group,
                 int scale_dtype, float *ys);
/* Per-token expert_forward on the timed kernels (runner.rs:1806-1821). */
void or_cpu_expert_forward(const uint16_t *x_bf16, size_t n_tokens, size_t hidden,
                           size_t inter, size_t group, int scale_dtype,
                           const uint8_t *expert_flat, uint16_t *out_bf16);
void or_cpu_moe_layer(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                      size_t group, int scale_dtype, const uint8_t *experts_base,
                      size_t expert_stride, size_t n_experts, const uint8_t *shared_flat,
                      size_t shared_inter, const int64_t *ids, const float *weights,
                      size_t top_k, float threshold, float *h_out);

#ifdef __cplusplus
}
#endif
#endif
