/*
 * int4_oracle.c -- CPU restatement of cascadia-int4-gemm (parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker / timed CPU reference, never by
 * the product library.  Compiled with -ffp-contract=off (see int4_oracle.h).
 *
 * Reference: labscommunity/cascadia, crates/cascadia-int4-gemm (Rust).  The
 * crate cannot be built here (no Rust toolchain), so this is a restatement of
 * its arithmetic, function by function, with file:line citations.
 */
#include "int4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Scalar conversions                                                  */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* format.rs:130-135 */
float or_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

/* format.rs:151-160 (== half::bf16::from_f32, pinned by format.rs:173-201) */
uint16_t or_f32_to_bf16(float x) {
  uint32_t b = f2u(x);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x0040u);
  uint32_t r = b + 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

/* IEEE binary16 -> binary32, exact (half 2.7.1 f16::to_f32). */
float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      int e = -1;
      do {
        e++;
        man <<= 1;
      } while (!(man & 0x400u));
      man &= 0x3FFu;
      out = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    out = sign | 0x7F800000u | (man << 13);
  } else {
    out = sign | ((exp + 112u) << 23) | (man << 13);
  }
  return u2f(out);
}

/* binary32 -> binary16, round to nearest even (half 2.7.1 f16::from_f32). */
uint16_t or_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) {
    if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13));
    return (uint16_t)(sign | 0x7C00u);
  }
  int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t half = 1u << (shift - 1);
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t r = man >> shift;
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
  return (uint16_t)(sign | r);
}

float or_scale_to_f32(uint16_t bits, int scale_dtype) {
  return scale_dtype == OR_SCALE_F16 ? or_f16_to_f32(bits) : or_bf16_to_f32(bits);
}

static inline uint16_t ld_u16(const uint8_t *p) {
  return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

/* ------------------------------------------------------------------ */
/* Layout (format.rs:3-17, 35-47, 98-126; ov_moe.rs:792-806)           */
/* ------------------------------------------------------------------ */

size_t or_packed_bytes(size_t n_rows, size_t k_cols) { return n_rows * (k_cols / 2); }
size_t or_scale_bytes(size_t n_rows, size_t k_cols, size_t group) {
  return n_rows * (k_cols / group) * 2;
}
size_t or_expert_bytes(size_t hidden, size_t inter, size_t group) {
  size_t off[6];
  or_expert_offsets(hidden, inter, group, off);
  return off[5] + or_scale_bytes(hidden, inter, group);
}
void or_expert_offsets(size_t hidden, size_t inter, size_t group, size_t off[6]) {
  size_t gp = or_packed_bytes(inter, hidden), gs = or_scale_bytes(inter, hidden, group);
  size_t dp = or_packed_bytes(hidden, inter);
  off[0] = 0;            /* gate_packed [inter, hidden/2]   */
  off[1] = gp;           /* gate_scale  [inter, hidden/G]   */
  off[2] = gp + gs;      /* up_packed                        */
  off[3] = 2 * gp + gs;  /* up_scale                         */
  off[4] = 2 * (gp + gs);/* down_packed [hidden, inter/2]   */
  off[5] = off[4] + dp;  /* down_scale  [hidden, inter/G]   */
}

/* signed nibble of column c in a packed row: kernel.rs:8-13 */
static inline int q_at(const uint8_t *row, size_t c) {
  uint8_t b = row[c >> 1];
  int n = (c & 1) ? (b >> 4) : (b & 0x0F);
  return n - 8;
}

void or_dequant(const uint8_t *packed, const uint8_t *scale_bits, size_t n_rows,
                size_t k_cols, size_t group, int scale_dtype, float *w_out) {
  size_t ng = k_cols / group;
  for (size_t r = 0; r < n_rows; r++) {
    const uint8_t *row = packed + r * (k_cols / 2);
    for (size_t c = 0; c < k_cols; c++) {
      float s = or_scale_to_f32(ld_u16(scale_bits + (r * ng + c / group) * 2), scale_dtype);
      w_out[r * k_cols + c] = (float)q_at(row, c) * s;
    }
  }
}

/* ------------------------------------------------------------------ */
/* GEMV                                                                */
/* ------------------------------------------------------------------ */

/* kernel.rs:31-71, one row: y = sum_g s_g * (sum_{i<G/2} lo*x + hi*x). */
static float row_scalar(const uint8_t *row, const uint8_t *srow, const float *x,
                        size_t k_cols, size_t group, int sdt) {
  size_t ng = k_cols / group;
  float acc = 0.0f;
  for (size_t g = 0; g < ng; g++) {
    float scale = or_scale_to_f32(ld_u16(srow + g * 2), sdt);
    const uint8_t *gp = row + g * (group / 2);
    float gd = 0.0f;
    for (size_t i = 0; i < group / 2; i++) {
      uint8_t byte = gp[i];
      int lo = (int)(byte & 0x0F) - 8;
      int hi = (int)((byte >> 4) & 0x0F) - 8;
      size_t col = g * group + i * 2;
      gd += (float)lo * x[col];
      gd += (float)hi * x[col + 1];
    }
    acc += scale * gd;
  }
  return acc;
}

/* kernel_avx512.rs:229-263, one row.  Lane j (0..15) of the 16-wide
 * accumulator takes column 32h+j then 32h+16+j of every 32-column chunk h
 * (unpacklo/unpackhi of the low/high nibbles, :62-65), with w = q*s
 * (_mm512_mul_ps, exact) and one fused multiply-add per column (:79-80).
 * The scale of chunk h is the scale of group (32h)/G, which is the crate's
 * per-group scale at G = 32.  _mm512_reduce_add_ps (:82) is restated as the
 * halving tree (lanes i+8, i+4, i+2, i+1 folded in turn) that LLVM emits. */
static float row_avx512(const uint8_t *row, const uint8_t *srow, const float *x,
                        size_t k_cols, size_t group, int sdt) {
  float acc[16];
  for (int j = 0; j < 16; j++) acc[j] = 0.0f;
  size_t nchunks = k_cols / 32;
  for (size_t h = 0; h < nchunks; h++) {
    float s = or_scale_to_f32(ld_u16(srow + ((h * 32) / group) * 2), sdt);
    const uint8_t *p = row + h * 16;
    float lo_w[16], hi_w[16];
    for (int j = 0; j < 16; j++) {
      lo_w[j] = (float)q_at(p, (size_t)j) * s;
      hi_w[j] = (float)q_at(p, (size_t)(16 + j)) * s;
    }
    const float *xp = x + h * 32;
    for (int j = 0; j < 16; j++) acc[j] = fmaf(lo_w[j], xp[j], acc[j]);
    for (int j = 0; j < 16; j++) acc[j] = fmaf(hi_w[j], xp[16 + j], acc[j]);
  }
  for (int w = 8; w >= 1; w >>= 1)
    for (int i = 0; i < w; i++) acc[i] = acc[i] + acc[i + w];
  return acc[0];
}

static inline float row_dot(const uint8_t *packed, const uint8_t *scale_bits,
                            const float *x, size_t r, size_t k_cols, size_t group,
                            int sdt, int order) {
  const uint8_t *row = packed + r * (k_cols / 2);
  const uint8_t *srow = scale_bits + r * (k_cols / group) * 2;
  return order == OR_ORDER_SCALAR ? row_scalar(row, srow, x, k_cols, group, sdt)
                                  : row_avx512(row, srow, x, k_cols, group, sdt);
}

void or_gemv(const uint8_t *packed, const uint8_t *scale_bits, const float *x,
             size_t n_rows, size_t k_cols, size_t group, int scale_dtype, int order,
             float *y) {
  for (size_t r = 0; r < n_rows; r++)
    y[r] = row_dot(packed, scale_bits, x, r, k_cols, group, scale_dtype, order);
}

/* The multi tile and the row-blocked tile are bit-identical per token to
 * the single-token kernel (kernel_avx512_multi.rs:293-396,
 * kernel_avx512_multi_blocked.rs:392-595), so per token is the contract. */
void or_gemm_multi(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
                   size_t n_rows, size_t k_cols, size_t seq, size_t group,
                   int scale_dtype, int order, float *ys) {
  for (size_t t = 0; t < seq; t++)
    or_gemv(packed, scale_bits, xs + t * k_cols, n_rows, k_cols, group, scale_dtype,
            order, ys + t * n_rows);
}

void or_gemv_rows_subset(const uint8_t *packed, const uint8_t *scale_bits,
                         const float *x, size_t n_rows, size_t k_cols, size_t group,
                         int scale_dtype, int order, const uint32_t *rows,
                         size_t n_active, float *y) {
  (void)n_rows;
  for (size_t i = 0; i < n_active; i++) {
    size_t r = rows[i];
    y[r] = row_dot(packed, scale_bits, x, r, k_cols, group, scale_dtype, order);
  }
}

/* ------------------------------------------------------------------ */
/* Expert FFN                                                          */
/* ------------------------------------------------------------------ */

/* shell.rs:360-368 / kernel.rs:115-120: silu(g) = g / (1 + exp(-g)). */
static inline float silu_plain(float g) { return g / (1.0f + expf(-g)); }

/* kernel.rs:75-136 */
void or_expert_forward(const uint16_t *x_bf16, size_t hidden, size_t inter, size_t group,
                       int scale_dtype, int order, const uint8_t *expert_flat,
                       uint16_t *out_bf16) {
  size_t off[6];
  or_expert_offsets(hidden, inter, group, off);
  float *x = (float *)malloc(hidden * sizeof(float));
  float *g = (float *)malloc(inter * sizeof(float));
  float *u = (float *)malloc(inter * sizeof(float));
  float *m = (float *)malloc(inter * sizeof(float));
  float *o = (float *)malloc(hidden * sizeof(float));
  for (size_t i = 0; i < hidden; i++) x[i] = or_bf16_to_f32(x_bf16[i]);
  or_gemv(expert_flat + off[0], expert_flat + off[1], x, inter, hidden, group, scale_dtype,
          order, g);
  or_gemv(expert_flat + off[2], expert_flat + off[3], x, inter, hidden, group, scale_dtype,
          order, u);
  for (size_t i = 0; i < inter; i++) m[i] = silu_plain(g[i]) * u[i];
  or_gemv(expert_flat + off[4], expert_flat + off[5], m, hidden, inter, group, scale_dtype,
          order, o);
  for (size_t i = 0; i < hidden; i++) out_bf16[i] = or_f32_to_bf16(o[i]);
  free(x);
  free(g);
  free(u);
  free(m);
  free(o);
}

/* ffn_sparsity.rs:131-179 (build_active_mask_mode).  thresholds == NULL is
 * SparsityMode::Global(tau); otherwise PerChannel(thresholds[0..n]), dense
 * when every threshold is <= 0 (:85-90).  Returns the number of active
 * lanes; active_out receives them in ascending order. */
size_t or_build_active_mask_mode(const float *gate_out, size_t n, float tau,
                                 const float *thresholds, float *silu_out,
                                 uint32_t *active_out) {
  float max_abs = 0.0f;
  for (size_t i = 0; i < n; i++) {
    float g = gate_out[i], s;
    if (g >= 0.0f) {
      s = g / (1.0f + expf(-g));
    } else {
      float eg = expf(g);
      s = g * eg / (1.0f + eg);
    }
    silu_out[i] = s;
    float a = fabsf(s);
    if (a > max_abs) max_abs = a;
  }
  int dense = thresholds ? 1 : tau <= 0.0f;
  if (thresholds)
    for (size_t i = 0; i < n; i++)
      if (!(thresholds[i] <= 0.0f)) dense = 0;
  size_t cnt = 0;
  if (max_abs == 0.0f || dense) {
    for (size_t i = 0; i < n; i++) active_out[cnt++] = (uint32_t)i;
    return cnt;
  }
  for (size_t i = 0; i < n; i++) {
    float cutoff = (thresholds ? thresholds[i] : tau) * max_abs;
    if (fabsf(silu_out[i]) >= cutoff) active_out[cnt++] = (uint32_t)i;
  }
  return cnt;
}

size_t or_build_active_mask(const float *gate_out, size_t n, float tau, float *silu_out,
                            uint32_t *active_out) {
  return or_build_active_mask_mode(gate_out, n, tau, NULL, silu_out, active_out);
}

/* ffn_sparsity.rs:438-538 (ffn_forward_sparse_f32_mode; thresholds as in
 * or_build_active_mask_mode). */
float or_ffn_forward_f32_mode(const float *x, size_t hidden, size_t inter, size_t group,
                              int scale_dtype, int order, const uint8_t *expert_flat,
                              float tau, const float *thresholds, float *out) {
  size_t off[6];
  or_expert_offsets(hidden, inter, group, off);
  float *g = (float *)malloc(inter * sizeof(float));
  float *u = (float *)calloc(inter, sizeof(float));
  float *m = (float *)calloc(inter, sizeof(float));
  float frac = 1.0f;
  or_gemv(expert_flat + off[0], expert_flat + off[1], x, inter, hidden, group, scale_dtype,
          order, g);
  int dense = thresholds ? 1 : tau <= 0.0f;
  if (thresholds)
    for (size_t i = 0; i < inter; i++)
      if (!(thresholds[i] <= 0.0f)) dense = 0;
  if (dense) { /* dense branch :465-496 */
    or_gemv(expert_flat + off[2], expert_flat + off[3], x, inter, hidden, group,
            scale_dtype, order, u);
    for (size_t i = 0; i < inter; i++) m[i] = silu_plain(g[i]) * u[i];
  } else { /* sparse branch :499-537 */
    float *sg = (float *)malloc(inter * sizeof(float));
    uint32_t *act = (uint32_t *)malloc(inter * sizeof(uint32_t));
    size_t na = or_build_active_mask_mode(g, inter, tau, thresholds, sg, act);
    frac = (float)na / (float)inter;
    or_gemv_rows_subset(expert_flat + off[2], expert_flat + off[3], x, inter, hidden, group,
                        scale_dtype, order, act, na, u);
    for (size_t i = 0; i < na; i++) m[act[i]] = sg[act[i]] * u[act[i]];
    free(sg);
    free(act);
  }
  or_gemv(expert_flat + off[4], expert_flat + off[5], m, hidden, inter, group, scale_dtype,
          order, out);
  free(g);
  free(u);
  free(m);
  return frac;
}

float or_ffn_forward_f32(const float *x, size_t hidden, size_t inter, size_t group,
                         int scale_dtype, int order, const uint8_t *expert_flat,
                         float tau, float *out) {
  return or_ffn_forward_f32_mode(x, hidden, inter, group, scale_dtype, order, expert_flat, tau,
                                 NULL, out);
}

/* ffn_sparsity.rs:756-867 (expert_forward_sparse_mode; thresholds as in
 * or_build_active_mask_mode). */
float or_expert_forward_sparse_mode(const uint16_t *x_bf16, size_t hidden, size_t inter,
                                    size_t group, int scale_dtype, int order,
                                    const uint8_t *expert_flat, float tau,
                                    const float *thresholds, uint16_t *out_bf16) {
  int dense = thresholds ? 1 : tau <= 0.0f;
  if (thresholds)
    for (size_t i = 0; i < inter; i++)
      if (!(thresholds[i] <= 0.0f)) dense = 0;
  if (dense) {
    or_expert_forward(x_bf16, hidden, inter, group, scale_dtype, order, expert_flat,
                      out_bf16);
    return 1.0f;
  }
  float *x = (float *)calloc(hidden, sizeof(float));
  float *o = (float *)malloc(hidden * sizeof(float));
  for (size_t i = 0; i < hidden; i++) x[i] = or_bf16_to_f32(x_bf16[i]);
  float frac = or_ffn_forward_f32_mode(x, hidden, inter, group, scale_dtype, order,
                                       expert_flat, tau, thresholds, o);
  for (size_t i = 0; i < hidden; i++) out_bf16[i] = or_f32_to_bf16(o[i]);
  free(x);
  free(o);
  return frac;
}

float or_expert_forward_sparse(const uint16_t *x_bf16, size_t hidden, size_t inter,
                               size_t group, int scale_dtype, int order,
                               const uint8_t *expert_flat, float tau, uint16_t *out_bf16) {
  return or_expert_forward_sparse_mode(x_bf16, hidden, inter, group, scale_dtype, order,
                                       expert_flat, tau, NULL, out_bf16);
}

/* ------------------------------------------------------------------ */
/* Routing                                                             */
/* ------------------------------------------------------------------ */

/* Top-k of `key` by value descending, ties to the lower id: the result of
 * Rust's stable sort_by(b.partial_cmp(a)) over ids in ascending order
 * (shell_int4.rs:606) and of glm/gate.rs:40-47's explicit tie rule. */
static void topk_desc(const float *key, size_t n, size_t k, int64_t *ids) {
  for (size_t s = 0; s < k; s++) {
    int64_t best = -1;
    for (size_t e = 0; e < n; e++) {
      int taken = 0;
      for (size_t p = 0; p < s; p++)
        if (ids[p] == (int64_t)e) {
          taken = 1;
          break;
        }
      if (taken) continue;
      if (best < 0 || key[e] > key[best]) best = (int64_t)e;
    }
    ids[s] = best;
  }
}

/* shell_int4.rs:588-620 (K2.6, scale 2.827, norm on) and glm/gate.rs:24-62. */
void or_route_sigmoid_bias(const float *logits, const float *bias, size_t n_experts,
                           size_t top_k, float scale, int norm, int64_t *ids,
                           float *weights) {
  float *sc = (float *)malloc(n_experts * sizeof(float));
  float *ch = (float *)malloc(n_experts * sizeof(float));
  for (size_t e = 0; e < n_experts; e++) {
    sc[e] = 1.0f / (1.0f + expf(-logits[e]));
    ch[e] = sc[e] + (bias ? bias[e] : 0.0f);
  }
  topk_desc(ch, n_experts, top_k, ids);
  for (size_t k = 0; k < top_k; k++) weights[k] = sc[ids[k]];
  if (norm && top_k > 1) {
    float s = 0.0f;
    for (size_t k = 0; k < top_k; k++) s += weights[k];
    s += 1.0e-20f;
    for (size_t k = 0; k < top_k; k++) weights[k] = weights[k] / s * scale;
  } else {
    for (size_t k = 0; k < top_k; k++) weights[k] = weights[k] * scale;
  }
  free(sc);
  free(ch);
}

/* Softmax over the selected top-k logits: w_k = exp(l_k - l_max) / sum. */
void or_route_softmax_topk(const float *logits, size_t n_experts, size_t top_k,
                           int64_t *ids, float *weights) {
  topk_desc(logits, n_experts, top_k, ids);
  float mx = logits[ids[0]];
  float s = 0.0f;
  for (size_t k = 0; k < top_k; k++) {
    weights[k] = expf(logits[ids[k]] - mx);
    s += weights[k];
  }
  for (size_t k = 0; k < top_k; k++) weights[k] = weights[k] / s;
}

/* ------------------------------------------------------------------ */
/* MoE layer                                                           */
/* ------------------------------------------------------------------ */

void or_moe_routed(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                   size_t group, int scale_dtype, int order, const uint8_t *experts_base,
                   size_t expert_stride, size_t n_experts, const int64_t *ids,
                   const float *weights, size_t top_k, float threshold, float *moe_out) {
  uint16_t *xb = (uint16_t *)malloc(hidden * sizeof(uint16_t));
  uint16_t *yb = (uint16_t *)malloc(hidden * sizeof(uint16_t));
  for (size_t t = 0; t < n_tokens; t++) {
    float *moe = moe_out + t * hidden;
    for (size_t j = 0; j < hidden; j++) moe[j] = 0.0f;
    /* runner.rs:1066: x_bf16 = bf16(attn_row) */
    for (size_t j = 0; j < hidden; j++) xb[j] = or_f32_to_bf16(x[t * hidden + j]);
    for (size_t k = 0; k < top_k; k++) {
      float w = weights[t * top_k + k];
      if (w < threshold) continue; /* runner.rs:1811-1813 */
      int64_t e = ids[t * top_k + k];
      if (e < 0 || (size_t)e >= n_experts) continue;
      or_expert_forward(xb, hidden, inter, group, scale_dtype, order,
                        experts_base + (size_t)e * expert_stride, yb);
      for (size_t j = 0; j < hidden; j++) moe[j] += w * or_bf16_to_f32(yb[j]);
    }
  }
  free(xb);
  free(yb);
}

void or_moe_layer(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                  size_t group, int scale_dtype, int order, const uint8_t *experts_base,
                  size_t expert_stride, size_t n_experts, const uint8_t *shared_flat,
                  size_t shared_inter, const int64_t *ids, const float *weights,
                  size_t top_k, float threshold, float *h_out) {
  float *moe = (float *)malloc(n_tokens * hidden * sizeof(float));
  float *sh = (float *)calloc(hidden, sizeof(float));
  or_moe_routed(x, n_tokens, hidden, inter, group, scale_dtype, order, experts_base,
                expert_stride, n_experts, ids, weights, top_k, threshold, moe);
  for (size_t t = 0; t < n_tokens; t++) {
    const float *xt = x + t * hidden;
    if (shared_flat) /* shell_int4.rs:629: shared expert, f32 in/out, tau 0 */
      or_ffn_forward_f32(xt, hidden, shared_inter, group, scale_dtype, order, shared_flat,
                         0.0f, sh);
    for (size_t j = 0; j < hidden; j++) /* runner.rs:1831 */
      h_out[t * hidden + j] = xt[j] + sh[j] + moe[t * hidden + j];
  }
  free(moe);
  free(sh);
}

/* ------------------------------------------------------------------ */
/* Load-time quantiser (shell_int4.rs:148-212, generalised to G)        */
/* ------------------------------------------------------------------ */

void or_quantize_int4_group(const uint16_t *w_bf16, size_t n_rows, size_t k_cols,
                            size_t group, uint8_t *packed, uint8_t *scale_bits) {
  size_t ng = k_cols / group;
  memset(packed, 0, n_rows * k_cols / 2);
  for (size_t r = 0; r < n_rows; r++) {
    for (size_t g = 0; g < ng; g++) {
      float max_abs = 0.0f;
      for (size_t k = 0; k < group; k++) {
        float a = fabsf(or_bf16_to_f32(w_bf16[r * k_cols + g * group + k]));
        if (a > max_abs) max_abs = a;
      }
      float scale = max_abs == 0.0f ? 1.0e-10f : max_abs / 7.0f;
      /* shell_int4.rs:214-220: RNE without the NaN branch */
      uint32_t b = f2u(scale);
      uint16_t sb = (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
      size_t so = (r * ng + g) * 2;
      scale_bits[so] = (uint8_t)(sb & 0xFF);
      scale_bits[so + 1] = (uint8_t)(sb >> 8);
      float inv = 1.0f / or_bf16_to_f32(sb);
      for (size_t k = 0; k < group; k++) {
        size_t c = g * group + k;
        float w = or_bf16_to_f32(w_bf16[r * k_cols + c]);
        float qf = roundf(w * inv); /* Rust f32::round: half away from zero */
        if (qf < -8.0f) qf = -8.0f;
        if (qf > 7.0f) qf = 7.0f;
        uint8_t nib = (uint8_t)(((int)qf + 8) & 0x0F);
        size_t po = (r * k_cols + c) / 2;
        if ((c & 1) == 0)
          packed[po] = (uint8_t)((packed[po] & 0xF0) | nib);
        else
          packed[po] = (uint8_t)((packed[po] & 0x0F) | (nib << 4));
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* Seeded generators (same algorithm as cascadia_amd/csrc/synth.hip)    */
/* ------------------------------------------------------------------ */

static inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t or_rng_u64(uint64_t seed, uint64_t stream, uint64_t idx) {
  uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
  return splitmix64(key + idx * 0x9E3779B97F4A7C15ull);
}

/* Box-Muller in f64 over two draws of the same stream. */
double or_rng_normal(uint64_t seed, uint64_t stream, uint64_t idx) {
  uint64_t a = or_rng_u64(seed, stream, 2 * idx), b = or_rng_u64(seed, stream, 2 * idx + 1);
  double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
  double u2 = (double)(b >> 11) * 0x1.0p-53;
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void or_fill_bytes(uint64_t seed, uint64_t stream, size_t n_bytes, uint8_t *out) {
  for (size_t i = 0; i < n_bytes; i++) {
    uint64_t w = or_rng_u64(seed, stream, i >> 3);
    out[i] = (uint8_t)(w >> (8 * (i & 7)));
  }
}

void or_fill_scales(uint64_t seed, uint64_t stream, size_t n, int scale_dtype,
                    double sigma, double offset, uint16_t *out) {
  for (size_t i = 0; i < n; i++) {
    double z = or_rng_normal(seed, stream, i);
    float s = (float)fma(fabs(z), sigma, offset);
    out[i] = scale_dtype == OR_SCALE_F16 ? or_f32_to_f16(s) : or_f32_to_bf16(s);
  }
}

void or_fill_normal_f32(uint64_t seed, uint64_t stream, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = (float)or_rng_normal(seed, stream, i);
}

void or_fill_normal_bf16(uint64_t seed, uint64_t stream, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; i++) out[i] = or_f32_to_bf16((float)or_rng_normal(seed, stream, i));
}

/* ------------------------------------------------------------------ */
/* AXPY-form down (ffn_axpy.rs)                                        */
/* ------------------------------------------------------------------ */

/* ffn_axpy.rs:342-440: the crate's down matrix [hidden, inter] (bf16 scales,
 * groups of 32 along inter) dequantised, transposed to [inter, hidden] and
 * quantised again in groups of 32 along hidden: scale = max|v| / 7 (1.0 for
 * an all-zero group, whose codes are then 0), stored as bf16, codes
 * round(v * (1 / scale)) with the f32 scale, half away from zero, clamped to
 * [-8, 7].  The max ignores NaN (f32::max); a NaN code is 0 (`as i32`). */
void or_transpose_requantize_down(const uint8_t *src_packed, const uint8_t *src_scale_bits,
                                  size_t hidden, size_t inter, uint8_t *packed_t,
                                  uint8_t *scale_t_bits) {
  const size_t gs = inter / 32, gd = hidden / 32;
  float *t = (float *)malloc(inter * hidden * sizeof(float));
  for (size_t h = 0; h < hidden; h++)
    for (size_t c = 0; c < inter; c++) {
      const uint8_t b = src_packed[h * (inter / 2) + c / 2];
      const int q = (int)((c & 1) ? (b >> 4) : (b & 15)) - 8;
      const uint16_t sb = (uint16_t)(src_scale_bits[(h * gs + c / 32) * 2] |
                                     (src_scale_bits[(h * gs + c / 32) * 2 + 1] << 8));
      t[c * hidden + h] = (float)q * or_bf16_to_f32(sb);
    }
  for (size_t r = 0; r < inter; r++)
    for (size_t g = 0; g < gd; g++) {
      const float *v = t + r * hidden + g * 32;
      float mx = 0.0f;
      for (int i = 0; i < 32; i++) {
        const float a = fabsf(v[i]);
        if (a > mx) mx = a;
      }
      const float scale = mx == 0.0f ? 1.0f : mx / 7.0f;
      const float inv = mx == 0.0f ? 0.0f : 1.0f / scale;
      const uint16_t sb = or_f32_to_bf16(scale);
      scale_t_bits[(r * gd + g) * 2] = (uint8_t)(sb & 0xFF);
      scale_t_bits[(r * gd + g) * 2 + 1] = (uint8_t)(sb >> 8);
      for (int i = 0; i < 16; i++) {
        uint8_t nib[2];
        for (int e = 0; e < 2; e++) {
          const float qf = roundf(v[2 * i + e] * inv);
          int q = qf != qf ? 0 : (qf > 7.0f ? 7 : (qf < -8.0f ? -8 : (int)qf));
          nib[e] = (uint8_t)(q + 8);
        }
        packed_t[r * (hidden / 2) + g * 16 + i] = (uint8_t)(nib[0] | (nib[1] << 4));
      }
    }
  free(t);
}

/* ffn_axpy.rs:82-160: y[hidden] += sum over r in active (in order) of
 * scalars[r] * dequant(packed_t[r, :]); per element the product is
 * (scalar * scale) * q, as the crate forms it. */
void or_dequant_axpy_active(const uint8_t *packed_t, const uint8_t *scale_t_bits,
                            const float *scalars, const uint32_t *active, size_t n_active,
                            size_t inter, size_t hidden, float *y) {
  const size_t gd = hidden / 32;
  (void)inter;
  for (size_t a = 0; a < n_active; a++) {
    const size_t r = active[a];
    for (size_t g = 0; g < gd; g++) {
      const uint16_t sb = (uint16_t)(scale_t_bits[(r * gd + g) * 2] |
                                     (scale_t_bits[(r * gd + g) * 2 + 1] << 8));
      const float comb = scalars[r] * or_bf16_to_f32(sb);
      for (int i = 0; i < 16; i++) {
        const uint8_t b = packed_t[r * (hidden / 2) + g * 16 + i];
        y[g * 32 + 2 * i] += comb * (float)((int)(b & 15) - 8);
        y[g * 32 + 2 * i + 1] += comb * (float)((int)(b >> 4) - 8);
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* AXPY-form sparse FFN (ffn_sparsity.rs:638-740)                      */
/* ------------------------------------------------------------------ */

/* ffn_forward_sparse_axpy_f32_mode: gate in full (f32 x), plain SiLU
 * g / (1 + e^-g) and its max |.| (:667-678); every lane active when the max
 * is 0 or the mode is dense (tau <= 0, or every per-channel threshold <= 0,
 * :679-681), else |silu| >= tau * max (:682-700); up for the active rows
 * (:704-714), inter = silu * up on them (:717-722), out = 0 then the AXPY of
 * the active rows of the transposed down (:730-738).  down_pt / down_st:
 * transpose_requantize_down's [inter, hidden] codes and bf16 scales.
 * Returns the active fraction. */
float or_ffn_forward_sparse_axpy_f32_mode(const float *x, size_t hidden, size_t inter,
                                          size_t group, int scale_dtype, int order,
                                          const uint8_t *gate_p, const uint8_t *gate_s,
                                          const uint8_t *up_p, const uint8_t *up_s,
                                          const uint8_t *down_pt, const uint8_t *down_st,
                                          float tau, const float *thresholds, float *out) {
  float *g = (float *)malloc(inter * sizeof(float));
  float *sg = (float *)malloc(inter * sizeof(float));
  float *u = (float *)calloc(inter, sizeof(float));
  float *m = (float *)calloc(inter, sizeof(float));
  uint32_t *act = (uint32_t *)malloc(inter * sizeof(uint32_t));
  or_gemv(gate_p, gate_s, x, inter, hidden, group, scale_dtype, order, g);
  float max_abs = 0.0f;
  for (size_t i = 0; i < inter; i++) {
    sg[i] = silu_plain(g[i]);
    const float a = fabsf(sg[i]);
    if (a > max_abs) max_abs = a;
  }
  /* SparsityMode::is_dense (ffn_sparsity.rs:85-90): tau <= 0, so a NaN tau is sparse */
  int dense = thresholds ? 1 : tau <= 0.0f;
  if (thresholds)
    for (size_t i = 0; i < inter; i++)
      if (!(thresholds[i] <= 0.0f)) dense = 0;
  size_t na = 0;
  for (size_t i = 0; i < inter; i++) {
    const float cut = (thresholds ? thresholds[i] : tau) * max_abs;
    if (max_abs == 0.0f || dense || fabsf(sg[i]) >= cut) act[na++] = (uint32_t)i;
  }
  or_gemv_rows_subset(up_p, up_s, x, inter, hidden, group, scale_dtype, order, act, na, u);
  for (size_t a = 0; a < na; a++) m[act[a]] = sg[act[a]] * u[act[a]];
  for (size_t j = 0; j < hidden; j++) out[j] = 0.0f;
  or_dequant_axpy_active(down_pt, down_st, m, act, na, inter, hidden, out);
  free(g);
  free(sg);
  free(u);
  free(m);
  free(act);
  return (float)na / (float)inter;
}

/* ------------------------------------------------------------------ */
/* OpenVINO CascadiaInt4Gemv (cascadia-ov-genai-shim/cpp/gemv_offload.cpp) */
/* ------------------------------------------------------------------ */

/* The op's scalar evaluate path (gemv_offload.cpp:623-638) for one row of
 * activations: packed [n, k/2], element 0 in the low nibble, each nibble a
 * two's-complement int4 (sign-extended: (b << 4) >> 4 and b >> 4 of the int8
 * byte, :630-632); f16 scales [n, k / gsize]; per group dot += lo * a[2j],
 * dot += hi * a[2j + 1] in order, then acc += f32(scale) * dot. */
void or_ov_gemv(const uint8_t *packed, const uint16_t *scale_f16, const float *act, size_t n,
                size_t k, size_t gsize, float *out) {
  const size_t groups = k / gsize;
  for (size_t r = 0; r < n; r++) {
    const uint8_t *wrow = packed + r * (k / 2);
    float acc = 0.0f;
    for (size_t gi = 0; gi < groups; gi++) {
      const uint8_t *gw = wrow + gi * (gsize / 2);
      const float *ga = act + gi * gsize;
      float dot = 0.0f;
      for (size_t j = 0; j < gsize / 2; j++) {
        const uint8_t b = gw[j];
        const int lo = (int)(int8_t)(uint8_t)(b << 4) >> 4;
        const int hi = (int)(int8_t)b >> 4;
        dot += (float)lo * ga[2 * j];
        dot += (float)hi * ga[2 * j + 1];
      }
      acc += or_f16_to_f32(scale_f16[r * groups + gi]) * dot;
    }
    out[r] = acc;
  }
}
