/*
 * cpu_baseline.c -- the timed CPU reference: the crate's AVX-512 kernels
 * restated with the same intrinsics, parallel over rows with OpenMP.
 *
 * TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests/).
 *
 *   gemv  : kernel_avx512.rs:209-266      (seq == 1)
 *   multi : kernel_avx512_multi.rs:66-168 (seq 2..64, ROW_CHUNK 64)
 *   block : kernel_avx512_multi_blocked.rs:109-280 (RB = 2, seq 4..16)
 *   dispatch: kernel_avx512_multi.rs:207-245, _blocked.rs:295-347 and the
 *             shape table of shell_int4.rs:72-140.
 *
 * The crate runs rows on the rayon pool; here OpenMP over rows / 64-row
 * chunks on all host cores.  All three tiles are bit-identical per token
 * to int4_oracle.c's OR_ORDER_AVX512 restatement (checked in tests/).
 * Hosts without AVX-512 use an AVX2 8-lane variant (different order, timing
 * only) or the scalar kernel.rs order.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "int4_oracle.h"

static inline uint16_t ld_u16(const uint8_t *p) {
  return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

int or_cpu_isa(void) {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
      __builtin_cpu_supports("avx512vl"))
    return 2;
  if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 1;
  return 0;
}

int or_cpu_threads(void) { return omp_get_max_threads(); }

/* ---------------- AVX-512 ---------------- */

__attribute__((target("avx512f,avx512bw,avx512vl"))) static inline void
deq32_avx512(const uint8_t *p, float s, __m512 *w_lo, __m512 *w_hi) {
  const __m128i lo_mask = _mm_set1_epi8(0x0F), bias = _mm_set1_epi8(8);
  __m128i pk = _mm_loadu_si128((const __m128i *)p);
  __m128i ln = _mm_and_si128(pk, lo_mask);
  __m128i hn = _mm_and_si128(_mm_srli_epi16(pk, 4), lo_mask);
  __m128i ls = _mm_sub_epi8(ln, bias), hs = _mm_sub_epi8(hn, bias);
  __m128i il = _mm_unpacklo_epi8(ls, hs), ih = _mm_unpackhi_epi8(ls, hs);
  __m512 sv = _mm512_set1_ps(s);
  *w_lo = _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(il)), sv);
  *w_hi = _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(ih)), sv);
}

__attribute__((target("avx512f,avx512bw,avx512vl"))) static void
gemv_avx512(const uint8_t *packed, const uint8_t *scale_bits, const float *x, size_t n_rows,
            size_t k_cols, size_t group, int sdt, float *y) {
  size_t ng = k_cols / group, nch = k_cols / 32;
#pragma omp parallel for schedule(static)
  for (size_t r = 0; r < n_rows; r++) {
    const uint8_t *row = packed + r * (k_cols / 2);
    const uint8_t *srow = scale_bits + r * ng * 2;
    __m512 acc = _mm512_setzero_ps();
    for (size_t h = 0; h < nch; h++) {
      float s = or_scale_to_f32(ld_u16(srow + ((h * 32) / group) * 2), sdt);
      __m512 wl, wh;
      deq32_avx512(row + h * 16, s, &wl, &wh);
      acc = _mm512_fmadd_ps(wl, _mm512_loadu_ps(x + h * 32), acc);
      acc = _mm512_fmadd_ps(wh, _mm512_loadu_ps(x + h * 32 + 16), acc);
    }
    y[r] = _mm512_reduce_add_ps(acc);
  }
}

#define MULTI_MAX_SEQ 64
#define ROW_CHUNK 64

__attribute__((target("avx512f,avx512bw,avx512vl"))) static void
multi_avx512(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
             size_t n_rows, size_t k_cols, size_t seq, size_t group, int sdt, float *ys) {
  size_t ng = k_cols / group, nch = k_cols / 32;
  size_t n_chunks = (n_rows + ROW_CHUNK - 1) / ROW_CHUNK;
#pragma omp parallel for schedule(dynamic)
  for (size_t ci = 0; ci < n_chunks; ci++) {
    size_t r0 = ci * ROW_CHUNK, r1 = r0 + ROW_CHUNK < n_rows ? r0 + ROW_CHUNK : n_rows;
    __m512 acc[MULTI_MAX_SEQ];
    for (size_t r = r0; r < r1; r++) {
      const uint8_t *row = packed + r * (k_cols / 2);
      const uint8_t *srow = scale_bits + r * ng * 2;
      for (size_t t = 0; t < seq; t++) acc[t] = _mm512_setzero_ps();
      for (size_t h = 0; h < nch; h++) {
        float s = or_scale_to_f32(ld_u16(srow + ((h * 32) / group) * 2), sdt);
        __m512 wl, wh;
        deq32_avx512(row + h * 16, s, &wl, &wh);
        for (size_t t = 0; t < seq; t++) {
          const float *xp = xs + t * k_cols + h * 32;
          acc[t] = _mm512_fmadd_ps(wl, _mm512_loadu_ps(xp), acc[t]);
          acc[t] = _mm512_fmadd_ps(wh, _mm512_loadu_ps(xp + 16), acc[t]);
        }
      }
      for (size_t t = 0; t < seq; t++) ys[t * n_rows + r] = _mm512_reduce_add_ps(acc[t]);
    }
  }
}

#define BLOCK_MAX_SEQ 16

__attribute__((target("avx512f,avx512bw,avx512vl"))) static void
blocked_avx512(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
               size_t n_rows, size_t k_cols, size_t seq, size_t group, int sdt,
               float *ys) {
  size_t ng = k_cols / group, nch = k_cols / 32;
  size_t n_chunks = (n_rows + ROW_CHUNK - 1) / ROW_CHUNK;
#pragma omp parallel for schedule(dynamic)
  for (size_t ci = 0; ci < n_chunks; ci++) {
    size_t r0 = ci * ROW_CHUNK, r1 = r0 + ROW_CHUNK < n_rows ? r0 + ROW_CHUNK : n_rows;
    size_t rb = r0;
    __m512 a0[BLOCK_MAX_SEQ], a1[BLOCK_MAX_SEQ];
    for (; rb + 2 <= r1; rb += 2) {
      const uint8_t *p0 = packed + rb * (k_cols / 2), *p1 = p0 + k_cols / 2;
      const uint8_t *s0 = scale_bits + rb * ng * 2, *s1 = s0 + ng * 2;
      for (size_t t = 0; t < seq; t++) a0[t] = a1[t] = _mm512_setzero_ps();
      for (size_t h = 0; h < nch; h++) {
        size_t go = ((h * 32) / group) * 2;
        __m512 w0l, w0h, w1l, w1h;
        deq32_avx512(p0 + h * 16, or_scale_to_f32(ld_u16(s0 + go), sdt), &w0l, &w0h);
        deq32_avx512(p1 + h * 16, or_scale_to_f32(ld_u16(s1 + go), sdt), &w1l, &w1h);
        for (size_t t = 0; t < seq; t++) {
          const float *xp = xs + t * k_cols + h * 32;
          __m512 xl = _mm512_loadu_ps(xp), xh = _mm512_loadu_ps(xp + 16);
          a0[t] = _mm512_fmadd_ps(w0l, xl, a0[t]);
          a0[t] = _mm512_fmadd_ps(w0h, xh, a0[t]);
          a1[t] = _mm512_fmadd_ps(w1l, xl, a1[t]);
          a1[t] = _mm512_fmadd_ps(w1h, xh, a1[t]);
        }
      }
      for (size_t t = 0; t < seq; t++) {
        ys[t * n_rows + rb] = _mm512_reduce_add_ps(a0[t]);
        ys[t * n_rows + rb + 1] = _mm512_reduce_add_ps(a1[t]);
      }
    }
    for (; rb < r1; rb++) {
      const uint8_t *p0 = packed + rb * (k_cols / 2);
      const uint8_t *s0 = scale_bits + rb * ng * 2;
      for (size_t t = 0; t < seq; t++) a0[t] = _mm512_setzero_ps();
      for (size_t h = 0; h < nch; h++) {
        __m512 wl, wh;
        deq32_avx512(p0 + h * 16, or_scale_to_f32(ld_u16(s0 + ((h * 32) / group) * 2), sdt),
                     &wl, &wh);
        for (size_t t = 0; t < seq; t++) {
          const float *xp = xs + t * k_cols + h * 32;
          a0[t] = _mm512_fmadd_ps(wl, _mm512_loadu_ps(xp), a0[t]);
          a0[t] = _mm512_fmadd_ps(wh, _mm512_loadu_ps(xp + 16), a0[t]);
        }
      }
      for (size_t t = 0; t < seq; t++) ys[t * n_rows + rb] = _mm512_reduce_add_ps(a0[t]);
    }
  }
}

/* ---------------- AVX2 (non-AVX-512 hosts; timing only) ---------------- */

__attribute__((target("avx2,fma"))) static void
gemv_avx2(const uint8_t *packed, const uint8_t *scale_bits, const float *x, size_t n_rows,
          size_t k_cols, size_t group, int sdt, float *y) {
  size_t ng = k_cols / group, nch = k_cols / 32;
#pragma omp parallel for schedule(static)
  for (size_t r = 0; r < n_rows; r++) {
    const uint8_t *row = packed + r * (k_cols / 2);
    const uint8_t *srow = scale_bits + r * ng * 2;
    __m256 acc = _mm256_setzero_ps();
    const __m128i lo_mask = _mm_set1_epi8(0x0F), bias = _mm_set1_epi8(8);
    for (size_t h = 0; h < nch; h++) {
      __m256 sv =
          _mm256_set1_ps(or_scale_to_f32(ld_u16(srow + ((h * 32) / group) * 2), sdt));
      __m128i pk = _mm_loadu_si128((const __m128i *)(row + h * 16));
      __m128i ls = _mm_sub_epi8(_mm_and_si128(pk, lo_mask), bias);
      __m128i hs = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(pk, 4), lo_mask), bias);
      __m128i il = _mm_unpacklo_epi8(ls, hs), ih = _mm_unpackhi_epi8(ls, hs);
      __m128i q[4] = {il, _mm_srli_si128(il, 8), ih, _mm_srli_si128(ih, 8)};
      for (int j = 0; j < 4; j++) {
        __m256 w = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q[j])), sv);
        acc = _mm256_fmadd_ps(w, _mm256_loadu_ps(x + h * 32 + 8 * j), acc);
      }
    }
    __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s4 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
    s4 = _mm_add_ss(s4, _mm_movehdup_ps(s4));
    y[r] = _mm_cvtss_f32(s4);
  }
}

static void gemv_any(const uint8_t *packed, const uint8_t *scale_bits, const float *x,
                     size_t n_rows, size_t k_cols, size_t group, int sdt, float *y) {
  int isa = or_cpu_isa();
  if (isa == 2) {
    gemv_avx512(packed, scale_bits, x, n_rows, k_cols, group, sdt, y);
  } else if (isa == 1) {
    gemv_avx2(packed, scale_bits, x, n_rows, k_cols, group, sdt, y);
  } else {
    /* kernel.rs:31-71 scalar order, rows in parallel */
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < n_rows; r++)
      or_gemv(packed + r * (k_cols / 2), scale_bits + r * (k_cols / group) * 2, x, 1, k_cols,
              group, sdt, OR_ORDER_SCALAR, y + r);
  }
}

void or_cpu_gemm(const uint8_t *packed, const uint8_t *scale_bits, const float *xs,
                 size_t n_rows, size_t k_cols, size_t seq, size_t group, int scale_dtype,
                 float *ys) {
  int isa = or_cpu_isa();
  if (isa == 2 && seq >= 4 && seq <= BLOCK_MAX_SEQ) {
    blocked_avx512(packed, scale_bits, xs, n_rows, k_cols, seq, group, scale_dtype, ys);
    return;
  }
  if (isa == 2 && seq >= 2 && seq <= MULTI_MAX_SEQ) {
    multi_avx512(packed, scale_bits, xs, n_rows, k_cols, seq, group, scale_dtype, ys);
    return;
  }
  for (size_t t = 0; t < seq; t++)
    gemv_any(packed, scale_bits, xs + t * k_cols, n_rows, k_cols, group, scale_dtype,
             ys + t * n_rows);
}

/* Expert FFN for n_tokens rows.  One token: kernel.rs:75-136 on the
 * GEMV.  Several tokens: the crate's batched chain (shell_int4.rs:1112-1158:
 * batched gate/up, per-token SwiGLU, batched down) with expert_forward's
 * bf16 output rounding; per token the two are bit-identical. */
void or_cpu_expert_forward(const uint16_t *x_bf16, size_t n_tokens, size_t hidden,
                           size_t inter, size_t group, int scale_dtype,
                           const uint8_t *expert_flat, uint16_t *out_bf16) {
  size_t off[6];
  or_expert_offsets(hidden, inter, group, off);
  float *x = (float *)malloc(n_tokens * hidden * sizeof(float));
  float *g = (float *)malloc(n_tokens * inter * sizeof(float));
  float *u = (float *)malloc(n_tokens * inter * sizeof(float));
  float *o = (float *)malloc(n_tokens * hidden * sizeof(float));
  for (size_t i = 0; i < n_tokens * hidden; i++) x[i] = or_bf16_to_f32(x_bf16[i]);
  or_cpu_gemm(expert_flat + off[0], expert_flat + off[1], x, inter, hidden, n_tokens, group,
              scale_dtype, g);
  or_cpu_gemm(expert_flat + off[2], expert_flat + off[3], x, inter, hidden, n_tokens, group,
              scale_dtype, u);
  for (size_t i = 0; i < n_tokens * inter; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
  or_cpu_gemm(expert_flat + off[4], expert_flat + off[5], g, hidden, inter, n_tokens, group,
              scale_dtype, o);
  for (size_t i = 0; i < n_tokens * hidden; i++) out_bf16[i] = or_f32_to_bf16(o[i]);
  free(x);
  free(g);
  free(u);
  free(o);
}

/* Dense SwiGLU FFN, f32 in / f32 out (ffn_sparsity.rs:465-496 at tau 0, the
 * shared expert of shell_int4.rs:629) on the crate-dispatch GEMV. */
static void cpu_ffn_f32(const float *x, size_t hidden, size_t inter, size_t group, int sdt,
                        const uint8_t *flat, float *out) {
  size_t off[6];
  or_expert_offsets(hidden, inter, group, off);
  float *g = (float *)malloc(inter * sizeof(float));
  float *u = (float *)malloc(inter * sizeof(float));
  gemv_any(flat + off[0], flat + off[1], x, inter, hidden, group, sdt, g);
  gemv_any(flat + off[2], flat + off[3], x, inter, hidden, group, sdt, u);
  for (size_t i = 0; i < inter; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
  gemv_any(flat + off[4], flat + off[5], g, hidden, inter, group, sdt, out);
  free(g);
  free(u);
}

/* One MoE layer as the runner runs it (runner.rs:1806-1832; multi-token
 * steps keep the same per-token, per-expert loop, :2079-2108): per token,
 * per slot in selection order, skip w < threshold (:1811), y =
 * expert_forward(bf16(x_t)) (:1066-1093), moe += w * y; then
 * h = (x + shared(x)) + moe with the shared expert f32 in / f32 out.  Each
 * GEMV is the crate's rayon-parallel AVX-512 kernel; per token the result is
 * bit-identical to or_moe_layer at OR_ORDER_AVX512 (checked in tests/). */
void or_cpu_moe_layer(const float *x, size_t n_tokens, size_t hidden, size_t inter,
                      size_t group, int scale_dtype, const uint8_t *experts_base,
                      size_t expert_stride, size_t n_experts, const uint8_t *shared_flat,
                      size_t shared_inter, const int64_t *ids, const float *weights,
                      size_t top_k, float threshold, float *h_out) {
  uint16_t *xb = (uint16_t *)malloc(hidden * sizeof(uint16_t));
  uint16_t *yb = (uint16_t *)malloc(hidden * sizeof(uint16_t));
  float *moe = (float *)malloc(hidden * sizeof(float));
  float *sh = (float *)calloc(hidden, sizeof(float));
  for (size_t t = 0; t < n_tokens; t++) {
    const float *xt = x + t * hidden;
    for (size_t j = 0; j < hidden; j++) moe[j] = 0.0f;
    for (size_t j = 0; j < hidden; j++) xb[j] = or_f32_to_bf16(xt[j]);
    for (size_t k = 0; k < top_k; k++) {
      float w = weights[t * top_k + k];
      if (w < threshold) continue;
      int64_t e = ids[t * top_k + k];
      if (e < 0 || (size_t)e >= n_experts) continue;
      or_cpu_expert_forward(xb, 1, hidden, inter, group, scale_dtype,
                            experts_base + (size_t)e * expert_stride, yb);
      for (size_t j = 0; j < hidden; j++) moe[j] += w * or_bf16_to_f32(yb[j]);
    }
    if (shared_flat) cpu_ffn_f32(xt, hidden, shared_inter, group, scale_dtype, shared_flat, sh);
    for (size_t j = 0; j < hidden; j++) h_out[t * hidden + j] = xt[j] + sh[j] + moe[j];
  }
  free(xb);
  free(yb);
  free(moe);
  free(sh);
}
