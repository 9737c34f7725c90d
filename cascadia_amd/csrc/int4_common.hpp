// int4_common.hpp -- device helpers shared by the gfx950 INT4 kernels.
//
// Weight format (the crate's, crates/cascadia-int4-gemm/src/format.rs:3-17 and
// kernel.rs:3-13): packed u8 [N, K/2], byte i of a row = column 2i (low nibble)
// and 2i+1 (high nibble); q = nibble - 8; scale u16 [N, K/G] little-endian,
// bf16 (the crate) or fp16; w = f32(q) * f32(scale).
//
// MFMA operand encoding used everywhere here (v_mfma_f32_16x16x32_bf16):
//   * weights enter as the bf16 value 128 + nibble (bits 0x43nn), built with one
//     v_perm_b32 per two nibbles -- exact, never a rounded q*s;
//   * the +136 offset (128 + zero-point 8) is removed by seeding the first MFMA
//     of each group with corr = -136 * sum(x) over the same k-slots, itself an
//     MFMA against the constant bf16 -136 (0xC308);
//   * the per-group scale is applied in fp32 to the group's partial sum.
//   * one MFMA's 32 k-slots are any permutation of 32 columns of one group, as
//     long as the activation fragment uses the same permutation; the nibble
//     decode yields k-slot order (0,2,4,6,1,3,5,7) inside each dword.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cai4 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define CAI4_DEV __device__ __forceinline__

enum ScaleDtype { SCALE_BF16 = 0, SCALE_F16 = 1 };

CAI4_DEV uint32_t fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
CAI4_DEV float bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

template <int SDT>
CAI4_DEV float scale_to_f32(uint32_t bits16) {
  if constexpr (SDT == SCALE_F16)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  else
    return bitsf(bits16 << 16);
}

// f32 -> bf16 bits, round to nearest even, NaN kept quiet: the crate's
// f32_to_bf16_bits (format.rs:151-160) == half::bf16::from_f32.
CAI4_DEV uint32_t f32_to_bf16_rne(float x) {
  uint32_t b = fbits(x);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return ((b >> 16) | 0x0040u) & 0xFFFFu;
  return ((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16) & 0xFFFFu;
}
CAI4_DEV float bf16_to_f32(uint32_t bits16) { return bitsf(bits16 << 16); }

CAI4_DEV f32x4_t mfma_bf16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 8 nibbles (n0 at bits 0-3 ... n7 at bits 28-31) -> 8 bf16 (128 + n) in
// k-slot order n0,n2,n4,n6,n1,n3,n5,n7.
CAI4_DEV u32x4_t decode8(uint32_t d) {
  const uint32_t t = d & 0x0F0F0F0Fu;         // bytes n0 n2 n4 n6
  const uint32_t u = (d >> 4) & 0x0F0F0F0Fu;  // bytes n1 n3 n5 n7
  const uint32_t C = 0x43434343u;
  u32x4_t r;
  r.x = __builtin_amdgcn_perm(C, t, 0x04010400u);  // [n0 | 0x43 | n2 | 0x43]
  r.y = __builtin_amdgcn_perm(C, t, 0x04030402u);  // [n4, n6]
  r.z = __builtin_amdgcn_perm(C, u, 0x04010400u);  // [n1, n3]
  r.w = __builtin_amdgcn_perm(C, u, 0x04030402u);  // [n5, n7]
  return r;
}

// 8 consecutive bf16 activations [x0|x1][x2|x3][x4|x5][x6|x7] -> the same
// k-slot order as decode8: x0,x2,x4,x6,x1,x3,x5,x7.
CAI4_DEV u32x4_t act_perm_bf16(u32x4_t d) {
  u32x4_t r;
  r.x = __builtin_amdgcn_perm(d.y, d.x, 0x05040100u);  // [x0 | x2]
  r.y = __builtin_amdgcn_perm(d.w, d.z, 0x05040100u);  // [x4 | x6]
  r.z = __builtin_amdgcn_perm(d.y, d.x, 0x07060302u);  // [x1 | x3]
  r.w = __builtin_amdgcn_perm(d.w, d.z, 0x07060302u);  // [x5 | x7]
  return r;
}

// 8 consecutive f32 activations -> hi (truncated to bf16) or lo (the exact
// f32 remainder x - hi, rounded to bf16) in the decode8 k-slot order.  hi + lo
// carries 16+ significant bits: |x - hi - lo| <= 2^-17 |x|.
CAI4_DEV u32x4_t act_split_f32(const f32x4_t &a, const f32x4_t &b, bool lo) {
  // a = x0..x3, b = x4..x7
  const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const int ord[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  u32x4_t r;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = xs[ord[2 * p]], x1 = xs[ord[2 * p + 1]];
    if (!lo) {
      w[p] = __builtin_amdgcn_perm(fbits(x1), fbits(x0), 0x07060302u);
    } else {
      const float r0 = x0 - bitsf(fbits(x0) & 0xFFFF0000u);
      const float r1 = x1 - bitsf(fbits(x1) & 0xFFFF0000u);
      f32x2_t v = {r0, r1};
      bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
      w[p] = __builtin_bit_cast(uint32_t, h);
    }
  }
  r.x = w[0];
  r.y = w[1];
  r.z = w[2];
  r.w = w[3];
  return r;
}

// 4x4 dword transpose across the four 16-lane rows: on entry row c, register
// d holds M[c][d]; on exit row c, register s holds M[s][c].
CAI4_DEV u32x4_t xpose_rows(u32x4_t v) {
  auto a = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
  auto b = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
  // a[0]=R0, a[1]=R2, b[0]=R1, b[1]=R3 after stage 1
  auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  u32x4_t r;
  r.x = c[0];
  r.y = c[1];
  r.z = d[0];
  r.w = d[1];
  return r;
}

CAI4_DEV float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// The two SiLU forms of the activation-sparse FFN, correctly rounded
// division: the plain g / (1 + e^-g) (ffn_sparsity.rs:487, 667-678) and the
// stable one of build_active_mask_mode (ffn_sparsity.rs:141-147: e^-g for
// g >= 0, e^g below).  The mask's max and its per-lane test must see the same
// bits, so every kernel computes them through these.
CAI4_DEV float silu_plain(float g) { return __fdiv_rn(g, 1.0f + expf(-g)); }
CAI4_DEV float silu_stable(float g) {
  if (g >= 0.0f) return __fdiv_rn(g, 1.0f + expf(-g));
  const float eg = expf(g);
  return __fdiv_rn(g * eg, 1.0f + eg);
}

// 8 consecutive f32 -> hi / lo bf16 in natural column order.
CAI4_DEV u32x4_t act_split_f32_nat(const f32x4_t &a, const f32x4_t &b, bool lo) {
  const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = xs[2 * p], x1 = xs[2 * p + 1];
    if (!lo) {
      w[p] = __builtin_amdgcn_perm(fbits(x1), fbits(x0), 0x07060302u);
    } else {
      const float r0 = x0 - bitsf(fbits(x0) & 0xFFFF0000u);
      const float r1 = x1 - bitsf(fbits(x1) & 0xFFFF0000u);
      f32x2_t v = {r0, r1};
      w[p] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    }
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

// Scale bits (u16 in the low half) -> f32: fp16 if sdt, else bf16.
CAI4_DEV float scale_bits_f32(uint32_t bits, int sdt) {
  return sdt ? scale_to_f32<SCALE_F16>(bits & 0xFFFFu) : scale_to_f32<SCALE_BF16>(bits & 0xFFFFu);
}

// ---- one-token helpers (gemv.hip, chain.hip) ----

typedef __amdgpu_buffer_rsrc_t buf_rsrc_t;
constexpr uint32_t kBufOOB = 0x80000000u;  // a buffer offset past any range: no data moves

// Raw buffer resource over [base, base + bytes) (clamped to 2^31 - 1 bytes).
CAI4_DEV buf_rsrc_t buf_rsrc(const void *base, size_t bytes) {
  const int n = bytes > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}
CAI4_DEV u32x4_t buf_load16(buf_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// The same load marked non-temporal (the cache-policy operand's bit 1: `nt`
// on gfx950): for weight bytes read once per call.
CAI4_DEV u32x4_t buf_load16_nt(buf_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

template <int CTRL>
CAI4_DEV float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
// Sum over a 16-lane DPP row (every lane of the row gets it).
CAI4_DEV float row16_sum(float t) {
  t += dpp_f32<0xB1>(t);   // quad_perm 1,0,3,2
  t += dpp_f32<0x4E>(t);   // quad_perm 2,3,0,1
  t += dpp_f32<0x124>(t);  // row_ror 4
  t += dpp_f32<0x128>(t);  // row_ror 8
  return t;
}

// Max over a 16-lane DPP row (every lane of the row gets it).
CAI4_DEV float row16_max(float t) {
  t = fmaxf(t, dpp_f32<0xB1>(t));
  t = fmaxf(t, dpp_f32<0x4E>(t));
  t = fmaxf(t, dpp_f32<0x124>(t));
  t = fmaxf(t, dpp_f32<0x128>(t));
  return t;
}

// Sum of 8 bf16 values (two per dword), exact pairs first.
CAI4_DEV float sum8_bf16(u32x4_t v) {
  auto lo = [](uint32_t w) { return bitsf(w << 16); };
  auto hi = [](uint32_t w) { return bitsf(w & 0xFFFF0000u); };
  return ((lo(v.x) + hi(v.x)) + (lo(v.y) + hi(v.y))) + ((lo(v.z) + hi(v.z)) + (lo(v.w) + hi(v.w)));
}


}  // namespace cai4
