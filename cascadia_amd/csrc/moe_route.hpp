// moe_route.hpp -- routing of one token in one wave (device code shared by the
// routing kernels and the one-token expert GEMV): sigmoid + bias top-k with
// optional renormalisation and scale, or softmax over the top-k logits
// (crates/cascadia-int4-gemm/src/shell_int4.rs:588-620, glm/gate.rs:24-62).
#pragma once
#include <math.h>

#include "int4_common.hpp"
#include "moe.hpp"

namespace cai4 {

// Wave-wide max of a float, in every lane: DPP within 16-lane rows (xor 1,
// xor 2, rotate 4, rotate 8), then row pairs and halves by permlane swaps --
// no LDS round trips.
CAI4_DEV float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm 1,0,3,2
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm 2,3,0,1
  v = fmaxf(v, dpp_f32<0x124>(v));  // row_ror 4
  v = fmaxf(v, dpp_f32<0x128>(v));  // row_ror 8
  auto a = __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false);
  v = fmaxf(bitsf(a[0]), bitsf(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
  return fmaxf(bitsf(b[0]), bitsf(b[1]));
}

CAI4_DEV float lane_f32(float v, int l) {
  return bitsf(__builtin_amdgcn_readlane(fbits(v), l));
}

// Selections of token t in one wave.  Lane l holds experts l * nj .. l * nj +
// nj - 1, so the lowest lane holding a maximum holds the lowest expert id of
// it.  Each of the k rounds takes the lane-local best (lowest j among equal
// keys), a wave-wide max, and the lowest lane whose best equals it.  NaN keys
// never win.  Lane kk < k returns selection kk: its expert and weight.
template <int R>  // R >= ceil(E / 64): registers per lane
CAI4_DEV void route_token(const MoeRouting &r, int t, int E, int lane, int &id_out,
                          float &w_out) {
  const bool sig = r.mode == ROUTE_SIGMOID_BIAS;
  const int nj = (E + 63) >> 6;
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(r.logits + (size_t)t * E), (short)0, E * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(r.bias), (short)0, r.bias ? E * 4 : 0, 0x00020000);
  // every load first (registers past nj read nothing), then the keys: one
  // memory round trip, not one per register
  float lg[R], bs[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const uint32_t off = j < nj ? (uint32_t)(lane * nj + j) * 4 : kBufOOB;
    lg[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, off, 0, 0));
    bs[j] = sig ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0)) : 0.f;
  }
  float key[R], val[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    key[j] = -INFINITY;
    val[j] = 0.f;
    if (j < nj) {  // uniform
      const float sv = sig ? 1.0f / (1.0f + expf(-lg[j])) : lg[j];
      const float c = sig ? sv + bs[j] : sv;
      val[j] = sv;
      key[j] = c != c ? -INFINITY : c;
    }
  }
  uint32_t valid = 0;  // experts of this lane that exist and are not yet taken
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (j < nj && lane * nj + j < E) valid |= 1u << j;
  int my_id = 0;
  float my_val = 0.f;
  for (int kk = 0; kk < r.top_k; ++kk) {
    float best = -INFINITY, bval = 0.f;
    int bj = -1;
#pragma unroll
    for (int j = 0; j < R; ++j) {  // selects, not branches: no exec-mask round trips
      const bool take = ((valid >> j) & 1u) & ((bj < 0) | (key[j] > best));
      best = take ? key[j] : best;
      bval = take ? val[j] : bval;
      bj = take ? j : bj;
    }
    const float m = wave_max_f32(bj < 0 ? -INFINITY : best);
    const uint64_t hit = __ballot(bj >= 0 && best == m);
    const int sl = __builtin_amdgcn_readfirstlane(__builtin_ffsll((long long)hit) - 1);
    const int sj = __builtin_amdgcn_readlane(bj, sl);
    const float sv = lane_f32(bval, sl);
    if (lane == sl) valid &= ~(1u << sj);
    if (lane == kk) {
      my_id = sl * nj + sj;
      my_val = sv;
    }
  }
  // weights, summed in selection order as the crate does
  const int k = r.top_k;
  float w;
  if (sig) {
    if (r.normalize && k > 1) {
      float s = 0.0f;
      for (int kk = 0; kk < k; ++kk) s += lane_f32(my_val, kk);
      s += 1.0e-20f;
      w = my_val / s * r.scale;
    } else {
      w = my_val * r.scale;
    }
  } else {
    const float mx = lane_f32(my_val, 0);
    const float ex = expf(my_val - mx);
    float s = 0.0f;
    for (int kk = 0; kk < k; ++kk) s += lane_f32(ex, kk);
    w = ex / s;
  }
  id_out = my_id;
  w_out = w;
}

}  // namespace cai4
