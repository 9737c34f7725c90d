// sparse.hip -- the activation-sparse (tau > 0) pieces of the expert FFN
// (ffn_sparsity.rs:131-179 build_active_mask_mode, :187-348 the rows-subset
// up GEMV, :499-537 the sparse branch).  The gate and down GEMMs are the
// ordinary kernels; between them:
//
//   sparse_prep_kernel   a lane per thread over many workgroups: stable SiLU
//                        of the gate output, each workgroup's max |silu| into
//                        the token's max cell (an unsigned max of the float
//                        bits: every value is >= 0 and NaN never enters), and
//                        for per-channel thresholds whether any is > 0.
//   rows_subset_kernel   one wave per intermediate lane: the mask test
//                        |silu| >= cutoff * max (every lane when the max is 0
//                        or the mode is dense), then for an active lane the up
//                        row's dot product with x, read from either weight
//                        layout, times the SiLU -> the intermediate; 0 for an
//                        inactive lane, whose up row is never read.
//   sparse_count_kernel  the active-lane count of each token, by the same
//                        test (only when the caller asks for it).
//
// HBM traffic per token: gate and down in full, up for the active rows only.
#include "int4_common.hpp"
#include "sparse.hpp"

namespace cai4 {

namespace {

constexpr int kMaskThreads = 1024;

__global__ void fill_u32_kernel(uint32_t *p, int n, uint32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
constexpr int kMaskWaves = kMaskThreads / 64;

// ffn_sparsity.rs:141-147: the stable form, e^-g for g >= 0, e^g below.
CAI4_DEV float silu_stable(float g) {
  if (g >= 0.0f) return __fdiv_rn(g, 1.0f + expf(-g));
  const float eg = expf(g);
  return __fdiv_rn(g * eg, 1.0f + eg);
}

// ffn_sparsity.rs:487 (the dense branch): g / (1 + e^-g).
CAI4_DEV float silu_plain(float g) { return __fdiv_rn(g, 1.0f + expf(-g)); }

CAI4_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float t = __shfl_xor(v, o, 64);
    v = t > v ? t : v;
  }
  return v;
}

CAI4_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// cells of a token: [0] max |silu| bits, [1] any per-channel threshold > 0.
// PLAIN: the AXPY form's SiLU g / (1 + e^-g) (ffn_sparsity.rs:667-678), else
// the stable one of build_active_mask_mode.
template <bool PLAIN>
__global__ void __launch_bounds__(256)
    sparse_prep_kernel(const float *__restrict__ gate, int I, const float *__restrict__ thr,
                       float *__restrict__ sg, uint32_t *__restrict__ cells) {
  __shared__ float s_max[4];
  const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t row = (size_t)t * I;
  float a = 0.0f;
  int pos = 0;
  if (i < I) {
    const float s = PLAIN ? silu_plain(gate[row + i]) : silu_stable(gate[row + i]);
    sg[row + i] = s;
    a = fabsf(s);
    a = a > 0.0f ? a : 0.0f;  // NaN -> 0 (a NaN lane never raises the max)
    if (thr) pos = !(thr[i] <= 0.0f);
  }
  a = wave_max(a);
  if (lane == 0) s_max[wave] = a;
  pos = __syncthreads_or(pos);
  if (threadIdx.x == 0) {
    float m = s_max[0];
    for (int w = 1; w < 4; ++w) m = s_max[w] > m ? s_max[w] : m;
    if (m > 0.0f) atomicMax(&cells[2 * t], fbits(m));
    if (pos) atomicOr(&cells[2 * t + 1], 1u);
  }
}

// The mask test of lane i of token t (ffn_sparsity.rs:131-179); *silu
// receives the SiLU the intermediate uses: the dense branch's plain form
// when the per-channel vector is dense (:85-90, 487).
CAI4_DEV bool lane_active(const float *__restrict__ gate, const float *__restrict__ sg,
                          const float *__restrict__ thr, float tau,
                          const uint32_t *__restrict__ cells, int t, size_t at, int i,
                          float *silu) {
  const bool sparse = thr ? cells[2 * t + 1] != 0u : !(tau <= 0.0f);
  const float mx = bitsf(cells[2 * t]);
  if (!sparse) {
    *silu = silu_plain(gate[at]);
    return true;
  }
  const float s = sg[at];
  *silu = s;
  return mx == 0.0f || fabsf(s) >= (thr ? thr[i] : tau) * mx;
}

__global__ void __launch_bounds__(kMaskThreads)
    sparse_count_kernel(const float *__restrict__ gate, int I, float tau,
                        const float *__restrict__ thr, const float *__restrict__ sg,
                        const uint32_t *__restrict__ cells, uint32_t *__restrict__ counts) {
  __shared__ uint32_t s_n[kMaskWaves];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t row = (size_t)t * I;
  uint32_t n = 0;
  for (int i = tid; i < I; i += kMaskThreads) {
    float s;
    n += lane_active(gate, sg, thr, tau, cells, t, row + i, i, &s) ? 1u : 0u;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o, 64);
  if (lane == 0) s_n[wave] = n;
  __syncthreads();
  if (tid == 0) {
    uint32_t tot = 0;
    for (int w = 0; w < kMaskWaves; ++w) tot += s_n[w];
    counts[t] = tot;
  }
}

// Weight reads of one lane: 16 bytes = 32 consecutive columns [c, c + 32) of
// row r, in either layout (layout.hip: the tiled byte b holds columns b and
// b + 4 of its dword, the crate byte b columns 2b and 2b + 1).
template <int TILED>
CAI4_DEV float row_chunk_dot(const uint8_t *__restrict__ w, const uint16_t *__restrict__ s,
                             int r, int c, int K, int G, int sdt, const float *xs) {
  u32x4_t v;
  uint32_t sb;
  const int NG = K / G;
  if (TILED) {
    const size_t KB = (size_t)(K + 127) / 128;
    v = *reinterpret_cast<const u32x4_t *>(
        w + ((size_t)(r >> 4) * KB + (c >> 7)) * 1024 + 16 * ((r & 15) + 16 * ((c & 127) >> 5)));
    sb = s[((size_t)(r >> 4) * NG + c / G) * 16 + (r & 15)];
  } else {
    v = *reinterpret_cast<const u32x4_t *>(w + (size_t)r * (K / 2) + c / 2);
    sb = s[(size_t)r * NG + c / G];
  }
  float p = 0.0f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t q = v[d];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sh = TILED ? (e < 4 ? 8 * e : 8 * (e - 4) + 4) : 4 * e;
      p += (float)((int)((q >> sh) & 15u) - 8) * xs[8 * d + e];
    }
  }
  return p * scale_bits_f32(sb, sdt);
}

template <int XF32>
CAI4_DEV void load_x(const void *__restrict__ x, size_t at, float *xs) {
  if (XF32) {
    const f32x4_t *xp = reinterpret_cast<const f32x4_t *>(static_cast<const float *>(x) + at);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f32x4_t q = xp[j];
      xs[4 * j] = q.x;
      xs[4 * j + 1] = q.y;
      xs[4 * j + 2] = q.z;
      xs[4 * j + 3] = q.w;
    }
  } else {
    const u32x4_t *xp = reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(x) + at);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4_t q = xp[j];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        xs[8 * j + 2 * h] = bitsf(q[h] << 16);
        xs[8 * j + 2 * h + 1] = bitsf(q[h] & 0xFFFF0000u);
      }
    }
  }
}

template <int TILED, int XF32>
__global__ void __launch_bounds__(256)
    rows_subset_kernel(const uint8_t *__restrict__ w, const uint16_t *__restrict__ s, int I,
                       int K, int G, int sdt, const void *__restrict__ x,
                       const float *__restrict__ gate, const float *__restrict__ sg,
                       const float *__restrict__ thr, float tau,
                       const uint32_t *__restrict__ cells, float *__restrict__ inter) {
  const int t = blockIdx.y;
  const int r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= I) return;  // wave-uniform
  const size_t row = (size_t)t * I;
  float silu;
  if (!lane_active(gate, sg, thr, tau, cells, t, row + r, r, &silu)) {
    if (lane == 0) inter[row + r] = 0.0f;
    return;
  }
  float acc = 0.0f;
  // two 32-column chunks per pass: both weight loads are issued before
  // either is used
  for (int c = 32 * lane; c < K; c += 4096) {
    const bool two = c + 2048 < K;
    float xa[32], xb[32];
    load_x<XF32>(x, (size_t)t * K + c, xa);
    if (two) load_x<XF32>(x, (size_t)t * K + c + 2048, xb);
    acc += row_chunk_dot<TILED>(w, s, r, c, K, G, sdt, xa);
    if (two) acc += row_chunk_dot<TILED>(w, s, r, c + 2048, K, G, sdt, xb);
  }
  acc = wave_sum(acc);
  if (lane == 0) inter[row + r] = silu * acc;
}

}  // namespace

// Active lanes of each token in ascending order (active[t * I ..]) and their
// count, by the mask test of rows_subset_kernel: one workgroup per token, a
// chunk of 1024 lanes per pass, ranks by ballot within waves and a scan of
// the wave totals.
__global__ void __launch_bounds__(kMaskThreads)
    sparse_compact_kernel(const float *__restrict__ gate, int I, float tau,
                          const float *__restrict__ thr, const float *__restrict__ sg,
                          const uint32_t *__restrict__ cells, uint32_t *__restrict__ active,
                          uint32_t *__restrict__ counts) {
  __shared__ uint32_t s_w[kMaskWaves];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t row = (size_t)t * I;
  uint32_t base = 0;
  for (int c0 = 0; c0 < I; c0 += kMaskThreads) {
    const int i = c0 + tid;
    float s;
    const bool on = i < I && lane_active(gate, sg, thr, tau, cells, t, row + i, i, &s);
    const uint64_t b = __ballot(on);
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
    if (lane == 0) s_w[wave] = (uint32_t)__popcll(b);
    __syncthreads();
    uint32_t off = base, tot = 0;
    for (int w = 0; w < kMaskWaves; ++w) {
      const uint32_t n = s_w[w];
      if (w < wave) off += n;
      tot += n;
    }
    if (on) active[row + off + rank] = (uint32_t)i;
    base += tot;
    __syncthreads();  // s_w is rewritten by the next pass
  }
  if (tid == 0) counts[t] = base;
}

hipError_t sparse_ffn_mid(const uint8_t *w, const uint8_t *s, int I, int K, int G, int sdt,
                          int tiled, const void *x, bool x_f32, int T, const float *gate,
                          float tau, const float *thr, float *sg, uint32_t *cells, float *inter,
                          uint32_t *counts_out, hipStream_t st, bool plain_silu) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((2 * T + 255) / 256), dim3(256), 0, st, cells, 2 * T,
                     0u);
  if (plain_silu)
    hipLaunchKernelGGL(sparse_prep_kernel<true>, dim3((I + 255) / 256, T), dim3(256), 0, st, gate,
                       I, thr, sg, cells);
  else
    hipLaunchKernelGGL(sparse_prep_kernel<false>, dim3((I + 255) / 256, T), dim3(256), 0, st,
                       gate, I, thr, sg, cells);
  const dim3 grid((I + 3) / 4, T), block(256);
  const uint16_t *sc = reinterpret_cast<const uint16_t *>(s);
  if (tiled) {
    if (x_f32)
      hipLaunchKernelGGL((rows_subset_kernel<1, 1>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         gate, sg, thr, tau, cells, inter);
    else
      hipLaunchKernelGGL((rows_subset_kernel<1, 0>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         gate, sg, thr, tau, cells, inter);
  } else {
    if (x_f32)
      hipLaunchKernelGGL((rows_subset_kernel<0, 1>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         gate, sg, thr, tau, cells, inter);
    else
      hipLaunchKernelGGL((rows_subset_kernel<0, 0>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         gate, sg, thr, tau, cells, inter);
  }
  if (counts_out)
    hipLaunchKernelGGL(sparse_count_kernel, dim3(T), dim3(kMaskThreads), 0, st, gate, I, tau, thr,
                       sg, cells, counts_out);
  return hipGetLastError();
}

hipError_t sparse_compact(const float *gate, int I, int T, float tau, const float *thr,
                          const float *sg, const uint32_t *cells, uint32_t *active,
                          uint32_t *counts, hipStream_t st) {
  hipLaunchKernelGGL(sparse_compact_kernel, dim3(T), dim3(kMaskThreads), 0, st, gate, I, tau, thr,
                     sg, cells, active, counts);
  return hipGetLastError();
}

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

}  // namespace cai4
