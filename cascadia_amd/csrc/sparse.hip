// sparse.hip -- the activation-sparse (tau > 0) pieces of the expert FFN
// (ffn_sparsity.rs:131-179 build_active_mask_mode, :187-348 the rows-subset
// up GEMV, :499-537 the sparse branch).  The gate and down GEMMs are the
// ordinary kernels; between them:
//
//   sparse_mask_kernel   one workgroup per token: stable SiLU of the gate
//                        output, max |silu|, the mask |silu| >= cutoff and the
//                        active lanes compacted in ascending order (a block
//                        prefix sum per 1024 lanes), inactive lanes of the
//                        intermediate zeroed.
//   rows_subset_kernel   one wave per active lane: the up row's dot product
//                        with x, read from either weight layout, times the
//                        lane's SiLU -> the intermediate.  Inactive rows are
//                        never read, which is the point of the sparse path.
//
// HBM traffic per token: gate and down in full, up for the active rows only.
#include "int4_common.hpp"
#include "sparse.hpp"

namespace cai4 {

namespace {

constexpr int kMaskThreads = 1024;
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

__global__ void __launch_bounds__(kMaskThreads)
    sparse_mask_kernel(const float *__restrict__ gate, int I, float tau,
                       const float *__restrict__ thr, float *__restrict__ sg,
                       uint32_t *__restrict__ act, uint32_t *__restrict__ cnt,
                       uint32_t *__restrict__ counts_out, float *__restrict__ inter) {
  __shared__ float s_max[kMaskWaves];
  __shared__ uint32_t s_pos[kMaskWaves];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t row = (size_t)t * I;
  const float *g = gate + row;
  // dense: SparsityMode::is_dense (ffn_sparsity.rs:85-90).  A per-channel
  // vector with every threshold <= 0 takes the dense branch's SiLU.
  int sparse_any = thr ? 0 : !(tau <= 0.0f);
  if (thr)
    for (int i = tid; i < I; i += kMaskThreads) sparse_any |= !(thr[i] <= 0.0f);
  sparse_any = __syncthreads_or(sparse_any);
  float mx = 0.0f;
  for (int i = tid; i < I; i += kMaskThreads) {
    const float s = sparse_any ? silu_stable(g[i]) : silu_plain(g[i]);
    sg[row + i] = s;
    const float a = fabsf(s);
    mx = a > mx ? a : mx;
  }
  mx = wave_max(mx);
  if (lane == 0) s_max[wave] = mx;
  __syncthreads();
  mx = 0.0f;
#pragma unroll
  for (int w = 0; w < kMaskWaves; ++w) mx = s_max[w] > mx ? s_max[w] : mx;
  const bool all = mx == 0.0f || !sparse_any;
  // compaction, 1024 lanes at a time, ascending
  uint32_t base = 0;
  for (int c0 = 0; c0 < I; c0 += kMaskThreads) {
    const int i = c0 + tid;
    bool on = false;
    if (i < I) {
      const float s = sg[row + i];
      on = all || fabsf(s) >= (thr ? thr[i] : tau) * mx;
      if (!on) inter[row + i] = 0.0f;
    }
    const uint64_t b = __ballot(on);
    const uint32_t below = __popcll(b & ((1ull << lane) - 1ull));
    __syncthreads();  // s_pos of the previous chunk is consumed
    if (lane == 0) s_pos[wave] = (uint32_t)__popcll(b);
    __syncthreads();
    uint32_t off = base;
    for (int w = 0; w < wave; ++w) off += s_pos[w];
    if (on) act[row + off + below] = (uint32_t)i;
    for (int w = 0; w < kMaskWaves; ++w) base += s_pos[w];
  }
  if (tid == 0) {
    cnt[t] = base;
    if (counts_out) counts_out[t] = base;
  }
}

// The same mask in one pass with each thread's NPT lanes (tid, tid + 1024,
// ...) held in registers: every load and store coalesced, the ascending
// compaction from one ballot per 1024-lane chunk and a scan of the 16 x NPT
// per-wave counts.  I <= 1024 * NPT.
template <int NPT>
__global__ void __launch_bounds__(kMaskThreads)
    sparse_mask_reg_kernel(const float *__restrict__ gate, int I, float tau,
                           const float *__restrict__ thr, float *__restrict__ sg,
                           uint32_t *__restrict__ act, uint32_t *__restrict__ cnt,
                           uint32_t *__restrict__ counts_out, float *__restrict__ inter) {
  __shared__ float s_max[kMaskWaves];
  __shared__ uint32_t s_off[NPT][kMaskWaves];
  __shared__ uint32_t s_base[NPT + 1];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t row = (size_t)t * I;
  float v[NPT], th[NPT];
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int i = k * kMaskThreads + tid;
    v[k] = i < I ? gate[row + i] : 0.0f;
    th[k] = thr && i < I ? thr[i] : 0.0f;
  }
  // SparsityMode::is_dense (ffn_sparsity.rs:85-90)
  int sparse_any = thr ? 0 : !(tau <= 0.0f);
  if (thr) {
#pragma unroll
    for (int k = 0; k < NPT; ++k) sparse_any |= (k * kMaskThreads + tid < I) & !(th[k] <= 0.0f);
  }
  sparse_any = __syncthreads_or(sparse_any);
  float mx = 0.0f;
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int i = k * kMaskThreads + tid;
    if (i < I) {
      v[k] = sparse_any ? silu_stable(v[k]) : silu_plain(v[k]);
      sg[row + i] = v[k];
      const float a = fabsf(v[k]);
      mx = a > mx ? a : mx;
    }
  }
  mx = wave_max(mx);
  if (lane == 0) s_max[wave] = mx;
  __syncthreads();
  mx = 0.0f;
#pragma unroll
  for (int w = 0; w < kMaskWaves; ++w) mx = s_max[w] > mx ? s_max[w] : mx;
  const bool all = mx == 0.0f || !sparse_any;
  uint64_t bal[NPT];
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int i = k * kMaskThreads + tid;
    const bool on = i < I && (all || fabsf(v[k]) >= (thr ? th[k] : tau) * mx);
    if (i < I && !on) inter[row + i] = 0.0f;
    bal[k] = __ballot(on);
    if (lane == 0) s_off[k][wave] = (uint32_t)__popcll(bal[k]);
  }
  __syncthreads();
  if (tid < NPT) {  // exclusive scan over the waves of chunk tid
    uint32_t run = 0;
#pragma unroll
    for (int w = 0; w < kMaskWaves; ++w) {
      const uint32_t c = s_off[tid][w];
      s_off[tid][w] = run;
      run += c;
    }
    s_base[tid + 1] = run;
  }
  __syncthreads();
  if (tid == 0) {  // exclusive scan over the chunks
    uint32_t run = 0;
    for (int k = 0; k < NPT; ++k) {
      const uint32_t c = s_base[k + 1];
      s_base[k] = run;
      run += c;
    }
    s_base[NPT] = run;
  }
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    if ((bal[k] >> lane) & 1ull)
      act[row + s_base[k] + s_off[k][wave] + __popcll(bal[k] & below)] =
          (uint32_t)(k * kMaskThreads + tid);
  }
  if (tid == 0) {
    cnt[t] = s_base[NPT];
    if (counts_out) counts_out[t] = s_base[NPT];
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
                       const uint32_t *__restrict__ act, const uint32_t *__restrict__ cnt,
                       const float *__restrict__ sg, float *__restrict__ inter) {
  const int t = blockIdx.y;
  const int slot = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (slot >= (int)cnt[t]) return;  // wave-uniform
  const size_t row = (size_t)t * I;
  const int r = (int)act[row + slot];
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
  if (lane == 0) inter[row + r] = sg[row + r] * acc;
}

}  // namespace

hipError_t sparse_mask(const float *gate, int T, int I, float tau, const float *thr, float *sg,
                       uint32_t *act, uint32_t *cnt, uint32_t *counts_out, float *inter,
                       hipStream_t st) {
  const dim3 grid(T), block(kMaskThreads);
  if (I <= 4 * kMaskThreads)
    hipLaunchKernelGGL(sparse_mask_reg_kernel<4>, grid, block, 0, st, gate, I, tau, thr, sg, act,
                       cnt, counts_out, inter);
  else if (I <= 8 * kMaskThreads)
    hipLaunchKernelGGL(sparse_mask_reg_kernel<8>, grid, block, 0, st, gate, I, tau, thr, sg, act,
                       cnt, counts_out, inter);
  else if (I <= 16 * kMaskThreads)
    hipLaunchKernelGGL(sparse_mask_reg_kernel<16>, grid, block, 0, st, gate, I, tau, thr, sg,
                       act, cnt, counts_out, inter);
  else
    hipLaunchKernelGGL(sparse_mask_kernel, grid, block, 0, st, gate, I, tau, thr, sg, act, cnt,
                       counts_out, inter);
  return hipGetLastError();
}

hipError_t rows_subset_up(const uint8_t *w, const uint8_t *s, int I, int K, int G, int sdt,
                          int tiled, const void *x, bool x_f32, int T, const uint32_t *act,
                          const uint32_t *cnt, const float *sg, float *inter, hipStream_t st) {
  const dim3 grid((I + 3) / 4, T), block(256);
  const uint16_t *sc = reinterpret_cast<const uint16_t *>(s);
  if (tiled) {
    if (x_f32)
      hipLaunchKernelGGL((rows_subset_kernel<1, 1>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         act, cnt, sg, inter);
    else
      hipLaunchKernelGGL((rows_subset_kernel<1, 0>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         act, cnt, sg, inter);
  } else {
    if (x_f32)
      hipLaunchKernelGGL((rows_subset_kernel<0, 1>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         act, cnt, sg, inter);
    else
      hipLaunchKernelGGL((rows_subset_kernel<0, 0>), grid, block, 0, st, w, sc, I, K, G, sdt, x,
                         act, cnt, sg, inter);
  }
  return hipGetLastError();
}

namespace {
__global__ void fill_u32_kernel(uint32_t *p, int n, uint32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
}  // namespace

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

}  // namespace cai4
