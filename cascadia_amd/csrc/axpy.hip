// axpy.hip -- the AXPY form of the sparse down projection (ffn_axpy.rs).
//
// transpose_requantize_kernel  load time: the down matrix [hidden, inter]
//   (crate layout, groups along inter) dequantised, transposed to
//   [inter, hidden] and quantised again in groups of 32 along hidden with
//   bf16 scales, bit-identical to ffn_axpy.rs:342-440.  One thread per
//   destination group; neighbouring threads take neighbouring source columns,
//   so the strided source reads share cache lines.
// axpy_active_kernel  y[hidden] += sum over the active rows r of
//   scalar[r] * W_t[r, :] (ffn_axpy.rs:82-160): only the active rows are
//   read, which is what the transposed layout buys.  Grid (column chunk of
//   2048, slice of 32 active rows); a lane holds 32 columns of f32 sums and
//   each of the block's eight waves keeps four rows' loads in flight; the
//   waves are folded through LDS into one partial row per slice, and
//   axpy_reduce_kernel adds the slices to y in slice order (deterministic).
#include "int4_common.hpp"
#include "axpy.hpp"

namespace cai4 {

namespace {

__global__ void __launch_bounds__(256)
    transpose_requantize_kernel(const uint8_t *__restrict__ src, const uint16_t *__restrict__ ssc,
                                int H, int I, int G, int sdt, uint8_t *__restrict__ dst,
                                uint16_t *__restrict__ dsc) {
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int GD = H / 32;
  if (tid >= (size_t)I * GD) return;
  const int r = (int)(tid % I), g = (int)(tid / I);  // r: destination row = source column
  const int NG = I / G;
  float v[32];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const size_t h = (size_t)g * 32 + j;
    const uint32_t b = src[h * (I / 2) + r / 2];
    const int q = (int)((r & 1) ? (b >> 4) : (b & 15u)) - 8;
    v[j] = (float)q * scale_bits_f32(ssc[h * NG + r / G], sdt);
    const float a = fabsf(v[j]);
    mx = a > mx ? a : mx;
  }
  const float scale = mx == 0.0f ? 1.0f : __fdiv_rn(mx, 7.0f);
  const float inv = mx == 0.0f ? 0.0f : __fdiv_rn(1.0f, scale);
  dsc[(size_t)r * GD + g] = (uint16_t)f32_to_bf16_rne(scale);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float qf = roundf(__fmul_rn(v[j], inv));
    const int q = qf != qf ? 0 : (int)fminf(fmaxf(qf, -8.0f), 7.0f);
    w[j >> 3] |= (uint32_t)(q + 8) << (4 * (j & 7));
  }
  *reinterpret_cast<u32x4_t *>(dst + (size_t)r * (H / 2) + (size_t)g * 16) =
      u32x4_t{w[0], w[1], w[2], w[3]};
}

constexpr int kAxWaves = 8, kAxRows = 4;  // a slice: 32 active rows, 4 per wave in flight

__global__ void __launch_bounds__(64 * kAxWaves)
    axpy_active_kernel(const uint8_t *__restrict__ pt, const uint16_t *__restrict__ st,
                       const float *__restrict__ scalars, const uint32_t *__restrict__ active,
                       int n_active, const uint32_t *__restrict__ n_dev, int per_slice, int H,
                       int I, float *__restrict__ partial) {
  __shared__ float s_acc[kAxWaves - 1][2048];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 2048 + 32 * lane;  // this lane's 32 columns
  if (n_dev) n_active = min(n_active, (int)*n_dev);  // the count the device found
  const int a0 = blockIdx.y * per_slice;
  if (a0 >= n_active) return;  // uniform: a slice past the count (its partial is never read)
  const int a1 = min(a0 + per_slice, n_active);
  const int GD = H / 32;
  float acc[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) acc[j] = 0.0f;
  if (c < H) {
    for (int a = a0 + wave; a < a1; a += kAxWaves * kAxRows) {
      uint32_t r[kAxRows];
#pragma unroll
      for (int k = 0; k < kAxRows; ++k) {
        const int ak = a + k * kAxWaves;
        r[k] = ak < a1 ? active[ak] : 0xFFFFFFFFu;
      }
      u32x4_t q[kAxRows];
      float comb[kAxRows];
#pragma unroll
      for (int k = 0; k < kAxRows; ++k) {
        const bool ok = r[k] < (uint32_t)I;  // ids past the intermediate size are skipped
        q[k] = ok ? *reinterpret_cast<const u32x4_t *>(pt + (size_t)r[k] * (H / 2) + c / 2)
                  : u32x4_t{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
        comb[k] = ok ? scalars[r[k]] * bf16_to_f32(st[(size_t)r[k] * GD + c / 32]) : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < kAxRows; ++k)
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            acc[8 * d + e] += comb[k] * (float)((int)((q[k][d] >> (4 * e)) & 15u) - 8);
    }
  }
  // fold waves 1.. into wave 0 through LDS (column-major per lane)
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < 32; ++j) s_acc[wave - 1][j * 64 + lane] = acc[j];
  }
  __syncthreads();
  if (wave == 0 && c < H) {
    float *out = partial + (size_t)blockIdx.y * H + c;
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
      f32x4_t o;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float v = acc[j + k];
#pragma unroll
        for (int w = 0; w < kAxWaves - 1; ++w) v += s_acc[w][(j + k) * 64 + lane];
        o[k] = v;
      }
      *reinterpret_cast<f32x4_t *>(out + j) = o;
    }
  }
}

// 64 columns per block; wave w adds slices w, w + 4, ... (eight loads in
// flight), and the four wave sums are added in wave order: deterministic.
__global__ void __launch_bounds__(256)
    axpy_reduce_kernel(const float *__restrict__ partial, int slices, int H, float *__restrict__ y,
                       const uint32_t *__restrict__ n_dev, int per_slice, int overwrite) {
  __shared__ float s_sum[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  if (n_dev) slices = min(slices, (int)((*n_dev + per_slice - 1) / per_slice));
  float s = 0.0f;
  if (h < H) {
    for (int k = wave; k < slices; k += 32) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = k + 4 * j;
        v[j] = kk < slices ? partial[(size_t)kk * H + h] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
  }
  s_sum[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && h < H) {
    const float v = ((s_sum[0][lane] + s_sum[1][lane]) + s_sum[2][lane]) + s_sum[3][lane];
    y[h] = overwrite ? v : y[h] + v;
  }
}

}  // namespace

hipError_t transpose_requantize(const uint8_t *src, const uint8_t *src_scale_bits, int H, int I,
                                int G, int sdt, uint8_t *dst, uint8_t *dst_scale_bits,
                                hipStream_t st) {
  const size_t n = (size_t)I * (H / 32);
  hipLaunchKernelGGL(transpose_requantize_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     st, src, reinterpret_cast<const uint16_t *>(src_scale_bits), H, I, G, sdt,
                     dst, reinterpret_cast<uint16_t *>(dst_scale_bits));
  return hipGetLastError();
}

AxpyPlan axpy_plan(int H, int n_active) {
  AxpyPlan p;
  p.per_slice = kAxWaves * kAxRows;
  p.slices = n_active > 0 ? (n_active + p.per_slice - 1) / p.per_slice : 0;
  if (p.slices > 4096) {  // bound the partial rows: longer slices instead
    p.slices = 4096;
    p.per_slice = (n_active + 4095) / 4096;
  }
  p.partial_bytes = (size_t)p.slices * H * sizeof(float);
  return p;
}

hipError_t axpy_active(const uint8_t *pt, const uint8_t *st_bits, const float *scalars,
                       const uint32_t *active, int n_active, int H, int I, float *partial,
                       float *y, hipStream_t st, const uint32_t *n_dev, bool overwrite) {
  const AxpyPlan p = axpy_plan(H, n_active);
  if (p.slices == 0) return hipSuccess;
  hipLaunchKernelGGL(axpy_active_kernel, dim3((H + 2047) / 2048, p.slices), dim3(64 * kAxWaves), 0,
                     st, pt,
                     reinterpret_cast<const uint16_t *>(st_bits), scalars, active, n_active,
                     n_dev, p.per_slice, H, I, partial);
  hipLaunchKernelGGL(axpy_reduce_kernel, dim3((H + 63) / 64), dim3(256), 0, st, partial,
                     p.slices, H, y, n_dev, p.per_slice, overwrite ? 1 : 0);
  return hipGetLastError();
}

}  // namespace cai4
