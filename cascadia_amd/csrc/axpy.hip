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
//   read, which is what the transposed layout buys.  Grid (512-column block,
//   slice of 32 ids): enough workgroups to fill the chip, each wave's ids and
//   then its rows loaded in one round trip each; one partial row per slice,
//   which axpy_reduce_kernel adds to y in slice order (deterministic).
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

// axpy_active_kernel: workgroup (512-column block, slice of kAxSlice ids);
// wave w takes the slice's ids w, w + 4, ... kAxBatch at a time, every load
// of a batch (ids first, then the rows) issued before any is used; a lane
// owns 8 columns (4 bytes of each row, one bf16 scale); combined = scalar *
// scale, acc += combined * n, the -8 of q = n - 8 applied once at the end
// (ffn_axpy.rs:118-134); the four waves' sums are added in wave order into
// the slice's partial row.
constexpr int kAxSlice = 32, kAxBatch = 8, kAxCols = 512;

__global__ void __launch_bounds__(256)
    axpy_active_kernel(const uint8_t *__restrict__ pt, const uint16_t *__restrict__ st,
                       const float *__restrict__ scalars, const uint32_t *__restrict__ active,
                       int n_active, int per_slice, int H, int I, float *__restrict__ partial) {
  __shared__ float s_acc[3][8][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = blockIdx.x * kAxCols + 8 * lane;  // this lane's 8 columns
  const bool cok = c0 < H;
  const int cc = cok ? c0 : 0;  // a lane past the columns reads column 0 and adds nothing
  const int a0 = blockIdx.y * per_slice, a1 = min(a0 + per_slice, n_active);
  const int GD = H / 32;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  float csum = 0.0f;
  for (int f0 = a0 + wave; f0 < a1; f0 += 4 * kAxBatch) {
    uint32_t id[kAxBatch], q[kAxBatch], sc[kAxBatch];
    float sv[kAxBatch];
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const int f = f0 + 4 * u;
      id[u] = active[f < a1 ? f : f0];
    }
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const uint32_t r = id[u] < (uint32_t)I ? id[u] : 0u;  // ids past inter: skipped
      q[u] = *reinterpret_cast<const uint32_t *>(pt + (size_t)r * (H / 2) + cc / 2);
      sc[u] = st[(size_t)r * GD + cc / 32];
      sv[u] = scalars[r];
    }
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const bool ok = f0 + 4 * u < a1 && id[u] < (uint32_t)I && cok;
      const float comb = ok ? sv[u] * bf16_to_f32(sc[u]) : 0.0f;
      const uint32_t lo = q[u] & 0x0F0F0F0Fu, hi = (q[u] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // byte k: columns 2k (low nibble) and 2k + 1
        acc[2 * k] = fmaf(comb, (float)((lo >> (8 * k)) & 0xFFu), acc[2 * k]);
        acc[2 * k + 1] = fmaf(comb, (float)((hi >> (8 * k)) & 0xFFu), acc[2 * k + 1]);
      }
      csum += comb;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = fmaf(-8.0f, csum, acc[e]);
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave - 1][e][lane] = acc[e];
  }
  __syncthreads();
  if (wave == 0 && cok) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      acc[e] = ((acc[e] + s_acc[0][e][lane]) + s_acc[1][e][lane]) + s_acc[2][e][lane];
    float *prow = partial + (size_t)blockIdx.y * H + c0;
    *reinterpret_cast<f32x4_t *>(prow) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4_t *>(prow + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
  }
}

// y[h] += sum over slices of partial[slice][h]: 64 columns per block, wave w
// adds slices w, w + 16, ... (eight loads in flight), the sixteen wave sums
// added in wave order: deterministic.
__global__ void __launch_bounds__(1024)
    axpy_reduce_kernel(const float *__restrict__ partial, int slices, int H,
                       float *__restrict__ y) {
  __shared__ float s_sum[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (h < H) {
    for (int k = wave; k < slices; k += 16 * 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = k + 16 * j;
        v[j] = kk < slices ? partial[(size_t)kk * H + h] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
  }
  s_sum[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && h < H) {
    float v = s_sum[0][lane];
#pragma unroll
    for (int w = 1; w < 16; ++w) v += s_sum[w][lane];
    y[h] += v;
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
  p.per_slice = kAxSlice;
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
                       float *y, hipStream_t st) {
  const AxpyPlan p = axpy_plan(H, n_active);
  if (p.slices == 0) return hipSuccess;
  hipLaunchKernelGGL(axpy_active_kernel, dim3((H + kAxCols - 1) / kAxCols, p.slices), dim3(256),
                     0, st, pt, reinterpret_cast<const uint16_t *>(st_bits), scalars, active,
                     n_active, p.per_slice, H, I, partial);
  hipLaunchKernelGGL(axpy_reduce_kernel, dim3((H + 63) / 64), dim3(1024), 0, st, partial,
                     p.slices, H, y);
  return hipGetLastError();
}

}  // namespace cai4
