// synth.hip -- seeded synthetic inputs generated in HBM (no host copies) and
// the debug dequantiser.
//
// Generator: splitmix64 over (seed, stream, index), Box-Muller in f64; the
// same algorithm as the test oracle's or_rng_u64 / or_rng_normal, so integer
// outputs (packed bytes) are bit-identical on both sides.  Floating outputs go
// through the same f64 -> f32 -> bf16/fp16 RNE steps; the f64 log/cos of the
// device math library may differ from the host libm in the last ulp, which
// survives the final rounding only in rare ties -- tests copy data between
// host and device rather than rely on regenerating it.
#include "int4_common.hpp"
#include "synth.hpp"

namespace cai4 {

CAI4_DEV uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

CAI4_DEV uint64_t rng_key(uint64_t seed, uint64_t stream) {
  return splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
}

CAI4_DEV uint64_t rng_at(uint64_t key, uint64_t idx) {
  return splitmix64(key + idx * 0x9E3779B97F4A7C15ull);
}

CAI4_DEV double rng_normal(uint64_t key, uint64_t idx) {
  const uint64_t a = rng_at(key, 2 * idx), b = rng_at(key, 2 * idx + 1);
  const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;
  const double u2 = (double)(b >> 11) * 0x1.0p-53;
  return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

// binary32 -> binary16 RNE; integer steps identical to the oracle's.
CAI4_DEV uint32_t f32_to_f16_rne(float f) {
  const uint32_t x = fbits(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFF) return man ? (sign | 0x7E00u | (man >> 13)) : (sign | 0x7C00u);
  const int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 0x1F) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    man |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    const uint32_t half = 1u << (shift - 1);
    const uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t r = man >> shift;
    if (rem > half || (rem == half && (r & 1u))) r++;
    return sign | r;
  }
  uint32_t r = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
  return sign | r;
}

__global__ void fill_bytes_kernel(uint64_t key, size_t n, uint8_t *out) {
  const size_t nw = n / 8;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nw; i += stride)
    reinterpret_cast<uint64_t *>(out)[i] = rng_at(key, i);
  if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
    const size_t b = nw * 8 + threadIdx.x;
    out[b] = (uint8_t)(rng_at(key, nw) >> (8 * threadIdx.x));
  }
}

__global__ void fill_scales_kernel(uint64_t key, size_t n, double sigma, double offset,
                                   int f16, uint16_t *out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float s = (float)fma(fabs(rng_normal(key, i)), sigma, offset);
    out[i] = (uint16_t)(f16 ? f32_to_f16_rne(s) : f32_to_bf16_rne(s));
  }
}

__global__ void fill_normal_kernel(uint64_t key, size_t n, int as_bf16, void *out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float z = (float)rng_normal(key, i);
    if (as_bf16)
      reinterpret_cast<uint16_t *>(out)[i] = (uint16_t)f32_to_bf16_rne(z);
    else
      reinterpret_cast<float *>(out)[i] = z;
  }
}

hipError_t fill_synthetic(int kind, uint64_t seed, uint64_t stream_id, size_t n, double p0,
                          double p1, int dtype, void *out, hipStream_t st) {
  if (n == 0) return hipSuccess;
  // the key is a pure function of (seed, stream): computed once on the host
  const uint64_t z = stream_id + 0x632BE59BD9B4E019ull;
  auto sm = [](uint64_t v) {
    v += 0x9E3779B97F4A7C15ull;
    v = (v ^ (v >> 30)) * 0xBF58476D1CE4E5B9ull;
    v = (v ^ (v >> 27)) * 0x94D049BB133111EBull;
    return v ^ (v >> 31);
  };
  const uint64_t k = sm(seed ^ sm(z));
  const int block = 256;
  const size_t work = kind == 0 ? (n + 7) / 8 : n;
  size_t grid = (work + block - 1) / block;
  if (grid > 8192) grid = 8192;
  if (grid == 0) grid = 1;
  switch (kind) {
    case 0:
      hipLaunchKernelGGL(fill_bytes_kernel, dim3(grid), dim3(block), 0, st, k, n,
                         (uint8_t *)out);
      break;
    case 1:
      hipLaunchKernelGGL(fill_scales_kernel, dim3(grid), dim3(block), 0, st, k, n, p0, p1,
                         dtype == SCALE_F16 ? 1 : 0, (uint16_t *)out);
      break;
    case 2:
    case 3:
      hipLaunchKernelGGL(fill_normal_kernel, dim3(grid), dim3(block), 0, st, k, n,
                         kind == 3 ? 1 : 0, out);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Debug dequantiser through the MFMA operand decode: decode8 gives
// bf16(128 + n) in k-slot order (0,2,4,6,1,3,5,7) of each dword; the column
// of slot e is 2*(e&3) + (e>>2).  w = (v - 136) * s, exact.
__global__ void dequant_kernel(const uint8_t *__restrict__ packed,
                               const uint8_t *__restrict__ scale_bits, int N, int K, int G,
                               int sdt, float *__restrict__ w) {
  const size_t dwords_per_row = (size_t)K / 8;
  const size_t total = (size_t)N * dwords_per_row;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t r = i / dwords_per_row, dq = i % dwords_per_row;
    const uint32_t d = reinterpret_cast<const uint32_t *>(packed + r * (size_t)(K / 2))[dq];
    const u32x4_t v = decode8(d);
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
    const int c0 = (int)dq * 8;
    const uint32_t bits = reinterpret_cast<const uint16_t *>(
        scale_bits + r * (size_t)(K / G) * 2)[c0 / G];
    const float s = sdt ? scale_to_f32<SCALE_F16>(bits) : scale_to_f32<SCALE_BF16>(bits);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = (words[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
      const float q = bf16_to_f32(h) - 136.0f;
      w[r * (size_t)K + c0 + 2 * (e & 3) + (e >> 2)] = q * s;
    }
  }
}

hipError_t debug_dequant(const uint8_t *packed, const uint8_t *scale_bits, int N, int K, int G,
                         int sdt, float *w, hipStream_t st) {
  const size_t total = (size_t)N * (K / 8);
  size_t grid = (total + 255) / 256;
  if (grid > 8192) grid = 8192;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(dequant_kernel, dim3(grid), dim3(256), 0, st, packed, scale_bits, N, K, G,
                     sdt, w);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// streaming read (the benchmark's HBM read ceiling)
// ---------------------------------------------------------------------------

// Each wave reads one contiguous 8 KB run (eight 1 KB wave loads, 16 bytes per
// lane, non-temporal, all issued before any is used: the access pattern of the
// decode GEMV's weight stream), XORs it, and each workgroup folds its eight
// waves into sink[blockIdx.x % 1024] by an atomic XOR, so no load is dead.
// Offsets past `bytes` read zeros (the buffer resource's range).
__global__ void __launch_bounds__(512)
    stream_read_kernel(const uint8_t *__restrict__ buf, size_t bytes, uint32_t *__restrict__ sink) {
  __shared__ uint32_t s_x[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t base = ((size_t)blockIdx.x * 8 + wave) * 8192;
  // one resource per 8 KB run (ranges up to 2 GiB; the run's bytes from base)
  const size_t left = bytes > base ? bytes - base : 0;
  const buf_rsrc_t r = buf_rsrc(buf + (left ? base : 0), left < 8192 ? left : 8192);
  u32x4_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = buf_load16_nt(r, (uint32_t)(1024 * j + 16 * lane));
  uint32_t x = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
  if (lane == 0) s_x[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t w = 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) w ^= s_x[k];
    atomicXor(sink + (blockIdx.x & 1023u), w);
  }
}

hipError_t stream_read(const void *buf, size_t bytes, uint32_t *sink, hipStream_t st) {
  const size_t grid = (bytes + 65535) / 65536;  // 8 waves x 8 KB per workgroup
  if (grid == 0 || grid > 0x7FFFFFFFu) return hipErrorInvalidValue;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(512), 0, st,
                     static_cast<const uint8_t *>(buf), bytes, sink);
  return hipGetLastError();
}

}  // namespace cai4
