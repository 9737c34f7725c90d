// sparse.hip -- the activation-sparse (tau > 0) expert FFN after its gate/up
// GEMM (ffn_sparsity.rs:131-179 build_active_mask_mode, :499-537 the sparse
// branch of the GEMV form, :638-740 the AXPY form; ffn_axpy.rs:82-160).
//
// Per token the mask needs the max |silu| over every intermediate lane, so the
// gate/up GEMM comes first and leaves, next to its f32 gate and up rows, one
// slot per workgroup: that workgroup's max |silu| (the f32 bits; every value
// is >= 0 and a NaN counts as 0) with bit 31 set when one of its lanes has a
// per-channel threshold > 0.  The one-token GEMV writes them from its
// epilogue (one per 16-row tile); after any other GEMM sparse_slots_kernel
// does (one per 256 lanes).  Every slot is written on every call, so nothing
// has to be cleared first.
//
// The up GEMM reads every row, as the dense FFN does: at one token on MI355X a
// rows-subset pass costs two dependent memory round trips and a launch more
// than the fused gate/up stream takes to read the inactive rows, and the
// intermediate of the active lanes is the same either way.  What the mask
// saves is the AXPY form's down: only the active rows of the transposed down
// are read.
//
//   sparse_mask_kernel   (GEMV form) a lane per thread: the token's max and
//                        flag from its slots, the test |silu| >= cutoff * max
//                        (every lane when the max is 0 or the mode is dense),
//                        inter = silu * up or 0, and the group's count.
//   sparse_axpy_kernel   (AXPY form) workgroup (512-column block, group of
//                        256 lanes, token): the same test, the active lanes
//                        listed in ascending order (ballot + mbcnt), then
//                        sum over them of inter * W_t[lane, block] into the
//                        group's partial output row.
//   sparse_axpy_reduce_kernel  the partial rows added in group order
//                        (deterministic), and the groups' counts.
#include "int4_common.hpp"
#include "sparse.hpp"

namespace cai4 {

namespace {

__global__ void fill_u32_kernel(uint32_t *p, int n, uint32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

CAI4_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float t = __shfl_xor(v, o, 64);
    v = t > v ? t : v;
  }
  return v;
}

CAI4_DEV uint32_t wave_rank(uint64_t b) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// |silu| of one lane as a slot contribution (NaN -> 0).
CAI4_DEV float slot_mag(float s) {
  const float m = fabsf(s);
  return m > 0.0f ? m : 0.0f;
}

// The slots of a gate [T, I] computed by any GEMM: one per 256 lanes.
template <bool STABLE>
__global__ void __launch_bounds__(256)
    sparse_slots_kernel(const float *__restrict__ gate, int I, const float *__restrict__ thr,
                        uint32_t *__restrict__ slots, int n_slots) {
  __shared__ float s_m[4], s_p[4];
  const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = 0.0f, pos = 0.0f;
  if (i < I) {
    const float g = gate[(size_t)t * I + i];
    m = slot_mag(STABLE ? silu_stable(g) : silu_plain(g));
    if (thr) pos = thr[i] <= 0.0f ? 0.0f : 1.0f;
  }
  m = wave_max(m);
  pos = wave_max(pos);
  if (lane == 0) {
    s_m[wave] = m;
    s_p[wave] = pos;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) {
      m = fmaxf(m, s_m[w]);
      pos = fmaxf(pos, s_p[w]);
    }
    slots[(size_t)t * n_slots + blockIdx.x] = fbits(m) | (pos > 0.0f ? 0x80000000u : 0u);
  }
}

constexpr int kSlotLoads = 8;  // slot words per thread in one round of loads

// The mask of lane i (this thread) of token t: every independent load issued
// first (the token's slots, the lane's gate / up / threshold), the slots
// folded across the workgroup (one barrier).  Returns whether the lane is
// active; *v = silu * up.  STABLE && sparse: build_active_mask_mode's SiLU.
template <bool STABLE>
CAI4_DEV bool lane_mask(const SparseMaskArgs &a, int t, int i, float *v, float *s_red,
                        uint32_t *s_flag) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t *sl = a.slots + (size_t)t * a.n_slots;
  uint32_t sv[kSlotLoads];
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    const int k = tid + 256 * u;
    sv[u] = k < a.n_slots ? sl[k] : 0u;
  }
  const bool in = i < a.I;
  const float g = in ? a.gate[(size_t)t * a.I + i] : 0.0f;
  const float up = in ? a.up[(size_t)t * a.I + i] : 0.0f;
  const float th = in && a.thr ? a.thr[i] : 0.0f;
  float m = 0.0f;
  uint32_t f = 0u;
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    m = fmaxf(m, bitsf(sv[u] & 0x7FFFFFFFu));
    f |= sv[u] >> 31;
  }
  for (int k = tid + 256 * kSlotLoads; k < a.n_slots; k += 256) {  // past 2048 slots
    const uint32_t u = sl[k];
    m = fmaxf(m, bitsf(u & 0x7FFFFFFFu));
    f |= u >> 31;
  }
  m = wave_max(m);
  const bool fw = __ballot(f != 0u) != 0ull;
  if (lane == 0) {
    s_red[wave] = m;
    s_flag[wave] = fw ? 1u : 0u;
  }
  __syncthreads();
  float mx = 0.0f;
  bool any = false;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mx = fmaxf(mx, s_red[w]);
    any = any || s_flag[w] != 0u;
  }
  // SparsityMode::is_dense (ffn_sparsity.rs:85-90): tau <= 0, or no
  // per-channel threshold > 0; then, or when the max is 0, every lane is on
  const bool sparse = a.thr ? any : !(a.tau <= 0.0f);
  const bool all = !sparse || mx == 0.0f;
  const float s = STABLE && sparse ? silu_stable(g) : silu_plain(g);
  // inter[r] = silu_gate[r] * up[r] (ffn_sparsity.rs:527, 711-716)
  *v = s * up;
  return in && (all || fabsf(s) >= (a.thr ? th : a.tau) * mx);
}

template <bool STABLE>
__global__ void __launch_bounds__(256) sparse_mask_kernel(SparseMaskArgs a) {
  __shared__ float s_red[4];
  __shared__ uint32_t s_flag[4], s_wn[4];
  const int t = blockIdx.y, i = blockIdx.x * kSparseGroup + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float v;
  const bool on = lane_mask<STABLE>(a, t, i, &v, s_red, s_flag);
  if (i < a.I) a.inter[(size_t)t * a.I + i] = on ? v : 0.0f;
  const uint64_t b = __ballot(on);
  if (lane == 0) s_wn[wave] = (uint32_t)__popcll(b);
  __syncthreads();
  if (threadIdx.x == 0)
    a.cnt[(size_t)t * gridDim.x + blockIdx.x] = ((s_wn[0] + s_wn[1]) + s_wn[2]) + s_wn[3];
}

// The AXPY form: workgroup (column block, group, token).  The group's active
// lanes are listed in ascending order; wave w takes entries w, w + 4, ...
// kAxBatch at a time, all of a batch's loads issued before any is used
// (entries past the list read its first row with weight 0); a lane owns 8
// columns (4 bytes of each transposed-down row, one bf16 scale);
// combined = inter * scale, acc += combined * n, the -8 of q = n - 8 applied
// once at the end (ffn_axpy.rs:118-134); the four waves' sums are added in
// wave order.
constexpr int kAxBatch = 16;

__global__ void __launch_bounds__(256) sparse_axpy_kernel(SparseMaskArgs a) {
  __shared__ float s_red[4];
  __shared__ uint32_t s_flag[4], s_wn[4];
  __shared__ uint32_t s_id[kSparseGroup];
  __shared__ float s_val[kSparseGroup];
  __shared__ float s_acc[3][8][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.y, tl = blockIdx.z, t = a.t0 + tl;
  const int i = g * kSparseGroup + tid;
  float v;
  const bool on = lane_mask<false>(a, t, i, &v, s_red, s_flag);
  const uint64_t b = __ballot(on);
  const uint32_t rank = wave_rank(b);
  if (lane == 0) s_wn[wave] = (uint32_t)__popcll(b);
  __syncthreads();
  uint32_t off = 0u, n = 0u;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (w < wave) off += s_wn[w];
    n += s_wn[w];
  }
  if (on) {
    s_id[off + rank] = (uint32_t)i;
    s_val[off + rank] = v;
  }
  if (blockIdx.x == 0 && tid == 0) a.cnt[(size_t)t * gridDim.y + g] = n;
  __syncthreads();

  const int c0 = blockIdx.x * kSparseAxCols + 8 * lane;  // this lane's 8 columns
  const bool cok = c0 < a.H;
  const int cc = cok ? c0 : 0;  // a lane past the columns reads column 0 and adds nothing
  const int GD = a.H / 32;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  float csum = 0.0f;
  for (int f0 = wave; f0 < (int)n; f0 += 4 * kAxBatch) {
    uint32_t q[kAxBatch], sc[kAxBatch];
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const int f = f0 + 4 * u;
      const uint32_t r = s_id[f < (int)n ? f : f0];
      q[u] = *reinterpret_cast<const uint32_t *>(a.dt + (size_t)r * (a.H / 2) + cc / 2);
      sc[u] = a.dt_s[(size_t)r * GD + cc / 32];
    }
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const int f = f0 + 4 * u;
      const float comb = f < (int)n && cok ? s_val[f] * bf16_to_f32(sc[u]) : 0.0f;
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
    float *prow = a.partial + ((size_t)tl * gridDim.y + g) * a.H + c0;
    *reinterpret_cast<f32x4_t *>(prow) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4_t *>(prow + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
  }
}

// Sum of the token's n group counts, by one wave (eight loads in flight).
CAI4_DEV uint32_t wave_count_sum(const uint32_t *__restrict__ cnt, int n, int lane) {
  uint32_t s = 0u;
  for (int k0 = lane; k0 < n; k0 += 64 * 8) {
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k0 + 64 * j < n ? cnt[k0 + 64 * j] : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  return s;
}

// out[t0 + y][h] = sum over groups of partial[y][group][h], in group order
// per wave (groups w, w + 16, ...; eight loads in flight) and the sixteen
// wave sums in wave order: deterministic.  Block (0, y) also sums the token's
// group counts.
__global__ void __launch_bounds__(1024)
    sparse_axpy_reduce_kernel(const float *__restrict__ partial, int n_groups, int H,
                              float *__restrict__ out, const uint32_t *__restrict__ cnt,
                              uint32_t *__restrict__ counts, int t0) {
  __shared__ float s_sum[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tl = blockIdx.y, t = t0 + tl, h = blockIdx.x * 64 + lane;
  const float *p = partial + (size_t)tl * n_groups * H;
  float s = 0.0f;
  if (h < H) {
    for (int k = wave; k < n_groups; k += 16 * 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = k + 16 * j;
        v[j] = kk < n_groups ? p[(size_t)kk * H + h] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s += v[j];
    }
  }
  s_sum[wave][lane] = s;
  if (counts && blockIdx.x == 0 && wave == 15) {
    const uint32_t c = wave_count_sum(cnt + (size_t)t * n_groups, n_groups, lane);
    if (lane == 0) counts[t] = c;
  }
  __syncthreads();
  if (wave == 0 && h < H) {
    float v = s_sum[0][lane];
#pragma unroll
    for (int w = 1; w < 16; ++w) v += s_sum[w][lane];
    out[(size_t)t * H + h] = v;
  }
}

__global__ void __launch_bounds__(64)
    sparse_counts_kernel(const uint32_t *__restrict__ cnt, int n_groups,
                         uint32_t *__restrict__ counts) {
  const uint32_t c = wave_count_sum(cnt + (size_t)blockIdx.x * n_groups, n_groups, threadIdx.x);
  if (threadIdx.x == 0) counts[blockIdx.x] = c;
}

}  // namespace

hipError_t sparse_slots(const float *gate, int I, int T, const float *thr, bool stable,
                        uint32_t *slots, hipStream_t st) {
  const int n = sparse_slots_per_token(I, false);
  const dim3 grid((unsigned)n, (unsigned)T);
  if (stable)
    hipLaunchKernelGGL(sparse_slots_kernel<true>, grid, dim3(256), 0, st, gate, I, thr, slots, n);
  else
    hipLaunchKernelGGL(sparse_slots_kernel<false>, grid, dim3(256), 0, st, gate, I, thr, slots,
                       n);
  return hipGetLastError();
}

hipError_t sparse_mask(const SparseMaskArgs &a, int T, bool stable, hipStream_t st) {
  const dim3 grid((unsigned)sparse_groups(a.I), (unsigned)T);
  if (stable)
    hipLaunchKernelGGL(sparse_mask_kernel<true>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(sparse_mask_kernel<false>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t sparse_axpy_ffn(const SparseMaskArgs &a, int n_tokens, float *out, uint32_t *counts,
                           hipStream_t st) {
  const int ng = sparse_groups(a.I);
  hipLaunchKernelGGL(sparse_axpy_kernel,
                     dim3((unsigned)((a.H + kSparseAxCols - 1) / kSparseAxCols), (unsigned)ng,
                          (unsigned)n_tokens),
                     dim3(256), 0, st, a);
  hipLaunchKernelGGL(sparse_axpy_reduce_kernel,
                     dim3((unsigned)((a.H + 63) / 64), (unsigned)n_tokens), dim3(1024), 0, st,
                     a.partial, ng, a.H, out, a.cnt, counts, a.t0);
  return hipGetLastError();
}

hipError_t sparse_counts(const uint32_t *cnt, int n_groups, int T, uint32_t *counts,
                         hipStream_t st) {
  hipLaunchKernelGGL(sparse_counts_kernel, dim3((unsigned)T), dim3(64), 0, st, cnt, n_groups,
                     counts);
  return hipGetLastError();
}

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

}  // namespace cai4
