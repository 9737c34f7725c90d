// moe.hip -- the sparse-MoE expert path of one layer on one GPU: routing,
// grouping of (token, slot) assignments by expert, and the weighted combine.
// The expert FFNs themselves run as two grouped skinny GEMMs (skinny.hip,
// grouped mode) over all active experts at once.
//
// Semantics follow the crate's CPU runner: per token, per slot in selection
// order, skip w < threshold, y = bf16 -> f32(expert_forward(bf16(x_t))),
// moe += w * y (multiply, then add: no fused multiply-add), and
// h = residual + shared + moe (crates/cascadia-engine-sparse-moe/src/runner.rs:
// 1806-1832).  Routing rules: sigmoid scores, top-k by score + bias, ties to
// the lower expert id, optional renormalisation (sum + 1e-20) times a scale
// (crates/cascadia-int4-gemm/src/shell_int4.rs:588-620, glm/gate.rs:24-62);
// or top-k by logit with a softmax over the selected logits.
//
// Positions inside an expert's group come from LDS atomics, so the order of
// tokens within a group varies between calls; every output is still
// deterministic, because each token row of a grouped GEMM is computed
// independently of its position and the combine reads slots in order.
#include <math.h>

#include "int4_common.hpp"
#include "moe.hpp"

namespace cai4 {

namespace {
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

int moe_chunk_rows(int T, int per_expert_max) {
  const int c = T <= 8 ? 8 : (T <= 64 ? 16 : 32);
  return per_expert_max < c ? per_expert_max : c;
}

int moe_max_chunks(int T, int E, int top_k, int chunk_rows) {
  // sum_e ceil(c_e / C) <= A + (n - A) / C for A active experts, largest at
  // A = min(n, E)
  const long n = (long)T * top_k, a = n < E ? n : E;
  return (int)(a + (n - a) / chunk_rows);
}

MoeWorkspace moe_workspace(int T, int H, int I, int E, int top_k, int chunk_rows,
                           size_t part_bytes, size_t shared_bytes, size_t shared_ws_bytes) {
  MoeWorkspace w{};
  const size_t n = (size_t)T * top_k;
  w.chunk_rows = chunk_rows;
  w.max_chunks = moe_max_chunks(T, E, top_k, w.chunk_rows);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  w.ids = take(n * 4);
  w.weights = take(n * 4);
  w.pos = take(n * 4);
  w.row_map = take(n * 4);
  w.chunks = take((size_t)w.max_chunks * sizeof(SkinnyChunk));
  w.counts = take(16);
  w.xg = take(n * H * 2);
  w.hi = take(n * I * 2);
  w.lo = take(n * I * 2);
  w.y = take(n * H * 2);
  w.shared = take(shared_bytes);
  w.part = take(part_bytes);
  w.shared_ws = take(shared_ws_bytes);
  w.total = o;
  return w;
}

// ---------------------------------------------------------------------------
// routing: one wave per token
// ---------------------------------------------------------------------------

CAI4_DEV bool better(float c, int i, float bc, int bi) { return c > bc || (c == bc && i < bi); }

__global__ __launch_bounds__(256) void moe_route_kernel(MoeRouting r, int T, int E, int32_t *ids,
                                                        float *wout) {
  constexpr int R = kMoeMaxExperts / 64;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves; no barriers in this kernel
  const bool sig = r.mode == ROUTE_SIGMOID_BIAS;
  const int nj = (E + 63) >> 6;  // registers in use per lane
  // all loads first, branch-free (experts past E read 0 from the range check)
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(r.logits + (size_t)t * E), (short)0, E * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(r.bias), (short)0, r.bias ? E * 4 : 0, 0x00020000);
  float lg[R], bs[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const uint32_t off = j < nj ? (uint32_t)(lane + 64 * j) * 4 : 0x80000000u;
    lg[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, off, 0, 0));
    bs[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0));
  }
  float choice[R], val[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const bool ok = lane + 64 * j < E;
    const float s = sig ? 1.0f / (1.0f + expf(-lg[j])) : lg[j];
    val[j] = s;
    choice[j] = ok ? (sig ? s + bs[j] : s) : -INFINITY;
  }
  // k rounds of a wave-wide argmax (ties to the lower id); lane kk keeps
  // selection kk
  uint32_t taken = 0;
  float my_val = 0.f;
  int my_id = 0;
  for (int kk = 0; kk < r.top_k; ++kk) {
    float bc = -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int e = lane + 64 * j;
      if (j < nj && e < E && !((taken >> j) & 1u) && better(choice[j], e, bc, bi)) {
        bc = choice[j];
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float oc = __shfl_xor(bc, off);
      const int oi = __shfl_xor(bi, off);
      if (better(oc, oi, bc, bi)) {
        bc = oc;
        bi = oi;
      }
    }
    const int jj = bi >> 6;
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < R; ++j) mine = j == jj ? val[j] : mine;
    const float v = __shfl(mine, bi & 63);
    if ((bi & 63) == lane) taken |= 1u << jj;
    if (lane == kk) {
      my_val = v;
      my_id = bi;
    }
  }
  // weights, summed in selection order as the crate does
  const int k = r.top_k;
  float w;
  if (sig) {
    if (r.normalize && k > 1) {
      float s = 0.0f;
      for (int kk = 0; kk < k; ++kk) s += __shfl(my_val, kk);
      s += 1.0e-20f;
      w = my_val / s * r.scale;
    } else {
      w = my_val * r.scale;
    }
  } else {
    const float mx = __shfl(my_val, 0);
    const float ex = expf(my_val - mx);
    float s = 0.0f;
    for (int kk = 0; kk < k; ++kk) s += __shfl(ex, kk);
    w = ex / s;
  }
  if (lane < k) {
    ids[(size_t)t * k + lane] = my_id;
    wout[(size_t)t * k + lane] = w;
  }
}

hipError_t moe_route(const MoeRouting &r, int T, int E, int32_t *ids, float *w, hipStream_t st) {
  const int waves = 4;
  hipLaunchKernelGGL(moe_route_kernel, dim3((T + waves - 1) / waves), dim3(64 * waves), 0, st, r,
                     T, E, ids, w);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// grouping: one workgroup
// ---------------------------------------------------------------------------

// Grouping runs in one wave: counts by LDS atomics, then each lane scans a
// contiguous run of experts and a wave prefix joins the runs.
CAI4_DEV int wave_exclusive_scan(int x, int *total) {
  const int lane = threadIdx.x & 63;
  int inc = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(inc, d);
    if (lane >= d) inc += y;
  }
  *total = __shfl(inc, 63);
  return inc - x;
}

__global__ __launch_bounds__(64) void moe_group_kernel(const int32_t *ids, const float *w,
                                                       float thr, int T, int E, int k, int C,
                                                       int max_chunks, int32_t *pos,
                                                       int32_t *row_map, SkinnyChunk *chunks,
                                                       int32_t *counts) {
  __shared__ int cnt[kMoeMaxExperts], off[kMoeMaxExperts], choff[kMoeMaxExperts];
  const int lane = threadIdx.x;
  const int n = T * k;
  for (int e = lane; e < E; e += 64) cnt[e] = 0;
  __syncthreads();
  // rank of each valid assignment within its expert (kept in pos for now)
  for (int i = lane; i < n; i += 64) {
    const int e = ids[i];
    const bool ok = !(w[i] < thr) && e >= 0 && e < E;  // runner.rs:1811: skip w < threshold
    pos[i] = ok ? atomicAdd(&cnt[e], 1) : -1;
  }
  __syncthreads();
  const int per = (E + 63) >> 6, e0 = lane * per, e1 = min(E, e0 + per);
  int rows = 0, chs = 0;
  for (int e = e0; e < e1; ++e) {
    rows += cnt[e];
    chs += (cnt[e] + C - 1) / C;
  }
  int total, total_chunks;
  int ro = wave_exclusive_scan(rows, &total), co = wave_exclusive_scan(chs, &total_chunks);
  for (int e = e0; e < e1; ++e) {
    off[e] = ro;
    choff[e] = co;
    const int c = cnt[e];
    for (int q = 0; q * C < c; ++q) {
      const int left = c - q * C;
      chunks[co + q] = SkinnyChunk{e, ro + q * C, left < C ? left : C, 0};
    }
    ro += c;
    co += (c + C - 1) / C;
  }
  __syncthreads();
  for (int i = lane; i < n; i += 64) {
    const int rk = pos[i];
    if (rk >= 0) {
      const int p = off[ids[i]] + rk;
      pos[i] = p;
      row_map[p] = i / k;
    }
  }
  for (int j = total_chunks + lane; j < max_chunks; j += 64) chunks[j] = SkinnyChunk{0, 0, 0, 0};
  if (lane == 0) {
    counts[0] = total;
    counts[1] = total_chunks;
  }
}

hipError_t moe_group(const int32_t *ids, const float *w, float threshold, int T, int E,
                     int top_k, int chunk_rows, int max_chunks, int32_t *pos, int32_t *row_map,
                     SkinnyChunk *chunks, int32_t *counts, hipStream_t st) {
  hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(64), 0, st, ids, w, threshold, T, E,
                     top_k, chunk_rows, max_chunks, pos, row_map, chunks, counts);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// gather (bf16 rows in grouped order) and combine
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void moe_gather_kernel(const float *x, const int32_t *row_map,
                                                         const int32_t *counts, int H,
                                                         uint16_t *xg) {
  const int p = blockIdx.y;
  if (p >= counts[0]) return;
  const int j = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (j >= H) return;
  const int t = row_map[p];
  const f32x4_t *src = reinterpret_cast<const f32x4_t *>(x + (size_t)t * H + j);
  const f32x4_t a = src[0], b = src[1];
  u32x4_t o;
  o.x = f32_to_bf16_rne(a.x) | (f32_to_bf16_rne(a.y) << 16);
  o.y = f32_to_bf16_rne(a.z) | (f32_to_bf16_rne(a.w) << 16);
  o.z = f32_to_bf16_rne(b.x) | (f32_to_bf16_rne(b.y) << 16);
  o.w = f32_to_bf16_rne(b.z) | (f32_to_bf16_rne(b.w) << 16);
  *reinterpret_cast<u32x4_t *>(xg + (size_t)p * H + j) = o;
}

hipError_t moe_gather(const float *x, const int32_t *row_map, const int32_t *counts, int T,
                      int H, int top_k, uint16_t *xg, hipStream_t st) {
  const int per_block = 256 * 8;
  hipLaunchKernelGGL(moe_gather_kernel, dim3((H + per_block - 1) / per_block, T * top_k),
                     dim3(256), 0, st, x, row_map, counts, H, xg);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void moe_combine_kernel(const float *residual,
                                                          const float *shared,
                                                          const uint16_t *y,
                                                          const int32_t *pos, const float *w,
                                                          int H, int k, float *out) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  const int j = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (j >= H) return;
  const size_t o = (size_t)t * H + j;
  f32x4_t h = {0.f, 0.f, 0.f, 0.f};
  if (residual) h = *reinterpret_cast<const f32x4_t *>(residual + o);
  if (shared) h += *reinterpret_cast<const f32x4_t *>(shared + o);
  f32x4_t moe = {0.f, 0.f, 0.f, 0.f};
  for (int kk = 0; kk < k; ++kk) {
    const int p = pos[(size_t)t * k + kk];
    if (p < 0) continue;
    const float wk = w[(size_t)t * k + kk];
    const u32x2_t yy = *reinterpret_cast<const u32x2_t *>(y + (size_t)p * H + j);
    const f32x4_t yf = {bf16_to_f32(yy.x & 0xFFFFu), bf16_to_f32(yy.x >> 16),
                        bf16_to_f32(yy.y & 0xFFFFu), bf16_to_f32(yy.y >> 16)};
    moe += wk * yf;
  }
  *reinterpret_cast<f32x4_t *>(out + o) = h + moe;
}

hipError_t moe_combine(const float *residual, const float *shared, const uint16_t *y,
                       const int32_t *pos, const float *w, int T, int H, int top_k, float *out,
                       hipStream_t st) {
  const int per_block = 256 * 4;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((H + per_block - 1) / per_block, T), dim3(256), 0,
                     st, residual, shared, y, pos, w, H, top_k, out);
  return hipGetLastError();
}

}  // namespace cai4
