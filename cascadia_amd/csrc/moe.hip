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
#include <stdlib.h>

#include "int4_common.hpp"
#include "moe.hpp"
#include "moe_route.hpp"
#include "tuning.hpp"

namespace cai4 {

namespace {
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

// Rows per chunk: the grouped GEMMs stage (and compute for) that many rows per
// chunk, and every chunk streams its expert's weights.  Measured on configs 3
// and 4: 16 rows beat 32 at 256 tokens (config 3 598 -> 432 us per layer: the
// 32-row down ran 8 waves per CU); 8 rows beat 16 at 32 tokens on config 3
// (-6 %) but lost 16 % at 64 tokens on config 4, whose skewed routing gives
// its hot experts many rows -- so 16 from 9 tokens up.  With at most two rows
// per expert and tiled experts (gemv_rows), one-row chunks on the grouped
// one-token GEMV: two routed tokens, config 3 40.1 -> 37.3 us per layer,
// config 4 (Zipf-skewed routing) 101.5 -> 100.4; at four tokens skewed routing
// already lost 15 % that way (a hot expert streams once per row).
int moe_chunk_rows(int T, int per_expert_max, bool gemv_rows) {
  // override 1 .. 32 (a 32-row chunk is the most one pass of the two-plane
  // down projection holds)
  const int ev = tuning_env("CASCADIA_INT4_MOE_CHUNK_ROWS", 0);
  const int c = ev >= 1 && ev <= 32 ? ev
                : gemv_rows && per_expert_max <= 2 ? 1
                : T <= 8 ? 8 : 16;
  return per_expert_max < c ? per_expert_max : c;
}

int moe_tile_tokens() {
  const int n = tuning_env("CASCADIA_INT4_MOE_TILE_TOKENS", 0);
  return n > 0 ? n : 512;
}

int moe_tile_rows() {
  const int n = tuning_env("CASCADIA_INT4_MOE_TILE_ROWS", 0);
  return n > 0 ? n : 48;
}

int moe_max_chunks(int T, int E, int top_k, int chunk_rows) {
  // sum_e ceil(c_e / C) <= A + (n - A) / C for A active experts, largest at
  // A = min(n, E)
  const long n = (long)T * top_k, a = n < E ? n : E;
  return (int)(a + (n - a) / chunk_rows);
}

MoeWorkspace moe_workspace(int T, int H, int I, int E, int top_k, int chunk_rows,
                           size_t part_bytes, size_t shared_bytes, size_t shared_ws_bytes,
                           size_t xg_bytes, size_t seeds_x_bytes, size_t seeds_i_bytes,
                           int chunk_rows2) {
  MoeWorkspace w{};
  const size_t n = (size_t)T * top_k;
  w.chunk_rows = chunk_rows;
  w.max_chunks = moe_max_chunks(T, E, top_k, w.chunk_rows);
  w.chunk_rows2 = chunk_rows2;
  w.max_chunks2 = chunk_rows2 ? moe_max_chunks(T, E, top_k, chunk_rows2) : 0;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  // one spare row map entry, chunk and hi / lo row: a one-token layer's
  // shared expert as an always-on slot
  w.ids = take(n * 4);
  w.weights = take(n * 4);
  w.pos = take(n * 4);
  w.row_map = take((n + 1) * 4);
  w.chunks = take((size_t)(w.max_chunks + 1) * sizeof(SkinnyChunk));
  w.counts = take(16);
  w.hi = take((n + 1) * I * 2);
  w.lo = take((n + 1) * I * 2);
  // [n, H] bf16 expert outputs; a one-token layer with a shared expert also
  // keeps its [H] f32 routed sum here, which is larger when top_k is 1
  w.y = take(n * H * 2 > (size_t)H * 4 ? n * H * 2 : (size_t)H * 4);
  w.shared = take(shared_bytes);
  w.part = take(part_bytes);
  w.shared_ws = take(shared_ws_bytes);
  w.xg = take(xg_bytes);
  w.seeds_x = take(seeds_x_bytes);
  w.seeds_i = take(seeds_i_bytes);
  w.chunks2 = take((size_t)w.max_chunks2 * sizeof(SkinnyChunk));
  w.total = o;
  return w;
}

// ---------------------------------------------------------------------------
// routing: one wave per token (route_token: moe_route.hpp)
// ---------------------------------------------------------------------------

template <int R>
__global__ __launch_bounds__(256) void moe_route_kernel(MoeRouting r, int T, int E, int32_t *ids,
                                                        float *wout) {
  const int lane = threadIdx.x & 63;
  // the token as a scalar: the logits' buffer descriptor must be uniform
  const int t = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= T) return;  // whole waves; no barriers in this kernel
  int id;
  float w;
  route_token<R>(r, t, E, lane, id, w);
  if (lane < r.top_k) {
    ids[(size_t)t * r.top_k + lane] = id;
    wout[(size_t)t * r.top_k + lane] = w;
  }
}

// Instantiations by registers per lane, ceil(E / 64) rounded up to a power
// of two: the loops over a lane's experts are unrolled.
#define CAI4_MOE_DISPATCH(E, CALL)           \
  do {                                       \
    const int nj_ = ((E) + 63) / 64;         \
    if (nj_ <= 1) { constexpr int R = 1; CALL; }        \
    else if (nj_ <= 2) { constexpr int R = 2; CALL; }   \
    else if (nj_ <= 4) { constexpr int R = 4; CALL; }   \
    else if (nj_ <= 8) { constexpr int R = 8; CALL; }   \
    else { constexpr int R = 16; CALL; }                \
  } while (0)

hipError_t moe_route(const MoeRouting &r, int T, int E, int32_t *ids, float *w, hipStream_t st) {
  const int waves = 4;
  CAI4_MOE_DISPATCH(E, hipLaunchKernelGGL(moe_route_kernel<R>, dim3((T + waves - 1) / waves),
                                          dim3(64 * waves), 0, st, r, T, E, ids, w));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// grouping: one workgroup
// ---------------------------------------------------------------------------

// Exclusive prefix sum over the 64 lanes of a wave, by DPP: Kogge-Stone
// within each 16-lane row (row_shr 1, 2, 4, 8), then the row totals carried
// by row_bcast 15 and 31.  *total gets the sum of all lanes.
template <int CTRL, int ROWS>
CAI4_DEV int dpp_add_in(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, true);
}
CAI4_DEV int wave_exclusive_scan(int x, int *total) {
  int v = x;
  v = dpp_add_in<0x111, 0xF>(v);  // row_shr 1
  v = dpp_add_in<0x112, 0xF>(v);  // row_shr 2
  v = dpp_add_in<0x114, 0xF>(v);  // row_shr 4
  v = dpp_add_in<0x118, 0xF>(v);  // row_shr 8
  v = dpp_add_in<0x142, 0xA>(v);  // row_bcast 15 into rows 1, 3
  v = dpp_add_in<0x143, 0xC>(v);  // row_bcast 31 into rows 2, 3
  *total = __builtin_amdgcn_readlane(v, 63);
  return v - x;
}

// Grouping of the n = T k assignments by expert, by every thread of the
// workgroup: counts by LDS atomics (rank of each valid assignment within its
// expert in rank[]), then wave 0 scans contiguous runs of experts per lane and
// writes the chunks, then every thread places its assignments.  ids/w may be
// global or LDS.  On return (after a barrier) rowmap[p] is the token of
// grouped row p, and *total / *nchunks hold the counts.
// Barrier for LDS data only: the global stores of these kernels are read by
// later launches, never by another thread of the same workgroup, so they need
// not be waited for (__syncthreads would wait for every store to complete).
CAI4_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ceil(a / C) for 0 <= a < 2^20 and 1 <= C <= 256: a float estimate (off by
// at most one), then one correction step each way (exact; no integer division).
CAI4_DEV int ceil_div_small(int a, int C, float invC) {
  const int n = a + C - 1;
  int q = (int)((float)n * invC);
  if (q * C > n) --q;
  if ((q + 1) * C <= n) ++q;
  return q;
}

struct GroupLds {
  int cnt[kMoeMaxExperts], off[kMoeMaxExperts];
  int total, nchunks;
};

// Two tables (chunks2 not null): experts with at least hot_min rows are cut
// into chunks of C rows in `chunks`, the others into chunks of C2 rows in
// `chunks2`; counts[1] / counts[2] get the two chunk counts.
template <int PMAX>  // PMAX >= ceil(E / 64)
CAI4_DEV void group_assignments(const int32_t *ids, const float *w, float thr, int T, int E,
                                int k, int C, int max_chunks, int *rank, GroupLds &g,
                                int32_t *pos, int *rowmap, SkinnyChunk *chunks,
                                int32_t *counts, int C2 = 0, int hot_min = 0,
                                SkinnyChunk *chunks2 = nullptr, int max_chunks2 = 0) {
  const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63;
  const int n = T * k;
  for (int e = tid; e < E; e += nth) g.cnt[e] = 0;
  lds_barrier();
  for (int i = tid; i < n; i += nth) {
    const int e = ids[i];
    const bool ok = !(w[i] < thr) && e >= 0 && e < E;  // runner.rs:1811: skip w < threshold
    rank[i] = ok ? atomicAdd(&g.cnt[e], 1) : -1;
  }
  lds_barrier();
  if (tid < 64) {
    // lane l scans experts l * per .. l * per + per - 1 (all its counts read
    // at once: the loop carries no LDS latency)
    const int per = (E + 63) >> 6, e0 = lane * per;
    const float invC = 1.0f / (float)C, invC2 = chunks2 ? 1.0f / (float)C2 : 0.f;
    int c[PMAX], nc[PMAX], nc2[PMAX];
    int rows = 0, chs = 0, chs2 = 0;
#pragma unroll
    for (int q = 0; q < PMAX; ++q) {
      c[q] = q < per && e0 + q < E ? g.cnt[e0 + q] : 0;
      const bool hot = !chunks2 || c[q] >= hot_min;
      nc[q] = hot ? ceil_div_small(c[q], C, invC) : 0;
      nc2[q] = hot ? 0 : ceil_div_small(c[q], C2, invC2);
      rows += c[q];
      chs += nc[q];
      chs2 += nc2[q];
    }
    int total, total_chunks, total_chunks2;
    int ro = wave_exclusive_scan(rows, &total), co = wave_exclusive_scan(chs, &total_chunks);
    int co2 = wave_exclusive_scan(chs2, &total_chunks2);
#pragma unroll
    for (int q = 0; q < PMAX; ++q) {
      if (q < per && e0 + q < E) {
        const int e = e0 + q;
        g.off[e] = ro;
        for (int h = 0; h < nc[q]; ++h) {
          const int left = c[q] - h * C;
          chunks[co + h] = SkinnyChunk{e, ro + h * C, left < C ? left : C, 0};
        }
        for (int h = 0; h < nc2[q]; ++h) {
          const int left = c[q] - h * C2;
          chunks2[co2 + h] = SkinnyChunk{e, ro + h * C2, left < C2 ? left : C2, 0};
        }
      }
      ro += c[q];
      co += nc[q];
      co2 += nc2[q];
    }
    for (int j = total_chunks + lane; j < max_chunks; j += 64) chunks[j] = SkinnyChunk{0, 0, 0, 0};
    if (chunks2)
      for (int j = total_chunks2 + lane; j < max_chunks2; j += 64)
        chunks2[j] = SkinnyChunk{0, 0, 0, 0};
    if (lane == 0) {
      g.total = total;
      g.nchunks = total_chunks;
      counts[0] = total;
      counts[1] = total_chunks;
      counts[2] = total_chunks2;
    }
  }
  lds_barrier();
  for (int i = tid; i < n; i += nth) {
    const int rk = rank[i];
    int p = -1;
    if (rk >= 0) {
      p = g.off[ids[i]] + rk;
      rowmap[p] = i / k;
    }
    pos[i] = p;
  }
  lds_barrier();
}

// One workgroup of 1024 threads: each thread's assignments are a couple of
// independent loads and LDS atomics (one wave took 26 us at 2048 assignments,
// its loop of dependent global loads and atomics being latency-bound).
template <int R>
__global__ __launch_bounds__(1024) void moe_group_kernel(const int32_t *ids, const float *w,
                                                       float thr, int T, int E, int k, int C,
                                                       int max_chunks, int32_t *pos,
                                                       int32_t *row_map, SkinnyChunk *chunks,
                                                       int32_t *counts, int C2, int hot_min,
                                                       SkinnyChunk *chunks2, int max_chunks2) {
  __shared__ GroupLds g;
  // pos doubles as the rank array: each slot is read before it is written
  group_assignments<R>(ids, w, thr, T, E, k, C, max_chunks, pos, g, pos, row_map, chunks,
                       counts, C2, hot_min, chunks2, max_chunks2);
}

hipError_t moe_group(const int32_t *ids, const float *w, float threshold, int T, int E,
                     int top_k, int chunk_rows, int max_chunks, int32_t *pos, int32_t *row_map,
                     SkinnyChunk *chunks, int32_t *counts, hipStream_t st, int chunk_rows2,
                     int hot_min, SkinnyChunk *chunks2, int max_chunks2) {
  CAI4_MOE_DISPATCH(E, hipLaunchKernelGGL(moe_group_kernel<R>, dim3(1), dim3(1024), 0, st, ids, w,
                                          threshold, T, E, top_k, chunk_rows, max_chunks, pos,
                                          row_map, chunks, counts, chunk_rows2, hot_min, chunks2,
                                          max_chunks2));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decode batches: routing and grouping in one workgroup
// ---------------------------------------------------------------------------

// T <= kMoePrepMaxTokens: wave w routes token w (or copies the given ids),
// and the selections stay in LDS for the grouping: one launch instead of two
// dependent ones.
template <int R>
__global__ __launch_bounds__(512) void moe_prep_kernel(MoeRouting r, int T, int E, int k, int C,
                                                        int max_chunks, int32_t *ids, float *wts,
                                                        int32_t *pos, int32_t *row_map,
                                                        SkinnyChunk *chunks, int32_t *counts) {
  constexpr int NMAX = kMoePrepMaxTokens * kMoeMaxTopK;
  __shared__ int s_ids[NMAX], s_rank[NMAX];
  __shared__ float s_w[NMAX];
  __shared__ GroupLds g;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int t = wave; t < T; t += nw) {
    int id = 0;
    float w = 0.f;
    if (r.mode == ROUTE_IDS) {
      if (lane < k) {
        id = r.ids[(size_t)t * k + lane];
        w = r.weights[(size_t)t * k + lane];
      }
    } else {
      route_token<R>(r, t, E, lane, id, w);
    }
    if (lane < k) {
      s_ids[t * k + lane] = id;
      s_w[t * k + lane] = w;
      ids[(size_t)t * k + lane] = id;
      wts[(size_t)t * k + lane] = w;
    }
  }
  lds_barrier();
  group_assignments<R>(s_ids, s_w, r.threshold, T, E, k, C, max_chunks, s_rank, g, pos, row_map,
                       chunks, counts);
}

hipError_t moe_prep(const MoeRouting &r, int T, int E, int top_k, int chunk_rows, int max_chunks,
                    int32_t *ids, float *w, int32_t *pos, int32_t *row_map, SkinnyChunk *chunks,
                    int32_t *counts, hipStream_t st) {
  CAI4_MOE_DISPATCH(E, hipLaunchKernelGGL(moe_prep_kernel<R>, dim3(1), dim3(512), 0, st, r, T, E,
                                          top_k, chunk_rows, max_chunks, ids, w, pos, row_map,
                                          chunks, counts));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// combine
// ---------------------------------------------------------------------------

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
  // all slot loads first (k <= kMoeMaxTopK), then the sum in slot order
  int ps[kMoeMaxTopK];
  float ws[kMoeMaxTopK];
#pragma unroll
  for (int kk = 0; kk < kMoeMaxTopK; ++kk) {
    ps[kk] = kk < k ? pos[(size_t)t * k + kk] : -1;
    ws[kk] = kk < k ? w[(size_t)t * k + kk] : 0.f;
  }
  u32x2_t yy[kMoeMaxTopK];
#pragma unroll
  for (int kk = 0; kk < kMoeMaxTopK; ++kk)
    if (ps[kk] >= 0) yy[kk] = *reinterpret_cast<const u32x2_t *>(y + (size_t)ps[kk] * H + j);
  f32x4_t moe = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < kMoeMaxTopK; ++kk) {
    if (ps[kk] < 0) continue;
    const f32x4_t yf = {bf16_to_f32(yy[kk].x & 0xFFFFu), bf16_to_f32(yy[kk].x >> 16),
                        bf16_to_f32(yy[kk].y & 0xFFFFu), bf16_to_f32(yy[kk].y >> 16)};
    moe += ws[kk] * yf;
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

// out = (residual + shared) + moe, per element: the combine's last two adds
// when the weighted expert sum `moe` came from another kernel.
__global__ __launch_bounds__(256) void moe_finish_kernel(const float *residual,
                                                         const float *shared, const float *moe,
                                                         int H, float *out) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= H) return;
  float h = residual ? residual[j] : 0.f;
  if (shared) h = __fadd_rn(h, shared[j]);
  out[j] = __fadd_rn(h, moe[j]);
}

hipError_t moe_finish(const float *residual, const float *shared, const float *moe, int H,
                      float *out, hipStream_t st) {
  hipLaunchKernelGGL(moe_finish_kernel, dim3((H + 255) / 256), dim3(256), 0, st, residual, shared,
                     moe, H, out);
  return hipGetLastError();
}

}  // namespace cai4
