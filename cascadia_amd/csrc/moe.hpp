// moe.hpp -- sparse-MoE expert path of one layer on one GPU.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "skinny.hpp"

namespace cai4 {

enum RouteMode { ROUTE_IDS = 0, ROUTE_SIGMOID_BIAS = 1, ROUTE_SOFTMAX_TOPK = 2 };

struct MoeRouting {
  int mode, top_k;
  const float *logits;  // [T, E] (modes 1, 2)
  const float *bias;    // [E] or null (mode 1)
  float scale;          // mode 1: scaling of the selected weights
  int normalize;        // mode 1: renormalise the top-k
  const int32_t *ids;   // [T, top_k] (mode 0)
  const float *weights; // [T, top_k] (mode 0)
  float threshold;      // slots with w < threshold are skipped
};

constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopK = 16;
constexpr int kMoePrepMaxTokens = 8;  // batches the one-workgroup prep kernel takes

// Device workspace regions of one moe_forward call (byte offsets).
struct MoeWorkspace {
  size_t ids, weights, pos, row_map, chunks, counts, hi, lo, y, shared, part, shared_ws, total;
  int chunk_rows, max_chunks;
};

MoeWorkspace moe_workspace(int T, int H, int I, int E, int top_k, int chunk_rows,
                           size_t part_bytes, size_t shared_bytes, size_t shared_ws_bytes);

// Rows per grouped chunk for T tokens, no expert receiving more than
// per_expert_max of them (T when routing picks distinct experts per token).
int moe_chunk_rows(int T, int per_expert_max);
// Upper bound on grouped chunks.
int moe_max_chunks(int T, int E, int top_k, int chunk_rows);

hipError_t moe_route(const MoeRouting &r, int T, int E, int32_t *ids, float *w,
                     hipStream_t st);
// T <= kMoePrepMaxTokens: routing (or the given ids) and grouping in one
// launch; the results as moe_route + moe_group leave them.
hipError_t moe_prep(const MoeRouting &r, int T, int E, int top_k, int chunk_rows, int max_chunks,
                    int32_t *ids, float *w, int32_t *pos, int32_t *row_map, SkinnyChunk *chunks,
                    int32_t *counts, hipStream_t st);
hipError_t moe_group(const int32_t *ids, const float *w, float threshold, int T, int E,
                     int top_k, int chunk_rows, int max_chunks, int32_t *pos, int32_t *row_map,
                     SkinnyChunk *chunks, int32_t *counts, hipStream_t st);
hipError_t moe_combine(const float *residual, const float *shared, const uint16_t *y,
                       const int32_t *pos, const float *w, int T, int H, int top_k, float *out,
                       hipStream_t st);
// One token: out = (residual + shared) + moe (residual / shared may be null).
hipError_t moe_finish(const float *residual, const float *shared, const float *moe, int H,
                      float *out, hipStream_t st);

}  // namespace cai4
