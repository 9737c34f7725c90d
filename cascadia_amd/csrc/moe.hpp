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
// xg / seeds_x / seeds_i: the MFMA-tile path's gathered bf16 rows and seeds
// (sizes 0 when unused).
// chunks2 / max_chunks2 / chunk_rows2: the second table of the hybrid path
// (experts with few rows, on the skinny kernels).
struct MoeWorkspace {
  size_t ids, weights, pos, row_map, chunks, counts, hi, lo, y, shared, part, shared_ws, xg,
      seeds_x, seeds_i, chunks2, total;
  int chunk_rows, max_chunks, chunk_rows2, max_chunks2;
};

MoeWorkspace moe_workspace(int T, int H, int I, int E, int top_k, int chunk_rows,
                           size_t part_bytes, size_t shared_bytes, size_t shared_ws_bytes,
                           size_t xg_bytes = 0, size_t seeds_x_bytes = 0,
                           size_t seeds_i_bytes = 0, int chunk_rows2 = 0);

// Tokens from which a layer runs on the MFMA-tile GEMMs (grouped.hip): experts
// with at least moe_tile_rows() rows in 128-row chunks over gathered bf16 rows,
// the others on the skinny kernels.  CASCADIA_INT4_MOE_TILE_TOKENS and
// CASCADIA_INT4_MOE_TILE_ROWS override.
int moe_tile_tokens();
int moe_tile_rows();

// Rows per grouped chunk for T tokens, no expert receiving more than
// per_expert_max of them (T when routing picks distinct experts per token).
// gemv_rows: tiled experts (one-row chunks can run on the one-token GEMV).
int moe_chunk_rows(int T, int per_expert_max, bool gemv_rows = false);
// Upper bound on grouped chunks.
int moe_max_chunks(int T, int E, int top_k, int chunk_rows);

hipError_t moe_route(const MoeRouting &r, int T, int E, int32_t *ids, float *w,
                     hipStream_t st);
// T <= kMoePrepMaxTokens: routing (or the given ids) and grouping in one
// launch; the results as moe_route + moe_group leave them.
hipError_t moe_prep(const MoeRouting &r, int T, int E, int top_k, int chunk_rows, int max_chunks,
                    int32_t *ids, float *w, int32_t *pos, int32_t *row_map, SkinnyChunk *chunks,
                    int32_t *counts, hipStream_t st);
// With chunks2: experts holding at least hot_min rows are cut into chunks of
// chunk_rows rows (chunks), the others into chunks of chunk_rows2 (chunks2).
hipError_t moe_group(const int32_t *ids, const float *w, float threshold, int T, int E,
                     int top_k, int chunk_rows, int max_chunks, int32_t *pos, int32_t *row_map,
                     SkinnyChunk *chunks, int32_t *counts, hipStream_t st, int chunk_rows2 = 0,
                     int hot_min = 0, SkinnyChunk *chunks2 = nullptr, int max_chunks2 = 0);
hipError_t moe_combine(const float *residual, const float *shared, const uint16_t *y,
                       const int32_t *pos, const float *w, int T, int H, int top_k, float *out,
                       hipStream_t st);
// One token: out = (residual + shared) + moe (residual / shared may be null).
hipError_t moe_finish(const float *residual, const float *shared, const float *moe, int H,
                      float *out, hipStream_t st);

}  // namespace cai4
