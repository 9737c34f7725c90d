// grouped.hpp -- INT4 weight-only GEMM in MFMA tiles of up to 128 rows, over
// one matrix (dense prefill) or over the row groups of many experts in one
// launch (MoE layers with many tokens per expert).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "skinny.hpp"

namespace cai4 {

// Output of a GEMM: f32, bf16 (RNE), or -- for a gate/up pair -- SwiGLU as the
// two bf16 planes hi = trunc(h), lo = RNE(h - hi) of h = silu(gate) * up.
enum GgEpi { GG_F32 = 0, GG_BF16 = 1, GG_SWIGLU_HILO = 2 };

struct GgArgs {
  // weights: gate (or the only matrix) w0 / s0, up w1 / s1 (SwiGLU); MFMA-tiled;
  // expert e's at + e * estride (grouped mode)
  const uint8_t *w0, *s0, *w1, *s1;
  size_t estride;
  const uint16_t *x;   // A: bf16 [rows, K] (the hi plane with hilo)
  const uint16_t *x2;  // hilo: the lo plane
  const float *seeds;  // [K / gw][rows_pad]: -136 * sum of A over each group of gw columns
  void *y, *y2;        // [rows, ldy]: f32 / bf16, or the hi / lo planes (SwiGLU)
  const SkinnyChunk *tiles;  // grouped: one (expert, row0, count) per workgroup row; null: dense
  int tile_split;  // grouped: workgroup rows per table entry (the entry's rows in BM parts)
  int M;         // dense: rows of A; grouped: rows addressable in A / seeds / y
  int N, K, G, sdt, ldy, rows_pad;
  int hilo;      // A has two bf16 planes (x + x2)
  int epi;       // GgEpi
  float *part;   // dense split-K partials [ksplit][M][N] (f32), or null
  int kper;      // k-blocks per K slice (blockIdx.z)
  // SwiGLU only, or null: the seeds of the hi / lo planes the epilogue writes,
  // for a GEMM that takes them as A: [N / seeds_gw][rows_pad], -136 * the sum
  // of hi + lo over each group of seeds_gw output columns (32, 64 or 128)
  float *seeds_out;
  int seeds_gw, seeds_rp;  // group width, row stride of seeds_out
  // grouped, one bf16 plane only, or null: A row r of the table is x row
  // row_map[r] (x: [x_rows, K], seeds [K / gw][rows_pad] per x row), so the
  // rows need no gathered copy
  const int32_t *row_map;
  int x_rows;
};

// Columns per seed group: min(G, 128).
inline int gg_group_width(int G) { return G >= 128 ? 128 : G; }

// Whether the kernel handles this shape: MFMA-tiled weights, K a multiple of
// 128, G 32, 64 or a multiple of 128.
bool gg_supported(int K, int G, int tiled);

// Seeds (and converted activations) of A, one wave per row:
//   mode 0: bf16 rows x [rows, K] -> seeds;
//   mode 1: bf16 hi/lo planes x, x2 -> seeds of hi + lo;
//   mode 2: f32 rows src gathered through row_map (row r = src row row_map[r];
//           src row r when row_map is null) -> bf16 (RNE) rows into out + seeds;
//   mode 3: f32 rows src -> hi/lo planes out / out2 + seeds.
// rows_dev (device, may be null): the row count, when only the device knows
// it (rows is then an upper bound).
hipError_t gg_prep(int mode, const void *src, const void *src2, const int32_t *row_map,
                   uint16_t *out, uint16_t *out2, float *seeds, int rows, int rows_pad, int K,
                   int G, const int32_t *rows_dev, hipStream_t st);

// Rows of seeds to allocate for `rows` A rows.
int gg_rows_pad(int rows);

// Rows per grouped table entry (the grouping's chunk_rows).
constexpr int kGgChunkRows = 128;

// Activation forms of the dense GEMM: bf16 rows a.x; f32 rows a.x (split into
// hi / lo planes in the workspace); hi / lo planes a.x / a.x2.
enum GgAMode { GG_A_BF16 = 0, GG_A_F32 = 1, GG_A_PLANES = 2 };

// Dense: workspace bytes (seeds, split planes, split-K partials) and the
// launches (gg_prep, the GEMM, the split-K reduce).
size_t gg_dense_workspace(int M, int N, int K, int G, int amode, int epi, int num_cus);
hipError_t gg_dense(GgArgs a, int amode, void *ws, int num_cus, hipStream_t st);

// Grouped: tiles = max_tiles entries (count 0: empty) of at most
// 128 rows; a.seeds over a.rows_pad rows made by gg_prep.
hipError_t gg_grouped(const GgArgs &a, int max_tiles, hipStream_t st);

}  // namespace cai4
