// skinny.hpp -- host-visible interface of the decode-regime INT4 GEMM.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cai4 {

// Epilogues: f32 out, bf16 (RNE) out, SwiGLU of a gate/up tile pair as f32,
// or as the two bf16 planes (hi, lo) that A_HILO consumes; a gate/up pair's
// two rows as f32, not combined (out = gate, out2 = up: the skinny kernel).
enum Epilogue { EPI_F32 = 0, EPI_SWIGLU = 1, EPI_BF16 = 2, EPI_SWIGLU_HILO = 3, EPI_PAIR_F32 = 4 };

__host__ __device__ inline bool epi_pair(int epi) {
  return epi == EPI_SWIGLU || epi == EPI_SWIGLU_HILO || epi == EPI_PAIR_F32;
}

// Activation modes: bf16; f32 (split into hi/lo bf16 planes while staged);
// precomputed hi/lo bf16 planes (x = hi plane, x2 = lo plane); f32 rows
// gathered through a row map (grouped row r is x row row_map[r]) and rounded
// to bf16 (RNE) while staged -- one bf16 plane, like A_BF16.
enum AMode { A_BF16 = 0, A_XF32 = 1, A_HILO = 2, A_GATHER = 3 };

// Modes whose staged activations are one bf16 plane (16 token slots per MFMA tile).
__host__ __device__ inline bool amode_single_plane(int amode) {
  return amode == A_BF16 || amode == A_GATHER;
}

// Grouped mode: one row chunk of one expert per workgroup row (blockIdx.y).
// Weights/scales of expert e are at w0/w1/s0/s1 + e * expert_stride; a chunk
// with count <= 0 is empty (its workgroups exit at once).
struct SkinnyChunk {
  int expert, row0, count, pad;
};

struct SkinnyArgs {
  const uint8_t *w0;  // packed weights (gate for the SwiGLU epilogues)
  const uint8_t *w1;  // up matrix (SwiGLU epilogues only)
  const uint8_t *s0;  // scales u16
  const uint8_t *s1;
  const void *x;      // activations [M, ldx]: bf16 bits, f32, or the hi plane
  const void *x2;     // A_HILO: the lo plane [M, ldx]
  void *out;          // [M, ldo]: f32, bf16 bits, or the hi plane (EPI_SWIGLU_HILO)
  void *out2;         // EPI_SWIGLU_HILO: the lo plane; EPI_PAIR_F32: up
  void *partials;     // split-K partial sums (SkinnyPlan::partial_bytes), or null
  const SkinnyChunk *chunks;  // grouped mode: [max_chunks] (device), else null
  const int32_t *row_map;     // A_GATHER: x row of each grouped row [M] (device)
  int x_rows;                 // A_GATHER: rows of x (the descriptor range)
  size_t expert_stride;       // grouped mode: bytes between experts' weights
  int N, K, G, M, ldx, ldo, sdt;
  int glog2;  // log2(G) when G is a power of two, else -1
  int tiled;  // weights/scales in the MFMA-tiled device layout (layout.hip)
  // The one-token GEMV's sparse-mask epilogue: y (the gate) goes to out as
  // f32 -- with a gate/up pair (EPI_SWIGLU) the up row to out2 as f32, not
  // combined -- and each 16-row tile writes slots[tile] = max |silu(y)| over
  // its rows (bits; NaN counts as 0) | (any thr[row] > 0) << 31; silu_slot
  // 1 = the plain SiLU, 2 = the stable one; thr may be null.  Null slots: the
  // ordinary epilogue.
  uint32_t *slots;
  const float *thr;
  int silu_slot;
};

// Launch plan.  A workgroup has rw x kw waves: rw row groups (each nt weight
// tiles of 16 rows) share the activations staged in LDS; kw waves split the
// workgroup's k-range.  ksplit > 1 splits K across workgroups, whose partial
// sums a second kernel adds in a fixed order.
struct SkinnyPlan {
  int nt, mt, rw, kw, ksplit, kper, kslice, row_blocks, m_chunks;
  int act_rows, act_stride, scale_off;
  size_t lds_bytes, partial_bytes;
};

// Device properties the planner uses (the library caches them per device).
struct SkinnyDevice {
  int num_cus;
  size_t max_lds;  // LDS bytes a workgroup may use
};

SkinnyPlan skinny_plan(int N, int K, int G, int M, int amode, int epi, const SkinnyDevice &d);
// Grouped mode: chunks of at most chunk_rows rows, max_chunks workgroup rows.
SkinnyPlan skinny_plan_grouped(int N, int K, int G, int chunk_rows, int max_chunks, int amode,
                               int epi, const SkinnyDevice &d);
hipError_t skinny_launch(const SkinnyArgs &a, const SkinnyPlan &p, int amode, int epi,
                         hipStream_t st);

}  // namespace cai4
