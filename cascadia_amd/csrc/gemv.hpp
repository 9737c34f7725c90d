// gemv.hpp -- one-token INT4 GEMV over MFMA-tiled weights (decode shape).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

#include "moe.hpp"
#include "skinny.hpp"

namespace cai4 {

// kw waves per workgroup (one 16-row tile or gate/up tile pair), kpw k-blocks each.
struct GemvPlan {
  int kw, kpw;
};

// MFMA-tiled weights, G a multiple of 128 dividing K; epilogues f32, bf16, SwiGLU
// (f32 or hi/lo); the plan's LDS within one CU's.  Dense: M = 1, activation
// modes A_BF16 / A_XF32 / A_HILO.  Grouped (a.chunks): chunks of one row
// (chunk_rows = 1), max_chunks of them, modes A_GATHER / A_HILO.
bool gemv_supported(const SkinnyArgs &a, int amode, int epi, int num_cus, int chunk_rows = 0,
                    int max_chunks = 0);
// max_kpw: most k-blocks per wave the instantiations cover (16; 8 for scale
// groups of 32 or 64 columns, gemv_max_kpw).
GemvPlan gemv_plan(int N, int K, int num_cus, int max_kpw = 16);
inline int gemv_max_kpw(int gpb) { return gpb > 1 ? 8 : 16; }
// The shared expert of one MoE token as an always-on slot of a grouped launch:
// the chunk flagged pad = 1 reads its matrix w / s and writes f32 to out.
struct GemvSharedSlot {
  const uint8_t *w, *s;
  float *out;
};
hipError_t gemv_launch(const SkinnyArgs &a, int amode, int epi, int num_cus, int max_chunks,
                       hipStream_t st, const GemvSharedSlot *sh = nullptr);

// One MoE token (T = 1) over MFMA-tiled experts, in two launches: the gate/up
// of every slot (each workgroup recomputes the token's routing for up to 256
// experts, or reads the ids and weights in route -- given, or left by
// moe_route; writes ids / weights / pos and the SwiGLU hi/lo rows per slot),
// then the down projections of all slots with the weighted combine.  With
// moe_sum set the second launch writes only the weighted expert sum there (no
// residual, no shared term: moe_finish adds them); else the shared expert's
// output must be complete before it.
struct Moe1Args {
  const uint8_t *gate, *gate_s, *up, *up_s, *down, *down_s;  // expert 0's sections
  size_t expert_stride;
  const float *x;  // [H]
  MoeRouting route;
  int E, top_k;
  int32_t *ids;
  float *wts;
  int32_t *pos;
  uint16_t *hi, *lo;               // [top_k, I] each
  const float *residual, *shared;  // [H] or null
  float *out;                      // [H]
  float *moe_sum;                  // [H] or null
  SkinnyChunk *chunks;             // [top_k] one-row chunks for a grouped down launch, or null
  int32_t *row_map;                // [top_k], with chunks
  int H, I, G, sdt;
  // the shared expert (its inter size I): sh = 1 runs its gate/up as slot
  // top_k of this launch (rows hi / lo [top_k]); sh = 2 only records chunk
  // top_k (pad = 1) for the grouped down, the rows coming from another launch;
  // 0: none.  With sh, chunks / row_map hold top_k + 1 entries.
  int sh;
  const uint8_t *sh_gate, *sh_gate_s, *sh_up, *sh_up_s;
};
// Whether the gate/up launch routes in-kernel (else route must hold ids): up
// to 256 experts, 4 per lane.  (384 experts routed in every workgroup, 8 per
// lane, measured 2.6 us per layer slower on config 4 than a routing launch.)
inline bool gemv_moe1_routes(const MoeRouting &r, int E) { return r.mode != ROUTE_IDS && E <= 256; }
bool gemv_moe1_supported(int H, int I, int G, int top_k, int E, int num_cus);
// Whether the down + combine launch fits (its workgroups of top_k slots each
// cover one 16-row tile; more tiles than CUs would run in two rounds: then
// the grouped down GEMV over the chunk table and the combine kernel instead).
bool gemv_moe1_down_fused(int H, int I, int G, int top_k, int num_cus);
hipError_t gemv_moe1_gate_up(const Moe1Args &m, int num_cus, hipStream_t st);
hipError_t gemv_moe1_down(const Moe1Args &m, hipStream_t st);

}  // namespace cai4
