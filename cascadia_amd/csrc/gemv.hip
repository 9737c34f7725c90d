// gemv.hip -- INT4 GEMV for one token over MFMA-tiled weights (gfx950): the
// decode shape of configs 0 and 1 (dequant_gemv_int4, kernel.rs:31-71;
// expert_forward's gate/up and down, kernel.rs:75-136, at seq = 1).
//
// A workgroup owns one 16-row weight tile (or a gate/up tile pair) and its kw
// waves split K; each wave streams a contiguous run of k-blocks (1 KB per
// tile each in the tiled layout) and nothing else:
//   * its slice of the activations (and their per-k-block sums, the
//     zero-point seeds) goes into the wave's own LDS region once, with no
//     barrier -- no wave reads another's region;
//   * so do the slice's scales (4-byte loads);
//   * the weight fragments stream through a small register ring, the only
//     loads of the k-loop, each slot refilled before its data is decoded;
//   * the kw partial sums meet once, through LDS, in wave order.
// This keeps every wave independent until the end, as a plain streaming read
// is.  Measured on MI355X, a plain read of ~60 MB is fastest as many short
// runs (4-8 KB per wave, ~30 waves per CU): the plan aims at 28 resident waves
// per CU, and each instantiation sizes its register arrays for the k-blocks
// per wave it serves and is compiled for the waves per SIMD that plan needs
// (64-80 VGPRs) -- with arrays sized for 16 k-blocks the same plan would not
// fit and run in two rounds.
//
// Arithmetic as the skinny kernel's: weights enter the MFMA as bf16 128 + n;
// each k-block's partial is seeded with -136 * sum(x) over the block (the
// zero point), the group scale (G a multiple of 128: one per k-block) is
// applied in f32, acc += s * p.  Activation slots of the 16 x 16 MFMA tile:
// bf16 x -> every slot holds the token; f32 x or hi/lo planes -> slots 0-7 the
// hi plane, 8-15 the lo plane, added at the end.
#include "gemv.hpp"
#include "int4_common.hpp"
#include "moe.hpp"
#include "moe_route.hpp"
#include "skinny.hpp"

namespace cai4 {

namespace {

// Sum over aligned groups of 16 / GPB lanes (every lane of a group gets it).
template <int GPB>
CAI4_DEV float group_sum(float t) {
  if constexpr (GPB == 1) {
    return row16_sum(t);
  } else {
    t += dpp_f32<0xB1>(t);  // quad_perm 1,0,3,2
    t += dpp_f32<0x4E>(t);  // quad_perm 2,3,0,1
    if constexpr (GPB == 2) t += __shfl_xor(t, 4);
    return t;
  }
}

// n consecutive f32 from LDS (n * 4-byte aligned) in one read.
template <int n>
CAI4_DEV void lds_read_f32(const float *p, float *v) {
  if constexpr (n == 4) {
    const f32x4_t t = *reinterpret_cast<const f32x4_t *>(p);
    v[0] = t[0], v[1] = t[1], v[2] = t[2], v[3] = t[3];
  } else if constexpr (n == 2) {
    const float2 t = *reinterpret_cast<const float2 *>(p);
    v[0] = t.x, v[1] = t.y;
  } else {
    v[0] = p[0];
  }
}

struct GvParams {
  const uint8_t *w0, *w1, *s0, *s1;
  const void *x, *x2;
  void *out, *out2;
  int N, K, G, sdt, epi, kw, kpw;
  // grouped mode: blockIdx.y = chunk of one row of one expert (count <= 1);
  // the expert's matrices at + expert * expert_stride, the x row
  // row_map[row0] (or row0), the output row row0; ldx / ldo in elements
  const SkinnyChunk *chunks;
  const int32_t *row_map;
  size_t expert_stride;
  int ldx, ldo;
  // one MoE token (MODE 1: routed gate/up; MODE 2: down + weighted combine):
  // the routing (or given ids) over E experts, top_k slots; MODE 1 writes
  // ids / weights / pos (slot or -1 under the threshold), MODE 2 reads them
  MoeRouting route;
  int E, top_k;
  int32_t *ids;
  float *wts;
  int32_t *pos;
  const float *residual, *shared;  // MODE 2: out = (residual + shared) + sum_k w_k y_k
  int moe_partial;                 // MODE 2: out = sum_k w_k y_k only
  SkinnyChunk *chunks_out;         // MODE 1: [top_k] chunk table of one row per slot, or null
  int32_t *row_map_out;            // MODE 1: [top_k] (all token 0), or null
  // the token's shared expert as an always-on slot (sh_slot = top_k; -1: none):
  // MODE 1 workgroup row sh_slot runs its gate/up over the f32 x split into hi /
  // lo planes (routed slots round x to bf16) and records chunk sh_slot with
  // pad = 1; a grouped launch reads such a chunk's matrix at sh_w0 / sh_s0 and
  // writes its f32 output row to sh_out (no bf16 rounding)
  const uint8_t *sh_w0, *sh_s0, *sh_w1, *sh_s1;
  float *sh_out;
  int sh_slot;
  // the sparse-mask epilogue (SkinnyArgs::slots)
  uint32_t *slots;
  const float *thr;
  int silu_slot;
};

// Slot kk of the one token: its expert, weight, position (kk, or -1 when
// skipped) and, for a grouped launch after this one, its chunk of one row.
CAI4_DEV void moe1_record(const GvParams &a, int kk, int id, float w, bool keep) {
  a.ids[kk] = id;
  a.wts[kk] = w;
  a.pos[kk] = keep ? kk : -1;
  if (a.chunks_out) {
    a.chunks_out[kk] = SkinnyChunk{keep ? id : 0, kk, keep ? 1 : 0, 0};
    a.row_map_out[kk] = 0;
  }
}

// The shared-expert slot's chunk (one row, flagged pad = 1) for the grouped
// down launch.
CAI4_DEV void moe1_record_shared(const GvParams &a) {
  if (a.sh_slot >= 0 && a.chunks_out) {
    a.chunks_out[a.sh_slot] = SkinnyChunk{0, a.sh_slot, 1, 1};
    a.row_map_out[a.sh_slot] = 0;
  }
}

// Kernel modes: a plain or grouped GEMV; one MoE token's routed gate/up (the
// workgroup row = the slot, the routing recomputed by each workgroup); one MoE
// token's down projections of all its slots with the combine.
enum GvMode { GV_PLAIN = 0, GV_MOE_GATE_UP = 1, GV_MOE_DOWN = 2 };

constexpr int kGvRing1 = 4;  // k-blocks in flight per wave: single tiles
constexpr int kGvRing2 = 2;  // gate/up tile pairs
constexpr int kGvWavesPerCu = 28;  // planned waves per CU

// One wave's LDS region: its activation planes [planes][kpw * 128] bf16, its
// scales as f32 [nt][kpw][16 rows][gpb] and its zero-point seeds, f32
// [planes][kpw][gpb] (rounded up to 16 bytes).
__host__ __device__ inline int gv_wave_bytes(int planes, int nt, int kpw, int gpb) {
  return planes * kpw * 256 + nt * kpw * gpb * 64 + ((planes * kpw * gpb * 4 + 15) & ~15);
}

// NT: weight tiles per wave (2 = a gate/up pair, SW epilogue); AM: activation
// mode (A_BF16, A_XF32, A_HILO; A_GATHER: f32 x rounded to bf16); RING: k-blocks in flight per wave; KPWM: most
// k-blocks per wave (sizes the per-wave register arrays: fewer registers, more
// resident waves); GPB: scale groups per 128-column k-block (128 / G for G of
// 32 or 64, else 1).  With GPB > 1 each MFMA step must cover whole groups: the
// tiled layout stores such blocks with the fragment's four dwords transposed
// across the four 16-lane rows (layout.hip; step s then holds columns
// 32 s .. 32 s + 31) and the activations are read to match; every group gets
// its own seed and scale.  MODE: GvMode; R: routing
// registers per lane (GV_MOE_GATE_UP; 0: given ids and weights only).
template <int NT, int AM, int RING, int KPWM, int GPB, int MODE, int R, bool SHWG = false>
CAI4_DEV void gemv_body(const GvParams &a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr bool two = AM == A_XF32 || AM == A_HILO;  // hi/lo planes
  constexpr bool xf32 = AM == A_XF32 || AM == A_GATHER;
  constexpr int PL = two ? 2 : 1;
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KB = a.K >> 7, NG = a.K / a.G;
  const int T = blockIdx.x;          // tile (pair) index
  // GV_MOE_DOWN: a.kw waves per slot; slot `slot`, k-range `wis` of it
  const int slot = MODE == GV_MOE_DOWN ? wave / a.kw : 0;
  const int wis = MODE == GV_MOE_DOWN ? wave - slot * a.kw : wave;
  const int kb0 = min(wis * a.kpw, KB), kb1 = min(kb0 + a.kpw, KB), nkb = kb1 - kb0;
  const int rbytes = a.kpw * 256;                // one plane of a wave's slice
  const int wbytes = gv_wave_bytes(PL, NT, a.kpw, GPB);
  uint8_t *reg = lds + (size_t)wave * wbytes;  // this wave's region
  float *sreg = reinterpret_cast<float *>(reg + PL * rbytes);        // scales
  float *seeds = sreg + NT * a.kpw * 16 * GPB;                        // seeds

  // ---- the matrices, the x row and the output row of this workgroup ----
  const uint8_t *w0 = a.w0, *w1 = a.w1, *s0 = a.s0, *s1 = a.s1;
  const uint8_t *xp = static_cast<const uint8_t *>(a.x), *xp2 = static_cast<const uint8_t *>(a.x2);
  size_t orow = 0;
  bool sh_chunk = false;  // grouped: this chunk is the shared-expert slot
  bool live = true;  // false: this wave's slot is skipped, all its loads read nothing
  const int nw = blockDim.x >> 6;
  float *red = reinterpret_cast<float *>(lds + (size_t)nw * wbytes);  // partials [nw - 1][NT][16]
  if constexpr (MODE == GV_MOE_GATE_UP) {
    const int k = a.top_k;
    int e;
    if constexpr (SHWG) {  // the shared expert: always on, its own matrices
      e = 0;
    } else if constexpr (R == 0) {  // given ids and weights (or another launch's routing)
      const int kk = blockIdx.y;
      const int id = a.route.ids[kk];
      const float w = a.route.weights[kk];
      // runner.rs:1811: skip w < threshold
      e = !(w < a.route.threshold) && id >= 0 && id < a.E ? id : -1;
      if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0 && lane < k) {
        const int li = a.route.ids[lane];
        const float lw = a.route.weights[lane];
        const bool keep = !(lw < a.route.threshold) && li >= 0 && li < a.E;
        moe1_record(a, lane, li, lw, keep);
      }
      if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0 && lane == k) moe1_record_shared(a);
    } else {  // every workgroup routes the token itself (wave 0), then broadcasts its slot
      int *bcast = reinterpret_cast<int *>(red + (nw - 1) * NT * 16);  // past the partials
      if (wave == 0) {
        int id = 0;
        float w = 0.f;
        if (a.route.mode == ROUTE_IDS) {
          if (lane < k) {
            id = a.route.ids[lane];
            w = a.route.weights[lane];
          }
        } else {
          route_token<R>(a.route, 0, a.E, lane, id, w);
        }
        const bool keep = !(w < a.route.threshold) && id >= 0 && id < a.E;
        if (blockIdx.x == 0 && blockIdx.y == 0 && lane < k) moe1_record(a, lane, id, w, keep);
        if (blockIdx.x == 0 && blockIdx.y == 0 && lane == k) moe1_record_shared(a);
        if (lane == (int)blockIdx.y) *bcast = keep ? id : -1;
      }
      __syncthreads();
      e = *bcast;
    }
    if (e < 0) return;  // the whole workgroup
    if constexpr (SHWG) {
      w0 = a.sh_w0;
      s0 = a.sh_s0;
      w1 = a.sh_w1;
      s1 = a.sh_s1;
    } else {
      const size_t eo = (size_t)e * a.expert_stride;
      w0 += eo;
      s0 += eo;
      w1 += eo;
      s1 += eo;
    }
    orow = (size_t)blockIdx.y * a.ldo;
  } else if constexpr (MODE == GV_MOE_DOWN) {
    live = a.pos[slot] >= 0;
    const size_t eo = live ? (size_t)a.ids[slot] * a.expert_stride : 0;
    w0 += eo;
    s0 += eo;
    xp += (size_t)slot * a.ldx * 2;
    xp2 += (size_t)slot * a.ldx * 2;
  } else if (a.chunks) {
    const SkinnyChunk c = a.chunks[blockIdx.y];
    if (c.count == 0) return;  // the whole workgroup
    if (NT == 1 && c.pad == 1 && a.sh_out) {  // the shared-expert slot: f32 out
      w0 = a.sh_w0;
      s0 = a.sh_s0;
      sh_chunk = true;
    } else {
      const size_t eo = (size_t)c.expert * a.expert_stride;
      w0 += eo;
      s0 += eo;
      if (NT == 2) {
        w1 += eo;
        s1 += eo;
      }
    }
    const size_t xr = (size_t)(a.row_map ? a.row_map[c.row0] : c.row0) * a.ldx;
    xp += xr * (xf32 ? 4 : 2);
    if (AM == A_HILO) xp2 += xr * 2;
    orow = (size_t)c.row0 * a.ldo;
  }

  // ---- activation slice [kb0, kb1) -> registers (issued first) ----
  // chunk c = 8 columns; lane holds chunks lane + 64 i, i < kpw / 4
  const int nch = nkb * 16;
  u32x4_t xa[KPWM / 4], xb[KPWM / 4];
  {
    const size_t xbytes = live ? (size_t)a.K * (xf32 ? 4 : 2) : 0;
    const buf_rsrc_t r0 = buf_rsrc(xp, xbytes);
    const buf_rsrc_t r1 = buf_rsrc(AM == A_HILO ? xp2 : xp, xbytes);
#pragma unroll
    for (int i = 0; i < KPWM / 4; ++i) {
      const int c = lane + 64 * i;
      const bool ok = i * 64 < nch && c < nch;
      const uint32_t col = (uint32_t)(kb0 * 128 + 8 * c);
      if (xf32) {
        xa[i] = buf_load16(r0, ok ? col * 4 : kBufOOB);
        xb[i] = buf_load16(r0, ok ? col * 4 + 16 : kBufOOB);
      } else {
        xa[i] = buf_load16(r0, ok ? col * 2 : kBufOOB);
        if (AM == A_HILO) xb[i] = buf_load16(r1, ok ? col * 2 : kBufOOB);
      }
    }
  }

  // ---- scales of the slice: 4-byte pieces, 8 GPB per k-block, per tile ----
  // (a loop per tile keeps each load's descriptor uniform: a per-lane choice
  // of descriptor would loop over its values)
  constexpr int kSv = (KPWM * 8 * GPB + 63) / 64;  // pieces per lane and tile at most
  uint32_t sv[NT][kSv];
  const int per = a.kpw * 8 * GPB;  // pieces per tile
  {
    const size_t sbytes = live ? (size_t)NG * 32 : 0;
    const buf_rsrc_t sr[2] = {buf_rsrc(s0 + (size_t)T * NG * 32, sbytes),
                              buf_rsrc(NT == 2 ? s1 + (size_t)T * NG * 32 : s0, sbytes)};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int i = 0; i < kSv; ++i) {
        const int q = lane + 64 * i, j = q / (8 * GPB);
        const bool ok = q < per && j < nkb;
        // the k-block's first group, then its GPB groups' 32-byte rows in turn
        const uint32_t off =
            ok ? (uint32_t)((((kb0 + j) * 128) / a.G) * 32 + 4 * (q - j * 8 * GPB)) : kBufOOB;
        sv[nt][i] = __builtin_amdgcn_raw_buffer_load_b32(sr[nt], off, 0, 0);
      }
    }
  }

  // ---- weight ring ----
  const size_t wbytes_t = live ? (size_t)KB * 1024 : 0;
  const buf_rsrc_t wr0 = buf_rsrc(w0 + (size_t)T * KB * 1024, wbytes_t);
  const buf_rsrc_t wr1 = buf_rsrc(NT == 2 ? w1 + (size_t)T * KB * 1024 : w0, wbytes_t);
  u32x4_t ring[RING][NT];
  // kb past the slice: dead loads (no data moves).  A gate/up pair's loads
  // are non-temporal: measured on config 1 (Infinity Cache flushed, every
  // matrix rotating past it) the gate/up ran 5 % faster; single tiles (the
  // down) gained nothing that way.
  auto issue = [&](int u, int kb) {
    const uint32_t wo = kb < kb1 ? (uint32_t)kb * 1024 + 16 * lane : kBufOOB;
    if constexpr (NT == 2) {
      ring[u][0] = buf_load16_nt(wr0, wo);
      ring[u][1] = buf_load16_nt(wr1, wo);
    } else {
      ring[u][0] = buf_load16(wr0, wo);
    }
  };
#pragma unroll
  for (int u = 0; u < RING; ++u) issue(u, kb0 + u);

  // ---- activation slice, its seeds and the scales -> this wave's LDS region ----
#pragma unroll
  for (int i = 0; i < KPWM / 4; ++i) {
    const int c = lane + 64 * i;
    u32x4_t hi = xa[i], lo = u32x4_t{0u, 0u, 0u, 0u};
    if (AM == A_XF32) {
      const f32x4_t fa = __builtin_bit_cast(f32x4_t, xa[i]);
      const f32x4_t fb = __builtin_bit_cast(f32x4_t, xb[i]);
      hi = act_split_f32_nat(fa, fb, false);
      lo = act_split_f32_nat(fa, fb, true);
    } else if (AM == A_HILO) {
      lo = xb[i];
    } else if (AM == A_GATHER) {  // eight f32 -> eight bf16 (RNE), natural order
      const u32x4_t f0 = xa[i], f1 = xb[i];
      hi.x = f32_to_bf16_rne(bitsf(f0.x)) | (f32_to_bf16_rne(bitsf(f0.y)) << 16);
      hi.y = f32_to_bf16_rne(bitsf(f0.z)) | (f32_to_bf16_rne(bitsf(f0.w)) << 16);
      hi.z = f32_to_bf16_rne(bitsf(f1.x)) | (f32_to_bf16_rne(bitsf(f1.y)) << 16);
      hi.w = f32_to_bf16_rne(bitsf(f1.z)) | (f32_to_bf16_rne(bitsf(f1.w)) << 16);
    }
    // group of chunk c: 16 / GPB consecutive chunks (lanes) of k-block c / 16,
    // its seed at [plane][c / (16 / GPB)]
    const float sh = -136.f * group_sum<GPB>(sum8_bf16(hi));
    const float sl = two ? -136.f * group_sum<GPB>(sum8_bf16(lo)) : 0.f;
    if (i * 64 < nch && c < nch) {
      *reinterpret_cast<u32x4_t *>(reg + 16 * c) = hi;
      if (two) *reinterpret_cast<u32x4_t *>(reg + rbytes + 16 * c) = lo;
      if ((c & (16 / GPB - 1)) == 0) {
        seeds[c / (16 / GPB)] = sh;
        if (two) seeds[a.kpw * GPB + c / (16 / GPB)] = sl;
      }
    }
  }
  // piece q of tile nt: rows 2 r, 2 r + 1 of group g of k-block j
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int i = 0; i < kSv; ++i) {
      const int q = lane + 64 * i, j = q / (8 * GPB);
      const int r = q - j * 8 * GPB, g = r >> 3, row = 2 * (r & 7);
      if (q < per) {
        float *d = sreg + ((nt * a.kpw + j) * 16 + row) * GPB + g;
        d[0] = scale_bits_f32(sv[nt][i], a.sdt);
        d[GPB] = scale_bits_f32(sv[nt][i] >> 16, a.sdt);
      }
    }
  }
  // own region only: no barrier, just this wave's LDS writes
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // ---- k-loop: only the ring's loads ----
  float acc[NT];  // D row 0 (and row 8) only: the token
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = 0.f;
  // step s of lane group lg: columns 32 lg + 8 s (GPB 1) or 32 s + 8 lg (GPB > 1)
  const uint8_t *arow = reg + (GPB > 1 ? 16 : 64) * lg + (two && lr >= 8 ? rbytes : 0);
  const bool lo_slot = two && lg >= 2;  // D rows 8-15: the lo plane
  const float *sdp = seeds + (lo_slot ? a.kpw * GPB : 0);
  const float *scp = sreg + lr * GPB;
  // Unrolled over runs of up to 8 k-blocks (one run unless KPWM is 16),
  // leaving at the slice's end, each refill unconditional (dead past the
  // slice): every ring load is then a value of its own.  A rolled loop, or a
  // refill under a branch, merges ring registers at a join, and the copies
  // that takes wait for the refill just issued.
  constexpr int KU = KPWM < 8 ? KPWM : 8;
#pragma nounroll
  for (int j0 = 0; j0 < (KU < KPWM ? nkb : 1); j0 += KU) {
#pragma unroll
    for (int jj = 0; jj < KU; ++jj) {
      const int j = j0 + jj;  // k-block within the slice
      if (j >= nkb) break;    // uniform
      const int u = jj % RING;
      u32x4_t af[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        af[s] = *reinterpret_cast<const u32x4_t *>(arow + j * 256 + (GPB > 1 ? 64 : 16) * s);
      // the k-block's GPB seeds of this lane's plane, one LDS read
      float sd[GPB];
      lds_read_f32<GPB>(sdp + j * GPB, sd);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const u32x4_t b = ring[u][nt];
        const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
        float sc[GPB];  // row lr's scales of the k-block's groups
        lds_read_f32<GPB>(scp + (nt * a.kpw + j) * 16 * GPB, sc);
#pragma unroll
        for (int q = 0; q < GPB; ++q) {
          // only D row 0 (and row 8) is read: C's other rows may hold anything
          f32x4_t p = __builtin_nondeterministic_value(f32x4_t{});
          p[0] = sd[q];
#pragma unroll
          for (int s = q * (4 / GPB); s < (q + 1) * (4 / GPB); ++s)
            p = mfma_bf16(af[s], decode8(bw[s]), p);
          // only D row 0 (and row 8, the lo plane) is the token
          acc[nt] += sc[q] * p[0];
        }
      }
      // refill the slot just decoded (its registers are free again)
      if (KU < KPWM || jj + RING < KU) {
        issue(u, kb0 + j + RING);
        // keeps the refill here: its only use is past a later exit, and a load
        // sunk to its use is issued just before it is waited for
        asm volatile("" ::: "memory");
      }
    }
  }

  if (two) {  // slot 0 (hi) + slot 8 (lo): lanes 0-31 receive lanes 32-63
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      auto sw = __builtin_amdgcn_permlane32_swap(fbits(acc[nt]), fbits(acc[nt]), false, false);
      acc[nt] += bitsf(sw[1]);
    }
  }

  if constexpr (MODE == GV_MOE_DOWN) {
    // (no multiply-add contraction: the crate rounds w * y, then the sum, as
    // moe_combine_kernel does.  __fmul_rn / __fadd_rn are plain operators
    // defined outside this scope, which the contraction would still fuse)
#pragma clang fp contract(off)
    // ---- every slot's partials -> y_k (RNE bf16) -> the combine in slot order
    // (runner.rs:1806-1832: moe += w * y, multiply then add; h = residual +
    // shared + moe), as moe_combine_kernel does for more tokens ----
    if (lane < 16) red[wave * 16 + lr] = acc[0];
    __syncthreads();
    if (wave > 0 || lane >= 16) return;
    const int r16 = 16 * T + lr;
    if (r16 >= a.N) return;
    float h = a.residual ? a.residual[r16] : 0.f;
    if (a.shared) h = h + a.shared[r16];
    // the top_k * kw <= 16 partials (slot-major, wave order within a slot),
    // every LDS read issued before the first add: a read per add waited for
    // each in turn (16 dependent LDS round trips at the workgroup's tail)
    const int n = a.top_k * a.kw;
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pv[i] = red[min(i, n - 1) * 16 + lr];
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(pv[i]));  // issued here, not per add
    float moe = 0.f, y = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i >= n) break;  // uniform
      y += pv[i];
      if ((i + 1) % a.kw == 0) {  // slot i / kw complete
        const int kk = i / a.kw;
        if (a.pos[kk] >= 0) moe = moe + a.wts[kk] * bf16_to_f32(f32_to_bf16_rne(y));
        y = 0.f;
      }
    }
    // the whole combine, or the weighted expert sum only (residual and shared
    // added later, in the same order)
    reinterpret_cast<float *>(a.out)[r16] = a.moe_partial ? moe : h + moe;
    return;
  }

  // ---- the kw partials (D row 0: lanes 0-15), added in wave order ----
  if (wave > 0 && lane < 16) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) red[((wave - 1) * NT + nt) * 16 + lr] = acc[nt];
  }
  __syncthreads();
  if (wave > 0) return;
  // added in wave order, the LDS reads of eight partials issued before their
  // adds (clamped indices: always inside the kw - 1 partials): a read per add
  // waited for each in turn, ~0.5 us at the tail of a 16-wave workgroup
  for (int w0 = 1; w0 < a.kw; w0 += 8) {
    float v[8][NT];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int w = min(w0 + q, a.kw - 1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) v[q][nt] = red[((w - 1) * NT + nt) * 16 + lr];
    }
    // pin every read here (the compiler would otherwise sink each into the
    // branch of its add, one LDS round trip apiece)
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) asm volatile("" : "+v"(v[q][nt]));
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (w0 + q >= a.kw) break;  // uniform
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] += v[q][nt];
    }
  }
  if (lg != 0) return;  // D row 0 = the token: lanes 0-15, component 0
  const int r16 = 16 * T + lr;
  if (MODE == GV_PLAIN && a.slots) {  // uniform: the sparse-mask epilogue
    float m = 0.f, pos = 0.f;
    if (r16 < a.N) {
      reinterpret_cast<float *>(a.out)[r16] = acc[0];
      if (NT == 2) reinterpret_cast<float *>(a.out2)[r16] = acc[NT - 1];  // up, unfused
      const float sv = a.silu_slot == 2 ? silu_stable(acc[0]) : silu_plain(acc[0]);
      m = fabsf(sv);
      m = m > 0.f ? m : 0.f;  // NaN -> 0: a NaN lane never raises the max
      if (a.thr) pos = a.thr[r16] <= 0.f ? 0.f : 1.f;
    }
    m = row16_max(m);  // lanes 0-15: one DPP row, all live
    pos = row16_max(pos);
    if (lr == 0) a.slots[T] = fbits(m) | (pos > 0.f ? 0x80000000u : 0u);
    return;
  }
  if (r16 >= a.N) return;
  const size_t row = orow + r16;
  const float y = acc[0];
  if (NT == 2) {
    const float h = silu_f32(y) * acc[NT - 1];
    if (a.epi == EPI_SWIGLU) {
      reinterpret_cast<float *>(a.out)[row] = h;
    } else {  // hi = h truncated to bf16, lo = bf16(h - hi): the A_HILO planes
      const uint32_t hb = fbits(h) >> 16;
      reinterpret_cast<uint16_t *>(a.out)[row] = (uint16_t)hb;
      reinterpret_cast<uint16_t *>(a.out2)[row] = (uint16_t)f32_to_bf16_rne(h - bitsf(hb << 16));
    }
  } else if (sh_chunk) {
    a.sh_out[r16] = y;
  } else if (a.epi == EPI_BF16) {
    reinterpret_cast<uint16_t *>(a.out)[row] = (uint16_t)f32_to_bf16_rne(y);
  } else {
    reinterpret_cast<float *>(a.out)[row] = y;
  }
}

// Waves per SIMD each instantiation is compiled for (its VGPR budget: 512 /
// waves, rounded down to 8): the plan's 28 waves per CU are 7 per SIMD.  Up to
// 4 k-blocks per wave with one scale group and one activation plane fit 64
// VGPRs (8), with two planes or small groups 72 (7); 8 k-blocks fit 72 (7); 16
// fit 80 (96 for a gate/up pair over two planes).
template <int NT, int AM, int KPWM, int GPB, int MODE, int R>
constexpr int gv_waves_per_simd() {
  constexpr bool two = AM == A_XF32 || AM == A_HILO;
  if constexpr (KPWM == 4) return two || GPB > 1 ? 7 : 8;
  if constexpr (KPWM == 8) return 7;
  return two && NT == 2 ? 5 : 6;
}

// SH (routed gate/up only): workgroup row a.sh_slot runs the shared expert's
// body (f32 x as hi / lo planes); the kernel then takes the smaller register
// budget of the two bodies.
template <int NT, int AM, int KPWM, int GPB, int MODE, int R, bool SH>
constexpr int gv_waves_per_simd_sh() {
  constexpr int a = gv_waves_per_simd<NT, AM, KPWM, GPB, MODE, R>();
  constexpr int b = gv_waves_per_simd<NT, A_XF32, KPWM, GPB, MODE, 0>();
  return SH && b < a ? b : a;
}

template <int NT, int AM, int KPWM, int GPB, int MODE = GV_PLAIN, int R = 1, bool SH = false>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(
    gv_waves_per_simd_sh<NT, AM, KPWM, GPB, MODE, R, SH>()))) void gemv_kernel(GvParams a) {
  constexpr int RING = NT == 2 ? kGvRing2 : kGvRing1;
  if constexpr (SH) {
    if ((int)blockIdx.y == a.sh_slot) {  // uniform per workgroup
      gemv_body<NT, A_XF32, RING, KPWM, GPB, MODE, 0, true>(a);
      return;
    }
  }
  gemv_body<NT, AM, RING, KPWM, GPB, MODE, R>(a);
}

}  // namespace

size_t gemv_lds_bytes(const GemvPlan &p, int amode, int nt, int gpb);
constexpr size_t kGvMaxLds = 160 * 1024;  // gfx950: LDS of one CU

// Scale groups per 128-column k-block: 4 (G 32), 2 (G 64), 1 (G a multiple of
// 128); 0 = not supported.
int gemv_gpb(int G) { return G == 32 ? 4 : G == 64 ? 2 : (G % 128 == 0 ? 1 : 0); }

bool gemv_supported(const SkinnyArgs &a, int amode, int epi, int num_cus, int chunk_rows,
                    int max_chunks) {
  const int gpb = gemv_gpb(a.G);
  if (!a.tiled || !gpb || a.K % 128 || a.K % a.G) return false;
  if (a.chunks) {  // grouped: one row per chunk, f32 rows gathered / hi-lo rows
    if (chunk_rows != 1 || max_chunks < 1 || max_chunks > 65535) return false;
    if (amode != A_GATHER && amode != A_HILO) return false;
  } else {
    if (a.M != 1) return false;
    if (amode != A_BF16 && amode != A_XF32 && amode != A_HILO) return false;
  }
  const bool sw = epi == EPI_SWIGLU || epi == EPI_SWIGLU_HILO;
  if (sw ? !(a.w1 && a.s1) : !(epi == EPI_F32 || epi == EPI_BF16)) return false;
  const int nt = sw ? 2 : 1;
  const long n_eff = (long)a.N * (a.chunks ? max_chunks : 1);
  if (n_eff > (1L << 30)) return false;
  // K > 256 k-blocks (128 for small groups): kw > 16
  const GemvPlan p = gemv_plan((int)n_eff, a.K, num_cus, gemv_max_kpw(gpb));
  return p.kw >= 1 && p.kw <= 16 && gemv_lds_bytes(p, amode, nt, gpb) <= kGvMaxLds;
}

GemvPlan gemv_plan(int N, int K, int num_cus, int max_kpw) {
  const int tiles = (N + 15) / 16, KB = K / 128;
  if (KB < 1 || tiles < 1 || num_cus < 1) return GemvPlan{0, 0};  // not supported
  // kGvWavesPerCu waves per CU, all resident at once (the register arrays are
  // sized by the k-blocks per wave): many short independent streams
  const long waves = (long)kGvWavesPerCu * num_cus;
  int kw = (int)((2 * waves + tiles) / (2L * tiles));  // nearest
  // at most 8 waves per tile to start from (the loop below adds waves when a
  // wave's k-range would exceed max_kpw): config 0 (one tile per CU) ran
  // 4.53-4.58 -> 4.44-4.45 us with 8 waves of 4 k-blocks instead of 16 of 2;
  // the decode chain and the one-token MoE layers measured the same
  if (kw > 8) kw = 8;
  if (kw < 1) kw = 1;
  if (kw > KB) kw = KB;
  int kpw = (KB + kw - 1) / kw;
  while (kpw > max_kpw) {
    ++kw;
    kpw = (KB + kw - 1) / kw;
  }
  kw = (KB + kpw - 1) / kpw;  // no wave without work
  return GemvPlan{kw, kpw};
}

size_t gemv_lds_bytes(const GemvPlan &p, int amode, int nt, int gpb) {
  const int planes = amode == A_XF32 || amode == A_HILO ? 2 : 1;
  return (size_t)p.kw * gv_wave_bytes(planes, nt, p.kpw, gpb) + (size_t)(p.kw - 1) * nt * 16 * 4 +
         16;
}

hipError_t gemv_launch(const SkinnyArgs &a, int amode, int epi, int num_cus, int max_chunks,
                       hipStream_t st, const GemvSharedSlot *sh) {
  const bool sw = epi == EPI_SWIGLU || epi == EPI_SWIGLU_HILO;
  const int nch = a.chunks ? max_chunks : 1;
  const int gpb = gemv_gpb(a.G);
  const GemvPlan p = gemv_plan(a.N * nch, a.K, num_cus, gemv_max_kpw(gpb));
  GvParams k{};
  k.w0 = a.w0;
  k.w1 = a.w1;
  k.s0 = a.s0;
  k.s1 = a.s1;
  k.x = a.x;
  k.x2 = a.x2;
  k.out = a.out;
  k.out2 = a.out2;
  k.N = a.N;
  k.K = a.K;
  k.G = a.G;
  k.sdt = a.sdt;
  k.epi = epi;
  k.kw = p.kw;
  k.kpw = p.kpw;
  k.slots = a.slots;
  k.thr = a.thr;
  k.silu_slot = a.silu_slot;
  k.chunks = a.chunks;
  k.row_map = a.row_map;
  k.expert_stride = a.expert_stride;
  k.ldx = a.ldx;
  k.ldo = a.ldo;
  k.sh_slot = -1;
  if (sh && a.chunks && !sw) {
    k.sh_w0 = sh->w;
    k.sh_s0 = sh->s;
    k.sh_out = sh->out;
  }
  const size_t lds = gemv_lds_bytes(p, amode, sw ? 2 : 1, gpb);
  const dim3 grid((a.N + 15) / 16, nch), block(64 * p.kw);
#define CAI4_GV_G(NT, AM, GPB)                                                             \
  do {                                                                                     \
    if (p.kpw <= 4)                                                                        \
      hipLaunchKernelGGL((gemv_kernel<NT, AM, 4, GPB>), grid, block, lds, st, k);          \
    else if (p.kpw <= 8)                                                                   \
      hipLaunchKernelGGL((gemv_kernel<NT, AM, 8, GPB>), grid, block, lds, st, k);          \
    else if constexpr (GPB == 1)                                                           \
      hipLaunchKernelGGL((gemv_kernel<NT, AM, 16, 1>), grid, block, lds, st, k);           \
  } while (0)
#define CAI4_GV(NT, AM)                                \
  do {                                                 \
    if (gpb == 4) CAI4_GV_G(NT, AM, 4);                \
    else if (gpb == 2) CAI4_GV_G(NT, AM, 2);           \
    else CAI4_GV_G(NT, AM, 1);                         \
  } while (0)
  if (sw) {
    if (amode == A_BF16) CAI4_GV(2, A_BF16);
    else if (amode == A_XF32) CAI4_GV(2, A_XF32);
    else if (amode == A_GATHER) CAI4_GV(2, A_GATHER);
    else CAI4_GV(2, A_HILO);
  } else {
    if (amode == A_BF16) CAI4_GV(1, A_BF16);
    else if (amode == A_XF32) CAI4_GV(1, A_XF32);
    else CAI4_GV(1, A_HILO);
  }
#undef CAI4_GV_G
#undef CAI4_GV
  return hipGetLastError();
}

namespace {

// GV_MOE_DOWN: waves per slot and k-blocks per wave (0 waves: not supported).
GemvPlan moe1_down_plan(int I, int top_k) {
  const int KB = I / 128, kw = top_k > 0 ? 16 / top_k : 0;
  if (kw < 1 || KB < 1) return GemvPlan{0, 0};
  const int kpw = (KB + kw - 1) / kw;
  return GemvPlan{(KB + kpw - 1) / kpw, kpw};
}

size_t moe1_down_lds(const GemvPlan &p, int top_k, int gpb) {
  const int nw = top_k * p.kw;
  return (size_t)nw * gv_wave_bytes(2, 1, p.kpw, gpb) + (size_t)nw * 64 + 16;
}

}  // namespace

bool gemv_moe1_supported(int H, int I, int G, int top_k, int E, int num_cus) {
  const int gpb = gemv_gpb(G);
  if (!gpb || H % 128 || I % 128 || H % G || I % G) return false;
  if (top_k < 1 || top_k > kMoeMaxTopK || E < 1 || E > kMoeMaxExperts) return false;
  if ((long)I * top_k > (1L << 30)) return false;
  // with a shared-expert slot: top_k + 1 rows of two activation planes
  const GemvPlan gu = gemv_plan(I * (top_k + 1), H, num_cus, 8);
  if (gu.kw < 1 || gu.kw > 16 || gu.kpw > 8) return false;
  const GemvPlan gu0 = gemv_plan(I * top_k, H, num_cus, 8);
  if (gu0.kw < 1 || gu0.kw > 16 || gu0.kpw > 8) return false;
  return gemv_lds_bytes(gu, A_XF32, 2, gpb) <= kGvMaxLds &&
         gemv_lds_bytes(gu0, A_GATHER, 2, gpb) <= kGvMaxLds;
}

bool gemv_moe1_down_fused(int H, int I, int G, int top_k, int num_cus) {
  const int gpb = gemv_gpb(G);
  if (!gpb || H % 128 || I % 128 || H % G || I % G) return false;
  if ((H + 15) / 16 > num_cus) return false;  // one round of workgroups
  const GemvPlan dn = moe1_down_plan(I, top_k);
  if (dn.kw < 1 || dn.kpw > 8) return false;
  return moe1_down_lds(dn, top_k, gpb) <= kGvMaxLds;
}

hipError_t gemv_moe1_gate_up(const Moe1Args &m, int num_cus, hipStream_t st) {
  const int gpb = gemv_gpb(m.G);
  const int rows = m.top_k + (m.sh == 1 ? 1 : 0);
  const GemvPlan p = gemv_plan(m.I * rows, m.H, num_cus, 8);
  GvParams k{};
  k.w0 = m.gate;
  k.s0 = m.gate_s;
  k.w1 = m.up;
  k.s1 = m.up_s;
  k.x = m.x;
  k.x2 = m.x;
  k.out = m.hi;
  k.out2 = m.lo;
  k.N = m.I;
  k.K = m.H;
  k.G = m.G;
  k.sdt = m.sdt;
  k.epi = EPI_SWIGLU_HILO;
  k.kw = p.kw;
  k.kpw = p.kpw;
  k.expert_stride = m.expert_stride;
  k.ldx = m.H;
  k.ldo = m.I;
  k.route = m.route;
  k.E = m.E;
  k.top_k = m.top_k;
  k.ids = m.ids;
  k.wts = m.wts;
  k.pos = m.pos;
  k.chunks_out = m.chunks;
  k.row_map_out = m.row_map;
  k.sh_slot = m.sh ? m.top_k : -1;
  k.sh_w0 = m.sh_gate;
  k.sh_s0 = m.sh_gate_s;
  k.sh_w1 = m.sh_up;
  k.sh_s1 = m.sh_up_s;
  // the shared slot stages two activation planes
  const size_t lds = gemv_lds_bytes(p, m.sh == 1 ? A_XF32 : A_GATHER, 2, gpb);
  const dim3 grid((m.I + 15) / 16, rows), block(64 * p.kw);
#define CAI4_GVR(KP, GP, R)                                                                   \
  do {                                                                                        \
    if (m.sh == 1)                                                                            \
      hipLaunchKernelGGL((gemv_kernel<2, A_GATHER, KP, GP, GV_MOE_GATE_UP, R, true>), grid,   \
                         block, lds, st, k);                                                  \
    else                                                                                      \
      hipLaunchKernelGGL((gemv_kernel<2, A_GATHER, KP, GP, GV_MOE_GATE_UP, R>), grid, block, \
                         lds, st, k);                                                         \
  } while (0)
#define CAI4_GVR_E(KP, GP)                                    \
  do {                                                        \
    if (m.route.mode != ROUTE_IDS && m.E <= 256) CAI4_GVR(KP, GP, 4); \
    else CAI4_GVR(KP, GP, 0);                                 \
  } while (0)
#define CAI4_GVR_K(GP)                        \
  do {                                        \
    if (p.kpw <= 4) CAI4_GVR_E(4, GP);        \
    else CAI4_GVR_E(8, GP);                   \
  } while (0)
  if (gpb == 4) CAI4_GVR_K(4);
  else if (gpb == 2) CAI4_GVR_K(2);
  else CAI4_GVR_K(1);
#undef CAI4_GVR_K
#undef CAI4_GVR_E
#undef CAI4_GVR
  return hipGetLastError();
}

hipError_t gemv_moe1_down(const Moe1Args &m, hipStream_t st) {
  const int gpb = gemv_gpb(m.G);
  const GemvPlan p = moe1_down_plan(m.I, m.top_k);
  GvParams k{};
  k.w0 = m.down;
  k.s0 = m.down_s;
  k.w1 = m.down;
  k.s1 = m.down_s;
  k.x = m.hi;
  k.x2 = m.lo;
  k.out = m.out;
  k.N = m.H;
  k.K = m.I;
  k.G = m.G;
  k.sdt = m.sdt;
  k.epi = EPI_F32;
  k.kw = p.kw;
  k.kpw = p.kpw;
  k.expert_stride = m.expert_stride;
  k.ldx = m.I;
  k.ldo = m.H;
  k.E = m.E;
  k.top_k = m.top_k;
  k.ids = m.ids;
  k.wts = m.wts;
  k.pos = m.pos;
  k.residual = m.residual;
  k.shared = m.shared;
  if (m.moe_sum) {  // the weighted expert sum only (a shared expert finishes later)
    k.out = m.moe_sum;
    k.residual = nullptr;
    k.shared = nullptr;
    k.moe_partial = 1;
  }
  const size_t lds = moe1_down_lds(p, m.top_k, gpb);
  const dim3 grid((m.H + 15) / 16), block(64 * m.top_k * p.kw);
#define CAI4_GVD(KP, GP) \
  hipLaunchKernelGGL((gemv_kernel<1, A_HILO, KP, GP, GV_MOE_DOWN, 1>), grid, block, lds, st, k)
#define CAI4_GVD_K(GP)               \
  do {                               \
    if (p.kpw <= 4) CAI4_GVD(4, GP); \
    else CAI4_GVD(8, GP);            \
  } while (0)
  if (gpb == 4) CAI4_GVD_K(4);
  else if (gpb == 2) CAI4_GVD_K(2);
  else CAI4_GVD_K(1);
#undef CAI4_GVD_K
#undef CAI4_GVD
  return hipGetLastError();
}

}  // namespace cai4
