// skinny.hip -- decode-regime INT4 weight-only GEMM for gfx950 (up to 64
// tokens per pass; larger M loops over M chunks).
//
// y[t, r] = sum_g s[r, g] * sum_{c in g} (nibble[r, c] - 8) * x[t, c]
//
// The GPU counterpart of dequant_gemv_int4 / dequant_gemm_int4_multi_auto
// (crates/cascadia-int4-gemm/src/kernel_avx512.rs:209-297,
// kernel_avx512_multi.rs:66-245) and, with fused epilogues, of the
// gate/up -> SiLU*up -> down chain of expert_forward (kernel.rs:75-136).
//
// Why it is shaped this way.  Decode streams every weight byte exactly once,
// so the k-loop must issue nothing but 16-byte weight loads: one
// buffer_load_dwordx4 per lane moves one 1 KB k-block of a 16-row tile.  The
// activations and scales, which every tile re-reads, are staged into LDS once
// per workgroup with wide cooperative loads (f32 activations are split into
// their hi/lo bf16 planes there, once, instead of at every use); the k-loop
// reads them with ds_read_b128 / ds_read_b32, off the vector-memory path.
//
// Work decomposition.  A workgroup has rw x kw waves.  Wave (r, k) owns the
// nt weight tiles of row unit (blockIdx.x * rw + r) -- one gate tile + one up
// tile of the same 16 output rows for the SwiGLU epilogues -- and the k-th
// contiguous span of the workgroup's k-blocks (128 columns each).  The rw row
// groups share the staged activations.  A register ring keeps U k-blocks of
// weights in flight per wave.  Partial sums of the kw spans are added through
// LDS in fixed wave order; with ksplit > 1 workgroups also split K and
// splitk_reduce_kernel adds their partials in fixed split order.  Every sum
// has one fixed order: results are deterministic (no atomics).
//
// Weight layouts.  CRATE (the crate's row-major bytes) or TILED (layout.hip:
// each 16-row x 128-column block is 1 KB contiguous in lane order, nibbles of
// a dword swizzled so that the decode yields natural column order).  All
// weight loads are buffer loads whose descriptor spans exactly the tile's
// valid bytes: rows past N read 0 from the hardware range check, and a dead
// prefetch (past the wave's span) uses an out-of-range offset, so it moves no
// data.
//
// k-slot mapping.  G % 128 == 0 ("contiguous"): MFMA step s of a k-block
// takes dword s of each lane's chunk; all 128 columns share one scale.
// Otherwise ("transposed", G = 32, 64, ...): step s covers columns
// 32s..32s+31 of the block -- inside one group for any G that is a multiple
// of 32 -- from the chunks transposed across the four lane rows: stored so in
// the tiled layout (layout.hip), transposed after the load with
// v_permlane32_swap / v_permlane16_swap for the crate's bytes.  K must be a
// multiple of 32 and of G.
//
// Token slots of a 16-slot MFMA tile:
//   A_BF16 / A_GATHER: slot i = token i (exact bf16 products);
//   A_XF32 / A_HILO: slots 0-7 = hi plane of tokens 0-7, slots 8-15 = lo plane
//   (hi = f32 truncated to bf16, lo = bf16 of the exact remainder); the two
//   halves of the MFMA result are added: y = D[hi] + D[lo].
#include <stdio.h>
#include <stdlib.h>

#include "int4_common.hpp"
#include "skinny.hpp"
#include "tuning.hpp"

namespace cai4 {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // gfx9 raw buffer: 32-bit data format
constexpr uint32_t kOOB = 0x80000000u;  // an offset past every descriptor's range

CAI4_DEV rsrc_t make_rsrc(const void *base, size_t bytes) {
  const int n = bytes > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, kRsrcFlags);
}

// Everything a launch needs (SkinnyArgs + SkinnyPlan), passed by value.
struct KParams {
  const uint8_t *w0, *w1, *s0, *s1;
  const void *x, *x2;
  void *out, *out2;
  f32x4_t *part;
  const SkinnyChunk *chunks;
  const int32_t *row_map;
  size_t wstride;
  int N, K, G, M, ldx, ldo, sdt, glog2, tiled, amode, epi, x_rows;
  int rw, kw, kper, kslice;
  int act_rows, act_stride, scale_off;
};

// Threads per workgroup the register file allows for an M-tile count.
constexpr int skinny_max_threads(int mt) { return mt >= 4 ? 512 : 1024; }

// k-blocks of weights in flight per wave.  Measured on MI355X: about 10-16 MB
// in flight chip-wide streams best; deeper rings lose bandwidth.
constexpr int skinny_ring_depth(int nt) { return nt == 1 ? 4 : 2; }

// ---------------------------------------------------------------------------
// staging into LDS
// ---------------------------------------------------------------------------


// Activations of tokens [m0, m0 + mcount) and k-blocks [kr0, kr1) go to LDS as
// bf16 planes [plane][row][column], row pitch act_stride bytes, columns in the
// k-slot order of the weight layout (natural when tiled, the decode8 order of
// the crate bytes otherwise), columns past K zero.  Staging is split in two:
// act_issue loads one batch of 16-byte chunks into registers with
// unconditional buffer loads -- invalid items get an out-of-range offset and
// read 0 -- and act_store writes it.  The kernel issues the first batch
// before the weight ring, so that storing it waits only for its own loads
// (loads complete in order).
//
// Item i of a batch is chunk c of row t, i = t * cpr + c; a thread's items
// are tid, tid + nth, ...  Pos steps (t, c) by nth without dividing.
struct Pos {
  int t, c;
};
CAI4_DEV Pos pos_start(int i, int per_row) {
  const int t = i / per_row;
  return Pos{t, i - t * per_row};
}
CAI4_DEV void pos_step(Pos &p, int dt, int dc, int per_row) {
  p.t += dt;
  p.c += dc;
  if (p.c >= per_row) {
    p.c -= per_row;
    p.t += 1;
  }
}

template <int B>
CAI4_DEV void act_issue(const KParams &a, int m0, int mcount, int kr0, int kr1, Pos p, int dt,
                        int dc, u32x4_t (&v)[2][B]) {
  const int cpr = (kr1 - kr0) * 16;
  const bool gat = a.amode == A_GATHER;
  const bool xf32 = a.amode == A_XF32 || gat, hilo = a.amode == A_HILO;
  const uint32_t esz = xf32 ? 4u : 2u;
  const size_t bytes = (size_t)(gat ? a.x_rows : a.M) * a.ldx * esz;
  const rsrc_t r0 = make_rsrc(a.x, bytes);
  const rsrc_t r1 = make_rsrc(hilo ? a.x2 : a.x, bytes);
  // A_GATHER: the x row of each item's grouped row first (all issued before
  // the data loads, which depend on them)
  int row[B];
  if (gat) {
    const rsrc_t rm = make_rsrc(a.row_map, (size_t)a.M * 4);
    Pos q = p;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const bool ok = q.t < mcount;
      row[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(rm, ok ? (uint32_t)(m0 + q.t) * 4 : kOOB,
                                                           0, 0);
      pos_step(q, dt, dc, cpr);
    }
  }
#pragma unroll
  for (int j = 0; j < B; ++j) {
    const int col = kr0 * 128 + 8 * p.c;
    const bool ok = p.t < mcount && col < a.K;
    const uint32_t r = gat ? (uint32_t)row[j] : (uint32_t)(m0 + p.t);
    const uint32_t off = ok ? (r * a.ldx + col) * esz : kOOB;
    v[0][j] = __builtin_amdgcn_raw_buffer_load_b128(r0, off, 0, 0);
    // second source: the lo plane, or the upper 4 floats of an f32 chunk
    v[1][j] = __builtin_amdgcn_raw_buffer_load_b128(
        r1, (ok && (hilo || xf32)) ? off + (xf32 ? 16u : 0u) : kOOB, 0, 0);
    pos_step(p, dt, dc, cpr);
  }
}

template <int B>
CAI4_DEV void act_store(const KParams &a, uint8_t *lds, int mcount, int kr0, int kr1, Pos p,
                        int dt, int dc, const u32x4_t (&v)[2][B]) {
  const int cpr = (kr1 - kr0) * 16;
  const uint32_t plane_bytes = (uint32_t)a.act_rows * a.act_stride;
#pragma unroll
  for (int j = 0; j < B; ++j) {
    if (p.t >= mcount) break;
    uint8_t *d = lds + (uint32_t)p.t * a.act_stride + 16 * p.c;
    if (a.amode == A_XF32) {
      const f32x4_t lo4 = __builtin_bit_cast(f32x4_t, v[0][j]);
      const f32x4_t hi4 = __builtin_bit_cast(f32x4_t, v[1][j]);
      *reinterpret_cast<u32x4_t *>(d) =
          a.tiled ? act_split_f32_nat(lo4, hi4, false) : act_split_f32(lo4, hi4, false);
      *reinterpret_cast<u32x4_t *>(d + plane_bytes) =
          a.tiled ? act_split_f32_nat(lo4, hi4, true) : act_split_f32(lo4, hi4, true);
    } else if (a.amode == A_GATHER) {
      // eight f32 -> eight bf16 (RNE) in natural column order
      const u32x4_t f0 = v[0][j], f1 = v[1][j];
      u32x4_t b;
      b.x = f32_to_bf16_rne(bitsf(f0.x)) | (f32_to_bf16_rne(bitsf(f0.y)) << 16);
      b.y = f32_to_bf16_rne(bitsf(f0.z)) | (f32_to_bf16_rne(bitsf(f0.w)) << 16);
      b.z = f32_to_bf16_rne(bitsf(f1.x)) | (f32_to_bf16_rne(bitsf(f1.y)) << 16);
      b.w = f32_to_bf16_rne(bitsf(f1.z)) | (f32_to_bf16_rne(bitsf(f1.w)) << 16);
      *reinterpret_cast<u32x4_t *>(d) = a.tiled ? b : act_perm_bf16(b);
    } else {
      *reinterpret_cast<u32x4_t *>(d) = a.tiled ? v[0][j] : act_perm_bf16(v[0][j]);
      if (a.amode == A_HILO)
        *reinterpret_cast<u32x4_t *>(d + plane_bytes) = a.tiled ? v[1][j] : act_perm_bf16(v[1][j]);
    }
    pos_step(p, dt, dc, cpr);
  }
}

// First row of weight tile `nt` of row unit `unit`.
template <int NT, bool SW>
CAI4_DEV int tile_row0(int unit, int nt) {
  return SW ? 16 * unit : 16 * (unit * NT + nt);
}

// Scales of the workgroup's rw * NT tiles, groups [g_lo, g_lo + ngw), go to LDS
// as their u16 bits [slot][group][16 rows] (slot = r * NT + nt); rows past N
// read 0.
// Tiled: an item is 8 rows of one group (16 contiguous bytes); crate: one
// scale.  Positions (t = row group, c = item of the slot) step like the
// activations'.  Issue / store split as for the activations.
template <int NT, bool SW, int B>
CAI4_DEV void sc_issue(const KParams &a, int unit0, int g_lo, int ngw, Pos p0, int dt, int dc,
                       u32x4_t (&v)[NT][B]) {
  const int NG = a.K / a.G;
  const int per_slot = ngw * (a.tiled ? 2 : 16);
  const size_t bytes =
      a.tiled ? (size_t)((a.N + 15) / 16) * NG * 32 : (size_t)a.N * NG * 2;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const rsrc_t rs = make_rsrc((SW && nt == 1) ? a.s1 : a.s0, bytes);
    Pos p = p0;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int row0 = tile_row0<NT, SW>(unit0 + p.t, nt);
      if (a.tiled) {
        const int g = p.c >> 1, h = p.c & 1;
        const bool ok = p.t < a.rw && row0 < a.N;
        const uint32_t off = ok ? (uint32_t)(((row0 >> 4) * NG + g_lo + g) * 16 + 8 * h) * 2 : kOOB;
        v[nt][j] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
      } else {
        const int g = p.c >> 4, row = row0 + (p.c & 15);
        const bool ok = p.t < a.rw && row < a.N;
        const uint32_t off = ok ? (uint32_t)(row * NG + g_lo + g) * 2 : kOOB;
        v[nt][j] = u32x4_t{(uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0), 0u, 0u, 0u};
      }
      pos_step(p, dt, dc, per_slot);
    }
  }
}


template <int NT, int B>
CAI4_DEV void sc_store(const KParams &a, uint16_t *dst, int ngw, Pos p0, int dt, int dc,
                       const u32x4_t (&v)[NT][B]) {
  const int per_slot = ngw * (a.tiled ? 2 : 16);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    Pos p = p0;
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (p.t >= a.rw) break;
      uint16_t *slot = dst + (size_t)(p.t * NT + nt) * ngw * 16;
      if (a.tiled) {
        const int g = p.c >> 1, h = p.c & 1;
        *reinterpret_cast<u32x4_t *>(slot + g * 16 + 8 * h) = v[nt][j];
      } else {
        slot[(p.c >> 4) * 16 + (p.c & 15)] = (uint16_t)v[nt][j].x;
      }
      pos_step(p, dt, dc, per_slot);
    }
  }
}

// ---------------------------------------------------------------------------
// the k-loop
// ---------------------------------------------------------------------------

// Weight loads are non-temporal (the cache-policy operand's bit 1, `nt` on
// gfx950): each weight byte is read once per call.  Measured with the
// Infinity Cache flushed and every matrix rotating past it: config 1 at 2-16
// tokens 2.5-4.5 % faster per chain, configs 3 and 4 at 8-32 tokens 3-7 %.
constexpr int kNtLoad = 2;

template <int NT>
CAI4_DEV void load_w(u32x4_t (&b)[NT], const rsrc_t (&wr)[NT], const uint32_t (&wv)[NT], int kb,
                     uint32_t wk, bool live) {
  const uint32_t koff = (uint32_t)kb * wk;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    b[nt] = __builtin_amdgcn_raw_buffer_load_b128(wr[nt], live ? wv[nt] + koff : kOOB, 0, kNtLoad);
}

// MFMAs of one k-block: weights from registers, activations and scales from LDS.
// xp: the fragments are the crate's bytes, not yet transposed (TR only).
// B136: the constant -136 bf16 operand of the zero-point MFMAs, kept in
// registers by the caller for the whole loop (a constant built here was
// rebuilt before every MFMA that used it).
template <int NT, int MT, bool TR>
CAI4_DEV void compute_kb(u32x4_t (&b)[NT], const u32x4_t B136, const uint8_t *lds,
                         const uint32_t (&abase)[MT], const uint32_t (&sbase)[NT], int k, int kr0,
                         int g_lo, int K, int G, int glog2, int sdt, bool xp,
                         f32x4_t (&acc)[MT][NT]) {
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  const uint32_t koff = (uint32_t)(k - kr0) * 256;
  u32x4_t af[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      af[mt][s] = *reinterpret_cast<const u32x4_t *>(lds + abase[mt] + koff + (TR ? 64 * s : 16 * s));
  const int kbase = k * 128;
  if constexpr (!TR) {
    const int g = (glog2 >= 0 ? (kbase >> glog2) : kbase / G) - g_lo;
    f32x4_t corr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      corr[mt] = mfma_bf16(af[mt][0], B136, zero4);
      corr[mt] = mfma_bf16(af[mt][1], B136, corr[mt]);
      corr[mt] = mfma_bf16(af[mt][2], B136, corr[mt]);
      corr[mt] = mfma_bf16(af[mt][3], B136, corr[mt]);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float sc = scale_bits_f32(*reinterpret_cast<const uint16_t *>(lds + sbase[nt] + 32 * g), sdt);
      const u32x4_t d0 = decode8(b[nt].x), d1 = decode8(b[nt].y);
      const u32x4_t d2 = decode8(b[nt].z), d3 = decode8(b[nt].w);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4_t p = mfma_bf16(af[mt][0], d0, corr[mt]);
        p = mfma_bf16(af[mt][1], d1, p);
        p = mfma_bf16(af[mt][2], d2, p);
        p = mfma_bf16(af[mt][3], d3, p);
        acc[mt][nt] += sc * p;
      }
    }
  } else {
    const int nsteps = min(4, (K - kbase) >> 5);
    if (xp) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b[nt] = xpose_rows(b[nt]);
    }
    // the scale group of each 32-column step, once per k-block (uniform;
    // steps past K take the last valid one), then every step's scales, their
    // LDS reads in flight together
    int gs[4];
    if (glog2 >= 0) {
#pragma unroll
      for (int s = 0; s < 4; ++s) gs[s] = ((kbase + 32 * min(s, nsteps - 1)) >> glog2) - g_lo;
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) gs[s] = (kbase + 32 * min(s, nsteps - 1)) / G - g_lo;
    }
    float sc[4][NT];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        sc[s][nt] = scale_bits_f32(
            *reinterpret_cast<const uint16_t *>(lds + sbase[nt] + 32 * gs[s]), sdt);
    // one 32-column step: both tiles' fragments decoded, then the MFMAs,
    // then the scaled adds
    auto step = [&](int s) {
      u32x4_t d[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        d[nt] = decode8(s == 0 ? b[nt].x : s == 1 ? b[nt].y : s == 2 ? b[nt].z : b[nt].w);
      f32x4_t p[MT][NT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const f32x4_t corr = mfma_bf16(af[mt][s], B136, zero4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) p[mt][nt] = mfma_bf16(af[mt][s], d[nt], corr);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] += sc[s][nt] * p[mt][nt];
    };
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s >= nsteps) break;
      step(s);
    }
  }
}

// hi + lo token slots: lanes 0-31 receive the lo half from lanes 32-63.
template <int MT, int NT>
CAI4_DEV void fold_hilo(f32x4_t (&acc)[MT][NT]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float f = acc[mt][nt][v];
        auto sw = __builtin_amdgcn_permlane32_swap(fbits(f), fbits(f), false, false);
        acc[mt][nt][v] = f + bitsf(sw[1]);
      }
}

// Output of one wave's row unit: D lane l holds weight row l % 16 and token
// slots 4 * (l / 16) + v.
template <int NT, int MT, bool SW>
CAI4_DEV void epilogue(const KParams &a, f32x4_t (&acc)[MT][NT], int unit, int m0,
                       int mcount) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const bool hilo = !amode_single_plane(a.amode);
  const int tpm = hilo ? 8 : 16;
  constexpr int NOUT = SW ? NT / 2 : NT;
  if (hilo) {
    fold_hilo<MT, NT>(acc);
    if (lg >= 2) return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NOUT; ++nt) {
      const int row = tile_row0<NT, SW>(unit, nt) + lr;
      if (row >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int ti = mt * tpm + 4 * lg + v;
        if (ti >= mcount) continue;
        const size_t o = (size_t)(m0 + ti) * a.ldo + row;
        const float y = acc[mt][nt][v];
        if constexpr (SW) {
          const float h = silu_f32(y) * acc[mt][nt + NOUT][v];
          if (a.epi == EPI_PAIR_F32) {
            reinterpret_cast<float *>(a.out)[o] = y;
            reinterpret_cast<float *>(a.out2)[o] = acc[mt][nt + NOUT][v];
          } else if (a.epi == EPI_SWIGLU) {
            reinterpret_cast<float *>(a.out)[o] = h;
          } else {
            // hi = h truncated to bf16, lo = bf16(h - hi): the A_HILO planes
            const uint32_t hb = fbits(h) >> 16;
            const float lo = h - bitsf(hb << 16);
            reinterpret_cast<uint16_t *>(a.out)[o] = (uint16_t)hb;
            reinterpret_cast<uint16_t *>(a.out2)[o] = (uint16_t)f32_to_bf16_rne(lo);
          }
        } else {
          if (a.epi == EPI_BF16)
            reinterpret_cast<uint16_t *>(a.out)[o] = (uint16_t)f32_to_bf16_rne(y);
          else
            reinterpret_cast<float *>(a.out)[o] = y;
        }
      }
    }
  }
}

// SDT: the scale dtype (a.sdt) as a constant: one conversion instruction per
// scale in the k-loop.
template <int NT, int MT, bool TR, bool SW, bool SLICED, int SDT>
__global__ __launch_bounds__(skinny_max_threads(MT)) void skinny_kernel(KParams a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int U = skinny_ring_depth(NT);
  constexpr int NI = MT * NT;
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rwi = wave % a.rw, kwi = wave / a.rw;
  const bool hilo = !amode_single_plane(a.amode);
  const int tpm = hilo ? 8 : 16;
  const int unit0 = blockIdx.x * a.rw, unit = unit0 + rwi;
  int m0 = blockIdx.y * tpm * MT;
  int mcount = min(a.M - m0, tpm * MT);
  if (a.chunks) {  // grouped: this workgroup row is one chunk of one expert
    const SkinnyChunk c = a.chunks[blockIdx.y];
    if (c.count <= 0) return;  // uniform, before any barrier
    const size_t eo = (size_t)c.expert * a.wstride;
    a.w0 += eo;
    a.s0 += eo;
    if (a.w1) a.w1 += eo;
    if (a.s1) a.s1 += eo;
    m0 = c.row0;
    mcount = min(c.count, tpm * MT);
  }
  const int kb_total = (a.K + 127) >> 7;
  const int kr0 = blockIdx.z * a.kper, kr1 = min(kr0 + a.kper, kb_total);

  // weight sources of this wave's tiles
  rsrc_t wr[NT];
  uint32_t wv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int r0 = tile_row0<NT, SW>(unit, nt);
    const uint8_t *wb = (SW && nt == 1) ? a.w1 : a.w0;
    const size_t rows_left = r0 < a.N ? (size_t)(a.N - r0) : 0;
    if (a.tiled) {
      const size_t T = (size_t)(r0 >> 4);
      wr[nt] = make_rsrc(wb + T * kb_total * 1024, rows_left ? (size_t)kb_total * 1024 : 0);
      wv[nt] = 16 * lane;
    } else {
      const size_t rb = (size_t)a.K / 2;
      wr[nt] = make_rsrc(wb + (size_t)r0 * rb, rows_left * rb);
      wv[nt] = lr * (uint32_t)rb + 16 * lg;
    }
  }
  const uint32_t wk = a.tiled ? 1024u : 64u;

  // Token slots past mcount read token 0's row: MFMA rows are independent and
  // those output rows are never stored, so no predicate is needed.
  uint32_t abase[MT];
  const uint32_t plane_bytes = (uint32_t)a.act_rows * a.act_stride;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int tok = mt * tpm + (hilo ? (lr & 7) : lr);
    abase[mt] = (hilo && lr >= 8 ? plane_bytes : 0u) +
                (uint32_t)(tok < mcount ? tok : 0) * a.act_stride + (TR ? 16u * lg : 64u * lg);
  }

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The workgroup's k-blocks [kr0, kr1) at once, or (SLICED) in slices of
  // kslice: each slice's activations and scales are staged into LDS, then
  // every wave runs its span of the slice.  Partial sums stay in registers
  // across slices, so a staging too large for LDS costs a barrier per slice
  // rather than a split of K across workgroups (whose f32 partials a second
  // launch must write and read back).  The unsliced instantiation keeps the
  // single stage's register budget.
  constexpr int BA = 4, BS = 2;
  const int nth = blockDim.x, tid = threadIdx.x;
  uint16_t *lds_sc = reinterpret_cast<uint16_t *>(lds + a.scale_off);
  auto run_slice = [&](const int s0, const int s1) {
    const int col_hi = min(a.K, s1 * 128);
    const int g_lo = (s0 * 128) / a.G, ngw = (col_hi + a.G - 1) / a.G - g_lo;
    // this wave's span of the slice
    const int nkb = s1 - s0, per = (nkb + a.kw - 1) / a.kw;
    const int kb0 = s0 + min(kwi * per, nkb), kb1 = s0 + min(kwi * per + per, nkb);

    // Staging loads first, then the weight ring: loads complete in order, so
    // storing the staged batch waits only for the staging loads.
    const int cpr = (s1 - s0) * 16, spr = ngw * (a.tiled ? 2 : 16);
    // thread positions and per-item steps (one division each, per thread)
    const Pos pa = pos_start(tid, cpr), ps = pos_start(tid, spr);
    const Pos da = pos_start(nth, cpr), ds = pos_start(nth, spr);
    u32x4_t av[2][BA];
    u32x4_t sv[NT][BS];
    act_issue<BA>(a, m0, mcount, s0, s1, pa, da.t, da.c, av);
    sc_issue<NT, SW, BS>(a, unit0, g_lo, ngw, ps, ds.t, ds.c, sv);
    u32x4_t ring[U][NT];
#pragma unroll
    for (int u = 0; u < U; ++u) load_w<NT>(ring[u], wr, wv, kb0 + u, wk, kb0 + u < kb1);
    if (s0 > kr0) __syncthreads();  // every wave is done with the previous slice's LDS
    act_store<BA>(a, lds, mcount, s0, s1, pa, da.t, da.c, av);
    sc_store<NT, BS>(a, lds_sc, ngw, ps, ds.t, ds.c, sv);
    // larger stagings: the remaining batches (these wait for the ring too)
    for (int base = BA * nth; base < mcount * cpr; base += BA * nth) {
      const Pos p = pos_start(base + tid, cpr);
      act_issue<BA>(a, m0, mcount, s0, s1, p, da.t, da.c, av);
      act_store<BA>(a, lds, mcount, s0, s1, p, da.t, da.c, av);
    }
    for (int base = BS * nth; base < a.rw * spr; base += BS * nth) {
      const Pos p = pos_start(base + tid, spr);
      sc_issue<NT, SW, BS>(a, unit0, g_lo, ngw, p, ds.t, ds.c, sv);
      sc_store<NT, BS>(a, lds_sc, ngw, p, ds.t, ds.c, sv);
    }
    __syncthreads();

    uint32_t sbase[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      sbase[nt] = a.scale_off + (uint32_t)(((rwi * NT + nt) * ngw * 16 + lr) * 2);

    if (mcount > 0) {
      u32x4_t B136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};  // bf16 -136 x 8
      asm volatile("" : "+v"(B136));  // one register copy for the loop, not rebuilt per use
      // Whole rounds of U k-blocks with no branch between them, then the
      // remainder (its refills would all be dead).  A refill under a branch
      // leaves the load counts of the two paths apart at the join, and the
      // wait there must assume the refill just issued: one load in flight.
      int kb = kb0;
      for (; kb + U <= kb1; kb += U) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          compute_kb<NT, MT, TR>(ring[u], B136, lds, abase, sbase, kb + u, s0, g_lo, a.K, a.G, a.glog2,
                                 SDT, !a.tiled, acc);
          load_w<NT>(ring[u], wr, wv, kb + u + U, wk, kb + u + U < kb1);
        }
      }
#pragma unroll
      for (int u = 0; u < U - 1; ++u)
        if (kb + u < kb1)
          compute_kb<NT, MT, TR>(ring[u], B136, lds, abase, sbase, kb + u, s0, g_lo, a.K, a.G, a.glog2,
                                 SDT, !a.tiled, acc);
    }
  };
  if constexpr (SLICED) {
    for (int s0 = kr0; s0 < kr1; s0 += a.kslice) run_slice(s0, min(s0 + a.kslice, kr1));
  } else {
    run_slice(kr0, kr1);
  }

  // add the kw spans of each row group in wave order (LDS reused)
  __syncthreads();
  f32x4_t *red = reinterpret_cast<f32x4_t *>(lds);
  if (a.kw > 1) {
    if (kwi > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          red[((size_t)((kwi - 1) * a.rw + rwi) * NI + mt * NT + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (kwi > 0) return;
    // in wave order, the LDS reads of GR spans issued before their adds
    // (clamped: always inside the kw - 1 spans written) and pinned there; a
    // read per add waited for each in turn
    constexpr int GR = MT * NT >= 8 ? 1 : 8 / (MT * NT);
    for (int w0 = 1; w0 < a.kw; w0 += GR) {
      f32x4_t v[GR][MT][NT];
#pragma unroll
      for (int q = 0; q < GR; ++q) {
        const int w = min(w0 + q, a.kw - 1);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            v[q][mt][nt] = red[((size_t)((w - 1) * a.rw + rwi) * NI + mt * NT + nt) * 64 + lane];
      }
#pragma unroll
      for (int q = 0; q < GR; ++q)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) asm volatile("" : "+v"(v[q][mt][nt]));
#pragma unroll
      for (int q = 0; q < GR; ++q) {
        if (w0 + q >= a.kw) break;  // uniform
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) acc[mt][nt] += v[q][mt][nt];
      }
    }
  }
  if (mcount <= 0) return;
  if (gridDim.z > 1) {
    const size_t base =
        (((size_t)(blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * a.rw + rwi) * NI;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) a.part[(base + mt * NT + nt) * 64 + lane] = acc[mt][nt];
    return;
  }
  epilogue<NT, MT, SW>(a, acc, unit, m0, mcount);
}

// Split-K: add the ksplit partials of each row unit in split order, then the
// epilogue.  One wave per row unit and M-tile (blockIdx.z), so that large row
// groups or M-tile counts still spread over many waves; the loads of four
// splits are in flight before their (ordered) adds.
template <int NT, int MT, bool SW>
__global__ __launch_bounds__(1024) void splitk_reduce_kernel(KParams a, int ksplit) {
  constexpr int NI = MT * NT;
  const int lane = threadIdx.x & 63;
  const int rwi = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tpm = amode_single_plane(a.amode) ? 16 : 8;
  const int mt = blockIdx.z;
  int m0 = blockIdx.y * tpm * MT;
  int mcount = min(a.M - m0, tpm * MT);
  if (a.chunks) {
    const SkinnyChunk c = a.chunks[blockIdx.y];
    m0 = c.row0;
    mcount = min(c.count, tpm * MT);
  }
  mcount -= mt * tpm;  // rows of this M-tile
  if (mcount <= 0) return;
  const size_t zstride = (size_t)gridDim.y * gridDim.x * a.rw * NI * 64;
  const size_t base = (((size_t)blockIdx.y * gridDim.x + blockIdx.x) * a.rw + rwi) * NI * 64 +
                      (size_t)mt * NT * 64 + lane;
  f32x4_t acc[1][NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[0][nt] = a.part[base + nt * 64];
  for (int z0 = 1; z0 < ksplit; z0 += 4) {
    f32x4_t v[4][NT];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)  // clamped: every load in range, all four in flight
        v[j][nt] = a.part[(size_t)min(z0 + j, ksplit - 1) * zstride + base + nt * 64];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) asm volatile("" : "+v"(v[j][nt]));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (z0 + j < ksplit) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[0][nt] += v[j][nt];
      }
  }
  epilogue<NT, 1, SW>(a, acc, blockIdx.x * a.rw + rwi, m0 + mt * tpm, min(mcount, tpm));
}

// ---------------------------------------------------------------------------
// host-side planning and dispatch
// ---------------------------------------------------------------------------

namespace {

int env_int(const char *name, int lo, int hi) {
  const int v = tuning_env(name, 0);
  return v >= lo && v <= hi ? v : 0;
}

size_t round16(size_t v) { return (v + 15) & ~(size_t)15; }

// Plan overrides: CASCADIA_INT4_SKINNY_{RW,KSPLIT,WAVES} for every plan,
// CASCADIA_INT4_GROUPED_{RW,KSPLIT,WAVES} for grouped (MoE) plans only, taking
// precedence there.  `what` is 0 (RW), 1 (KSPLIT) or 2 (WAVES).
int plan_env(int what, bool grouped, int lo, int hi) {
  static const char *const kGrouped[3] = {"CASCADIA_INT4_GROUPED_RW",
                                          "CASCADIA_INT4_GROUPED_KSPLIT",
                                          "CASCADIA_INT4_GROUPED_WAVES"};
  static const char *const kSkinny[3] = {"CASCADIA_INT4_SKINNY_RW", "CASCADIA_INT4_SKINNY_KSPLIT",
                                         "CASCADIA_INT4_SKINNY_WAVES"};
  if (grouped)
    if (int v = env_int(kGrouped[what], lo, hi)) return v;
  return env_int(kSkinny[what], lo, hi);
}

}  // namespace

namespace {

// m_rows: rows per workgroup row to plan for (M, or a grouped chunk's
// capacity); m_chunks: workgroup rows (0: derive from m_rows).
SkinnyPlan plan_core(int N, int K, int G, int m_rows, int m_chunks, int amode, int epi,
                     const SkinnyDevice &d) {
  SkinnyPlan p{};
  const int tpm = amode_single_plane(amode) ? 16 : 8;
  const int planes = amode_single_plane(amode) ? 1 : 2;
  int mt = (m_rows + tpm - 1) / tpm;
  if (mt > 4) mt = 4;
  if (mt == 3) mt = 4;
  p.mt = mt;
  p.m_chunks = m_chunks > 0 ? m_chunks : (m_rows + tpm * mt - 1) / (tpm * mt);
  p.act_rows = m_rows < tpm * mt ? m_rows : tpm * mt;
  const bool sw = epi_pair(epi);
  const int kb_total = (K + 127) / 128;
  const int maxw = skinny_max_threads(mt) / 64;
  const long target = 16L * d.num_cus;  // about 4 resident waves per SIMD
  // weight tiles per wave: a gate/up pair, else 2 unless that leaves too few waves
  p.nt = 2;
  if (!sw && (long)((N + 31) / 32) * p.m_chunks * maxw < target) p.nt = 1;
  const int nout = sw ? 1 : p.nt;
  const long units = (N + 16 * nout - 1) / (16 * nout);
  // row groups sharing one copy of the staged activations: grow until the
  // staging traffic is at most half the weight bytes, and beyond that while
  // every CU still gets a workgroup (fewer, fuller workgroups stage less)
  // weight bytes the launch streams (grouped: every chunk its own expert's)
  const double wbytes = (sw ? 2.0 : 1.0) * N * (K / 2.0) * (m_chunks > 0 ? m_chunks : 1);
  // Grouped launches weigh each staged activation byte 4x: their staging is a
  // row gather per workgroup (f32 rows for the gate/up), and measured on the
  // MoE layers (configs 3 and 4, 8-64 tokens) the wider row groups this buys
  // run 7-15 % faster; the dense plan keeps the plain byte count (its M = 4
  // and 16 chains ran 4 % slower with the weighting).
  const double stage_weight = m_chunks > 0 ? 4.0 : 1.0;
  int rw = 1;
  while (rw < maxw && rw < units) {
    const double sbytes = (double)((units + rw - 1) / rw) * p.m_chunks * p.act_rows * planes *
                          2.0 * K * stage_weight;
    const long wgs_next = (units + 2 * rw - 1) / (2 * rw) * p.m_chunks;
    if (2.0 * sbytes <= wbytes && (rw >= 2 || wgs_next < d.num_cus)) break;
    rw *= 2;
  }
  if (rw > maxw) rw = maxw;
  // Dense plans: one round of workgroups, between 7/8 of the CUs and all of
  // them, each staging at most kDenseStageBytes of its k-range, K split across
  // workgroups as needed (dense_window).  Without a SwiGLU pair (the down
  // projection, plain GEMMs) from the fewest row groups per workgroup; with
  // one only when the rule above leaves CUs idle, and then the split with the
  // fewest staged plus partial bytes.  Measured on config 1's down (4096 x
  // 14336) at 2 / 4 / 8 / 16 tokens: 11.0 / 13.6 / 13.8 / 17.8 us against 14.4
  // / 16.0 / 16.5 / 22.3 us; config 4's shared expert (f32 x, 7168 / 2048) at 8
  // / 32 / 64 tokens: gate/up 13.1 / 19.9 / 27.9 us against 15.2 / 26.8 / 44.2,
  // down 8.3 / 14.3 / 21.0 against 9.5 / 20.5 / 27.3.
  const bool grouped = m_chunks > 0;
  int ks_min = 0;
  const bool dense_auto =
      !grouped && !plan_env(0, false, 1, 16) && !plan_env(1, false, 1, 64);
  auto dense_window = [&](bool fewest_rows, int *rw_out, int *ks_out) {
    constexpr double kDenseStageBytes = 132.0 * 1024;
    const long lo = (long)d.num_cus * 7 / 8, hi = d.num_cus;
    double best = -1.0;
    for (int r = 1; r <= maxw && r <= units; r *= 2) {
      const long per = (units + r - 1) / r * p.m_chunks;
      const int ks = (int)(hi / per);  // the most splits that stay in one round
      if (ks < 1 || per * ks < lo || ks > kb_total) continue;
      const int kper = (kb_total + ks - 1) / ks;
      const double stage = (double)planes * p.act_rows * 256.0 * kper;
      if (stage > kDenseStageBytes) continue;
      // bytes beyond the weights: staged activations, split-K partials written and read
      const double extra = stage * per * ks +
                           (ks > 1 ? 2.0 * ks * per * r * mt * p.nt * 1024.0 : 0.0);
      if (best < 0 || (!fewest_rows && extra < best)) {
        best = extra;
        *rw_out = r;
        *ks_out = ks;
        if (fewest_rows) break;
      }
    }
    return best >= 0;
  };
  if (dense_auto && !sw) {
    int r, ks;
    if (dense_window(true, &r, &ks)) {
      rw = r;
      ks_min = ks;
    }
  }
  if (int v = plan_env(0, grouped, 1, 16)) rw = v <= maxw ? v : maxw;
  p.rw = rw;
  p.row_blocks = (int)((units + rw - 1) / rw);
  long wgs0 = (long)p.row_blocks * p.m_chunks;
  auto lds_need = [&](int kper, int kw) {
    const size_t stride = (size_t)kper * 256 + 16;
    const size_t act = (size_t)planes * p.act_rows * stride;
    const size_t ngw = ((size_t)kper * 128 + G - 1) / G + 1;
    const size_t sc = (size_t)rw * p.nt * ngw * 32;
    const size_t red = (size_t)(kw - 1) * rw * mt * p.nt * 1024;
    const size_t st = round16(act) + sc;
    return st > red ? st : red;
  };
  const int ks_env = plan_env(1, grouped, 1, 64);
  const int kw_env = plan_env(2, grouped, 1, 16);
  // K decomposition.  Split K across workgroups when fewer than half the CUs
  // would get a workgroup (the reduce launch costs more than that), and --
  // unsliced -- also when the staging does not fit in LDS; or (sliced) stage
  // such a range in slices of K inside the workgroup.  Waves per workgroup:
  // enough that the workgroups sharing a CU (as many as LDS allows, at most
  // those the grid has per CU) bring about 16 waves.  A forced split is a
  // minimum.
  struct KPlan {
    int ksplit, kper, kslice, kw;
  };
  auto plan_k = [&](bool sliced) {
    KPlan q{1, kb_total, kb_total, 1};
    for (int ks = ks_env ? ks_env : (ks_min ? ks_min : 1); ks <= kb_total; ++ks) {
      q.kper = (kb_total + ks - 1) / ks;
      q.ksplit = (kb_total + q.kper - 1) / q.kper;
      const long wgs = wgs0 * q.ksplit;
      q.kslice = q.kper;
      if (sliced)
        while (q.kslice > 1 && lds_need(q.kslice, 1) > d.max_lds) --q.kslice;
      const size_t need1 = lds_need(q.kslice, 1);
      if (!sliced && need1 > d.max_lds && q.ksplit < kb_total) continue;
      long per_cu = (long)(d.max_lds / (need1 ? need1 : 1));
      const long grid_per_cu = (wgs + d.num_cus - 1) / d.num_cus;
      if (per_cu > grid_per_cu) per_cu = grid_per_cu;
      if (per_cu < 1) per_cu = 1;
      long w = target / d.num_cus / (per_cu * rw);
      q.kw = (int)(w < 1 ? 1 : (w > maxw / rw ? maxw / rw : w));
      if (kw_env)
        q.kw = kw_env / rw < 1 ? 1 : (kw_env / rw > maxw / rw ? maxw / rw : kw_env / rw);
      if (q.kw > q.kslice) q.kw = q.kslice;
      while (q.kw > 1 && lds_need(q.kslice, q.kw) > d.max_lds) --q.kw;
      if (ks_env || wgs * 2 >= d.num_cus || q.ksplit >= 64) break;
    }
    return q;
  };
  auto partials = [&](const KPlan &q) {
    return q.ksplit > 1 ? (double)q.ksplit * wgs0 * rw * mt * p.nt * 64 * sizeof(f32x4_t) : 0.0;
  };
  // Slices when the split's f32 partials (written, then read back) would add
  // more than a fifth of the weight bytes: measured, config 3 at 256 tokens
  // 777 -> 608 us per layer; with fewer partial bytes (config 4 gate/up at 8
  // tokens: 7 %) the split ran faster.
  KPlan q = plan_k(false);
  if (2.0 * partials(q) > 0.2 * wbytes) q = plan_k(true);
  // Dense SwiGLU pairs of at most 8 token rows: one round of workgroups (the
  // window above, fewest staged + partial bytes) of 8 waves each -- fewer,
  // longer weight streams per CU than the rule below gives.  Measured on
  // config 1's chain at 2 / 4 / 8 tokens: 27.0 -> 26.4, 32.1-32.4 -> 31.1-31.4,
  // 33.2 -> 32.4-32.8 us; at 16 tokens the window splits K and lost 7 %.
  constexpr int kSwWaves = 8;
  if (dense_auto && sw && p.act_rows <= 8) {
    int r, ks;
    if (dense_window(false, &r, &ks)) {
      rw = r;
      p.rw = rw;
      p.row_blocks = (int)((units + rw - 1) / rw);
      wgs0 = (long)p.row_blocks * p.m_chunks;
      ks_min = ks;
      q = plan_k(false);
      if (2.0 * partials(q) > 0.2 * wbytes) q = plan_k(true);
      q.kw = kSwWaves / rw < 1 ? 1 : kSwWaves / rw;
      if (q.kw > q.kslice) q.kw = q.kslice;
      while (q.kw > 1 && lds_need(q.kslice, q.kw) > d.max_lds) --q.kw;
    }
  } else if (dense_auto && sw && (long)q.ksplit * wgs0 < (long)d.num_cus * 7 / 8) {
    int r, ks;
    if (dense_window(false, &r, &ks)) {
      rw = r;
      p.rw = rw;
      p.row_blocks = (int)((units + rw - 1) / rw);
      wgs0 = (long)p.row_blocks * p.m_chunks;
      ks_min = ks;
      q = plan_k(false);
      if (2.0 * partials(q) > 0.2 * wbytes) q = plan_k(true);
    }
  }
  const int ksplit = q.ksplit, kper = q.kper, kslice = q.kslice, kw = q.kw;
  p.ksplit = ksplit;
  p.kper = kper;
  p.kslice = kslice;
  p.kw = kw;
  p.act_stride = kslice * 256 + 16;
  p.scale_off = (int)round16((size_t)planes * p.act_rows * p.act_stride);
  p.lds_bytes = lds_need(kslice, kw);
  p.partial_bytes =
      ksplit > 1 ? (size_t)ksplit * wgs0 * rw * mt * p.nt * 64 * sizeof(f32x4_t) : 0;
  return p;
}

}  // namespace

SkinnyPlan skinny_plan(int N, int K, int G, int M, int amode, int epi, const SkinnyDevice &d) {
  return plan_core(N, K, G, M, 0, amode, epi, d);
}

SkinnyPlan skinny_plan_grouped(int N, int K, int G, int chunk_rows, int max_chunks, int amode,
                               int epi, const SkinnyDevice &d) {
  return plan_core(N, K, G, chunk_rows, max_chunks < 1 ? 1 : max_chunks, amode, epi, d);
}

namespace {

template <int NT, int MT, bool TR, bool SW>
hipError_t launch_one(const KParams &k, const SkinnyPlan &p, hipStream_t st) {
  dim3 grid(p.row_blocks, p.m_chunks, p.ksplit), block(64 * p.rw * p.kw, 1, 1);
  const bool sliced = p.kslice < p.kper;
  if (k.sdt) {
    if (sliced)
      hipLaunchKernelGGL((skinny_kernel<NT, MT, TR, SW, true, SCALE_F16>), grid, block,
                         p.lds_bytes, st, k);
    else
      hipLaunchKernelGGL((skinny_kernel<NT, MT, TR, SW, false, SCALE_F16>), grid, block,
                         p.lds_bytes, st, k);
  } else {
    if (sliced)
      hipLaunchKernelGGL((skinny_kernel<NT, MT, TR, SW, true, SCALE_BF16>), grid, block,
                         p.lds_bytes, st, k);
    else
      hipLaunchKernelGGL((skinny_kernel<NT, MT, TR, SW, false, SCALE_BF16>), grid, block,
                         p.lds_bytes, st, k);
  }
  if (hipError_t e = hipGetLastError()) return e;
  if (p.ksplit > 1) {
    dim3 g2(p.row_blocks, p.m_chunks, p.mt), b2(64 * p.rw, 1, 1);
    hipLaunchKernelGGL((splitk_reduce_kernel<NT, MT, SW>), g2, b2, 0, st, k, p.ksplit);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <int NT, bool TR, bool SW>
hipError_t launch_mt(const KParams &k, const SkinnyPlan &p, hipStream_t st) {
  switch (p.mt) {
    case 1: return launch_one<NT, 1, TR, SW>(k, p, st);
    case 2: return launch_one<NT, 2, TR, SW>(k, p, st);
    default: return launch_one<NT, 4, TR, SW>(k, p, st);
  }
}

template <bool TR>
hipError_t launch_nt(const KParams &k, const SkinnyPlan &p, bool sw, hipStream_t st) {
  if (sw) return launch_mt<2, TR, true>(k, p, st);
  if (p.nt == 1) return launch_mt<1, TR, false>(k, p, st);
  return launch_mt<2, TR, false>(k, p, st);
}

}  // namespace

hipError_t skinny_launch(const SkinnyArgs &a, const SkinnyPlan &p, int amode, int epi,
                         hipStream_t st) {
  if (p.ksplit > 1 && !a.partials) return hipErrorInvalidValue;
  KParams k{};
  k.w0 = a.w0;
  k.w1 = a.w1;
  k.s0 = a.s0;
  k.s1 = a.s1;
  k.x = a.x;
  k.x2 = a.x2;
  k.out = a.out;
  k.out2 = a.out2;
  k.part = static_cast<f32x4_t *>(a.partials);
  k.chunks = a.chunks;
  k.row_map = a.row_map;
  k.x_rows = a.x_rows;
  k.wstride = a.expert_stride;
  k.N = a.N;
  k.K = a.K;
  k.G = a.G;
  k.M = a.M;
  k.ldx = a.ldx;
  k.ldo = a.ldo;
  k.sdt = a.sdt;
  k.glog2 = a.glog2;
  k.tiled = a.tiled;
  k.amode = amode;
  k.epi = epi;
  k.rw = p.rw;
  k.kw = p.kw;
  k.kper = p.kper;
  k.kslice = p.kslice;
  k.act_rows = p.act_rows;
  k.act_stride = p.act_stride;
  k.scale_off = p.scale_off;
  const bool sw = epi_pair(epi);
  const bool tr = (a.G % 128) != 0;
  return tr ? launch_nt<true>(k, p, sw, st) : launch_nt<false>(k, p, sw, st);
}

}  // namespace cai4
