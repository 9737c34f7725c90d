// grouped.hip -- INT4 weight-only GEMM on MFMA tiles of up to 128 rows, for
// one matrix (dense prefill) or for the row groups of many experts in one
// launch (a MoE layer whose experts receive many tokens each).
//
// The crate runs these as per-token GEMVs (kernel_avx512_multi.rs:240-244;
// the runner's per-(token, expert) loop, runner.rs:2079-2108); every output
// element is the same sum, y = sum_g s_g * sum_{c in g} (nibble - 8) x_c, with
// exact products and f32 accumulation.
//
// Arithmetic (as in prefill.hip): weights enter v_mfma_f32_16x16x32_bf16 as
// the exact bf16 value 128 + nibble; each group's partial starts from the
// seed -136 * sum(x) over the group's columns (computed once per row and
// group by gg_prep) and is scaled in f32 when the group ends, acc += s * p.
// A group of 32 or 64 columns spans one or two 32-column MFMA steps: the
// tiled layout stores those matrices' fragments with their four dwords (one
// 32-column segment of the 128-column k-block each, per 16-lane row)
// transposed across the lane rows (layout.hip), so that step s holds columns
// 32 s .. 32 s + 31 as loaded, and the activation fragment of lane row c in
// step s is chunk 4 s + c.  Groups of 128 or more keep the untransposed order
// (step s = chunk 4 c + s).
//
// Two-plane activations (hilo): the A operand is hi + lo (two bf16 planes
// whose sum carries an f32 value to 2^-16: the SwiGLU intermediate, or an f32
// input); each step runs the MFMA on both planes with the same decoded weights.
//
// SwiGLU: a workgroup holds gate and up tiles of the same columns; each wave
// has NT / 2 of each, and the epilogue writes hi / lo of silu(g) * u.
//
// Grouped mode: workgroup row y takes chunk y of a table written by the MoE
// grouping -- (expert, first grouped row, rows) -- and reads expert e's
// matrices at + e * estride.  A tile's rows past its count read zeros and are
// not stored; M-tiles wholly past the count skip their MFMAs, so an expert
// with few rows costs little more than streaming its weights.
//
// Pipeline (as in prefill.hip): three LDS stages; every stage's activations,
// weight tiles, scales and seeds go global -> LDS by buffer loads with an LDS
// destination, two k-blocks ahead, issued in eight parts over the steps.
#include "grouped.hpp"
#include "int4_common.hpp"

namespace cai4 {

namespace {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;

CAI4_DEV rsrc_t rsrc(const void *base, size_t bytes) {
  const int n = bytes > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

template <int n>
CAI4_DEV void gg_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(n) : "memory");
}

CAI4_DEV uint32_t lds_addr(const uint8_t *p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)p);
}

// One global -> LDS buffer load (16 or 4 bytes per lane, lane i at M0 +
// bytes * i).  Inline asm: the compiler cannot tell the stage buffers apart
// and would make LDS reads of any stage wait for the newest prefetch.
template <int bytes>
CAI4_DEV void gg_dma(rsrc_t r, uint32_t lds, uint32_t voff) {
  if constexpr (bytes == 16)
    asm volatile("buffer_load_dwordx4 %1, %2, 0 offen lds" ::"{m0}"(lds), "v"(voff), "s"(r)
                 : "memory");
  else
    asm volatile("buffer_load_dword %1, %2, 0 offen lds" ::"{m0}"(lds), "v"(voff), "s"(r)
                 : "memory");
}

// Workgroup geometry and the LDS of one stage: activations [PL][BM][256 B]
// (XOR-swizzled 16-byte chunks), weight tiles [NT16][1 KB], scales
// [NT16][GPK][16] u16, seeds [GPK][BM] f32.
template <int MS, int NT, int WM, int WN, int GPK, bool HILO, bool SW>
struct Gg {
  static constexpr int W = WM * WN;
  static constexpr int PL = HILO ? 2 : 1;
  static constexpr int BM = 16 * MS * WM, BN = 16 * NT * WN;
  static constexpr int RM = 16 * MS;
  static constexpr int NT16 = NT * WN;                 // weight tiles per stage
  static constexpr int OUTC = SW ? BN / 2 : BN;        // output columns per workgroup
  static constexpr int A = 0, B = PL * BM * 256, S = B + NT16 * 1024, X = S + NT16 * 32 * GPK,
                       BYTES = X + BM * 4 * GPK;
  static constexpr int AL = PL * BM / (4 * W);         // 1 KB activation loads per wave
  static constexpr int BL = NT16 / W;                  // weight tiles per wave
  static constexpr int SLANES = NT16 * 8 * GPK / W;    // 4-byte scale lanes per wave
  static constexpr int SLD = (SLANES + 63) / 64;
  static constexpr int XLANES = GPK * BM / (4 * W);    // 16-byte seed lanes per wave
  static constexpr int LOADS = AL + BL + SLD + 1;
  static_assert(AL >= 1 && BL >= 1 && XLANES >= 1 && XLANES <= 64, "workgroup shape");
  static_assert(SLANES < 64 || SLANES % 64 == 0, "scale lanes");
  static_assert(!SW || (W % 2 == 0 && NT % 2 == 0 && (NT16 / 2) % BL == 0), "SwiGLU shape");
  static_assert(3 * BYTES <= 160 * 1024, "LDS");
};

constexpr uint32_t kGgOOB = 0x80000000u;  // an offset past every range: no data moves

// What a wave's loads of a k-block read: its rsrcs (the weight / scale ones
// are the wave's own matrix in SwiGLU mode) and geometry.
struct GgLd {
  rsrc_t xr0, xr1, wr, sr, qr;
  int K, KB, NG, G, Rp, wave, lane, half;  // half: SwiGLU, the wave loads up tiles
  int mrows;  // live rows of the tile
  // rows through a row map (GgArgs::row_map): each A load's byte offset at
  // k-block 0 (its x row and chunk; kGgOOB for a row past the count) and the
  // seed lane's (one x row and group per lane, 4 bytes)
  int ind;
  uint32_t aoff[4], soff;
};

template <class P, int GPK, bool SW>
CAI4_DEV void gg_load(int l, uint8_t *buf, const GgLd &d, int kb) {
  const int lane = d.lane;
  if (l < P::AL) {
    const int blk = d.wave * P::AL + l;
    const int pl = blk / (P::BM / 4), rb = blk - pl * (P::BM / 4);
    const int row = 4 * rb + (lane >> 4);
    const int q = (lane & 15) ^ (row & 15);
    if (4 * rb < d.mrows)
      gg_dma<16>(P::PL > 1 && pl ? d.xr1 : d.xr0, lds_addr(buf + P::A + blk * 1024),
                 d.ind ? d.aoff[l < 4 ? l : 0] + (uint32_t)kb * 256
                       : (uint32_t)(row * d.K + kb * 128 + 8 * q) * 2);
    else if (lane == 0)
      // a block of dead rows (past the tile's count, never stored): one 4-byte
      // load instead, so that every stage issues the same number of loads (the
      // stage waits count them)
      gg_dma<4>(d.xr0, lds_addr(buf + P::A + blk * 1024), 0);
  } else if (l < P::AL + P::BL) {
    const int tile = d.wave * P::BL + (l - P::AL);
    const int mt = SW && d.half ? tile - P::NT16 / 2 : tile;  // tile within its matrix
    gg_dma<16>(d.wr, lds_addr(buf + P::B + tile * 1024),
               (uint32_t)(mt * d.KB + kb) * 1024 + 16 * lane);
  } else if (l < P::AL + P::BL + P::SLD) {
    // scales: the wave's BL tiles, 32 GPK bytes each, 4 bytes per lane; lanes
    // past SLANES must not run (they would write the next wave's slots)
    const int i = (l - P::AL - P::BL) * 64 + lane;
    const int tile = d.wave * P::BL + i / (8 * GPK), j = i % (8 * GPK);
    const int mt = SW && d.half ? tile - P::NT16 / 2 : tile;
    const int g0 = (kb * 128) / d.G;
    if (i < P::SLANES)
      gg_dma<4>(d.sr, lds_addr(buf + P::S + (d.wave * P::SLANES + (i & ~63)) * 4),
                (uint32_t)((mt * d.NG + g0) * 32 + 4 * j));
  } else if (d.ind) {
    // seeds through the row map: one row of one group per lane
    constexpr int XL4 = GPK * P::BM / P::W;
    if (lane < XL4)
      gg_dma<4>(d.qr, lds_addr(buf + P::X + d.wave * XL4 * 4),
                d.soff + (uint32_t)(kb * GPK * d.Rp) * 4);
  } else {
    // seeds: 4 rows of one group per lane
    if (lane < P::XLANES) {
      const int idx = d.wave * P::XLANES + lane;
      const int g = idx / (P::BM / 4), rq = idx - g * (P::BM / 4);
      gg_dma<16>(d.qr, lds_addr(buf + P::X + d.wave * P::XLANES * 16),
                 (uint32_t)((kb * GPK + g) * d.Rp + 4 * rq) * 4);
    }
  }
}

struct GgNext {
  uint8_t *buf;
  GgLd d;
  int kb, KE;
};

template <class P, int GPK, bool SW>
CAI4_DEV void gg_issue_part(const GgNext &n, int part) {
  if (n.kb < n.KE) {
#pragma unroll
    for (int l = 0; l < P::LOADS; ++l)
      if (l >= part * P::LOADS / 8 && l < (part + 1) * P::LOADS / 8)
        gg_load<P, GPK, SW>(l, n.buf, n.d, n.kb);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Activation fragments of step s for the MS M-tiles (and the lo plane).
template <class P, int MS, int GPK>
CAI4_DEV void gg_read_a(const uint8_t *buf, int wm, int lane, int s, u32x4_t (&af)[P::PL][MS]) {
  const int lr = lane & 15, lg = lane >> 4;
  const int chunk = GPK > 1 ? 4 * s + lg : 4 * lg + s;
#pragma unroll
  for (int p = 0; p < P::PL; ++p)
#pragma unroll
    for (int i = 0; i < MS; ++i) {
      const int row = wm * P::RM + 16 * i + lr;  // row & 15 == lr
      af[p][i] = *reinterpret_cast<const u32x4_t *>(buf + P::A + p * P::BM * 256 + row * 256 +
                                                    16 * (chunk ^ lr));
    }
}

// LDS tile index of the wave's j-th weight tile.
template <class P, int NT, bool SW>
CAI4_DEV int gg_tile(int wn, int j) {
  if constexpr (SW)
    return j < NT / 2 ? wn * (NT / 2) + j : P::NT16 / 2 + wn * (NT / 2) + (j - NT / 2);
  else
    return NT * wn + j;
}

template <class P, int MS, int NT, int GPK, bool HILO, bool SW>
CAI4_DEV void gg_compute(const uint8_t *buf, int wm, int wn, int lane, int sdt, int mt_live,
                         const GgNext &nx, f32x4_t (&acc)[MS][NT]) {
  constexpr int SPG = 4 / GPK;  // MFMA steps per group
  const int lr = lane & 15, lg = lane >> 4;
  u32x4_t b[NT];
  float sc[GPK][NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int tile = gg_tile<P, NT, SW>(wn, j);
    b[j] = *reinterpret_cast<const u32x4_t *>(buf + P::B + tile * 1024 + 16 * lane);
#pragma unroll
    for (int g = 0; g < GPK; ++g) {
      const uint32_t bits =
          *reinterpret_cast<const uint16_t *>(buf + P::S + tile * 32 * GPK + g * 32 + 2 * lr);
      sc[g][j] = scale_bits_f32(bits, sdt);
    }
  }
  f32x4_t p[MS][NT];
  u32x4_t af[P::PL][MS], an[P::PL][MS];
  gg_read_a<P, MS, GPK>(buf, wm, lane, 0, af);
  f32x4_t seed[MS];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int g = s / SPG;
    const bool first = s % SPG == 0, last = s % SPG == SPG - 1;
    if (first) {
#pragma unroll
      for (int i = 0; i < MS; ++i)
        // D layout: lane holds rows 4 (lane / 16) + v of the 16-row tile
        seed[i] = *reinterpret_cast<const f32x4_t *>(
            buf + P::X + 4 * (g * P::BM + wm * P::RM + 16 * i + 4 * lg));
    }
    if (s < 3) gg_read_a<P, MS, GPK>(buf, wm, lane, s + 1, an);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4_t d[NT / 2];
#pragma unroll
      for (int j = 0; j < NT / 2; ++j) d[j] = decode8(b[h * NT / 2 + j][s]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < NT / 2; ++j)
#pragma unroll
        for (int i = 0; i < MS; ++i) {
          if (i >= mt_live) continue;  // uniform: M-tile past the rows
          f32x4_t c = first ? seed[i] : p[i][h * NT / 2 + j];  // NOLINT
          c = mfma_bf16(af[0][i], d[j], c);
          if constexpr (HILO) c = mfma_bf16(af[1][i], d[j], c);
          p[i][h * NT / 2 + j] = c;
        }
      __builtin_amdgcn_sched_barrier(0);
      gg_issue_part<P, GPK, SW>(nx, 2 * s + h);
    }
    if (last) {
#pragma unroll
      for (int i = 0; i < MS; ++i) {
        if (i >= mt_live) continue;
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] += sc[g][j] * p[i][j];
      }
    }
#pragma unroll
    for (int q = 0; q < P::PL; ++q)
#pragma unroll
      for (int i = 0; i < MS; ++i) af[q][i] = an[q][i];
  }
}

template <class P, int MS, int NT, int GPK, bool HILO, bool SW>
CAI4_DEV void gg_stage(uint8_t *cur, uint8_t *nxt2, const GgLd &d, int kb, int KE, int wm, int wn,
                       int sdt, int mt_live, f32x4_t (&acc)[MS][NT]) {
  if (kb >= KE) return;  // uniform
  if (kb + 1 < KE)
    gg_wait_barrier<P::LOADS>();
  else
    gg_wait_barrier<0>();
  const GgNext nx{nxt2, d, kb + 2, KE};
  gg_compute<P, MS, NT, GPK, HILO, SW>(cur, wm, wn, d.lane, sdt, mt_live, nx, acc);
}

// SDT: the scale dtype (a.sdt) as a constant, so that each scale's f32
// conversion is one instruction in the k-loop.
template <int MS, int NT, int WM, int WN, int GPK, bool HILO, bool SW, int SDT>
__global__ __launch_bounds__(64 * WM * WN) void gg_kernel(GgArgs a) {
  using P = Gg<MS, NT, WM, WN, GPK, HILO, SW>;
  __shared__ __attribute__((aligned(16))) uint8_t stages[3 * P::BYTES];
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave % WM, wn = wave / WM;
  // this workgroup's rows
  int e = 0, row0, mrows;
  if (a.tiles) {
    const int sub = blockIdx.y % a.tile_split;
    const SkinnyChunk c = a.tiles[blockIdx.y / a.tile_split];
    const int cnt = c.count - sub * P::BM;
    if (cnt <= 0) return;  // uniform: an empty table entry, or past its rows
    e = c.expert;
    row0 = c.row0 + sub * P::BM;
    mrows = cnt < P::BM ? cnt : P::BM;
  } else {
    row0 = blockIdx.y * P::BM;
    mrows = a.M - row0 < P::BM ? a.M - row0 : P::BM;
  }
  e = __builtin_amdgcn_readfirstlane(e);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  mrows = __builtin_amdgcn_readfirstlane(mrows);
  const int live = mrows - wm * P::RM;
  const int mt_live = live <= 0 ? 0 : (live + 15) >> 4;  // this wave's M-tiles holding rows
  const int KB = a.K >> 7, NG = a.K / a.G;
  const int ntiles = (a.N + 15) >> 4;
  const int T0 = blockIdx.x * (P::OUTC / 16);
  constexpr int TM = SW ? P::NT16 / 2 : P::NT16;  // tiles per matrix per workgroup
  const int tv = __builtin_amdgcn_readfirstlane(ntiles - T0 > TM ? TM : ntiles - T0);
  const size_t eo = (size_t)e * a.estride;
  const int half = SW ? (wave >= P::W / 2 ? 1 : 0) : 0;
  const uint8_t *wm0 = half ? a.w1 : a.w0, *sm0 = half ? a.s1 : a.s0;
  GgLd d;
  d.wr = rsrc(wm0 + eo + (size_t)T0 * KB * 1024, (size_t)tv * KB * 1024);
  d.sr = rsrc(sm0 + eo + (size_t)T0 * NG * 32, (size_t)tv * NG * 32);
  d.xr0 = rsrc(a.x + (size_t)row0 * a.K, (size_t)mrows * a.K * 2);
  d.xr1 = rsrc(HILO ? a.x2 + (size_t)row0 * a.K : a.x, HILO ? (size_t)mrows * a.K * 2 : 0);
  d.qr = rsrc(a.seeds + row0, ((size_t)(KB * GPK - 1) * a.rows_pad + P::BM) * 4);
  d.K = a.K;
  d.KB = KB;
  d.NG = NG;
  d.G = a.G;
  d.Rp = a.rows_pad;
  d.wave = wave;
  d.lane = lane;
  d.half = half;
  d.mrows = mrows;
  d.ind = 0;
  // rows through a row map: the grouped one-plane shapes only (gg_grouped
  // refuses the others); uniform
  if constexpr (!HILO && P::AL <= 4 && GPK * P::BM / P::W <= 64) {
    if (a.row_map) {
      d.ind = 1;
      d.xr0 = rsrc(a.x, (size_t)a.x_rows * a.K * 2);
      d.qr = rsrc(a.seeds, (size_t)KB * GPK * a.rows_pad * 4);
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const int blk = wave * P::AL + l, rb = blk % (P::BM / 4);
        const int row = 4 * rb + (lane >> 4), q = (lane & 15) ^ (row & 15);
        d.aoff[l] = l < P::AL && row < mrows
                        ? (uint32_t)(((size_t)a.row_map[row0 + row] * a.K + 8 * q) * 2)
                        : kGgOOB;
      }
      constexpr int XL4 = GPK * P::BM / P::W;
      const int idx = wave * XL4 + lane, g = idx / P::BM, rq = idx - g * P::BM;
      d.soff = lane < XL4 && rq < mrows
                   ? (uint32_t)(((size_t)g * a.rows_pad + a.row_map[row0 + rq]) * 4)
                   : kGgOOB;
    }
  }

  f32x4_t acc[MS][NT];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int kb0 = blockIdx.z * a.kper, KE = min(KB, kb0 + a.kper);
#pragma unroll
  for (int l = 0; l < P::LOADS; ++l) gg_load<P, GPK, SW>(l, stages, d, kb0);
  if (kb0 + 1 < KE) {
#pragma unroll
    for (int l = 0; l < P::LOADS; ++l) gg_load<P, GPK, SW>(l, stages + P::BYTES, d, kb0 + 1);
  }
  // one stage per iteration, not unrolled: the stage buffers rotate at run
  // time, so the compiler cannot hoist one stage's work into another's
  int cur = 0;
#pragma unroll 1
  for (int kb = kb0; kb < KE; ++kb) {
    const int nx2 = cur == 0 ? 2 : cur - 1;  // (cur + 2) % 3
    gg_stage<P, MS, NT, GPK, HILO, SW>(stages + cur * P::BYTES, stages + nx2 * P::BYTES, d, kb,
                                       KE, wm, wn, SDT, mt_live, acc);
    cur = cur == 2 ? 0 : cur + 1;
  }

  // epilogue: D lane l holds column l % 16 and rows 4 (l / 16) + v
  constexpr int NOUT = SW ? NT / 2 : NT;
  // SwiGLU: this lane's sum of hi + lo over its NOUT columns, per row
  float rsum[SW ? MS : 1][4];
#pragma unroll
  for (int i = 0; i < (SW ? MS : 1); ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) rsum[i][v] = 0.f;
#pragma unroll
  for (int i = 0; i < MS; ++i) {
#pragma unroll
    for (int j = 0; j < NOUT; ++j) {
      const int n = T0 * 16 + 16 * (SW ? wn * (NT / 2) + j : NT * wn + j) + lr;
      if (n >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = wm * P::RM + 16 * i + 4 * lg + v;
        if (m >= mrows) continue;
        const size_t o = (size_t)(row0 + m) * a.ldy + n;
        const float y = acc[i][j][v];
        if constexpr (SW) {
          const float h = silu_f32(y) * acc[i][j + NT / 2][v];
          const uint32_t hb = fbits(h) >> 16;  // hi = h truncated, lo = RNE(h - hi)
          const uint32_t lb = f32_to_bf16_rne(h - bitsf(hb << 16));
          reinterpret_cast<uint16_t *>(a.y)[o] = (uint16_t)hb;
          reinterpret_cast<uint16_t *>(a.y2)[o] = (uint16_t)lb;
          rsum[SW ? i : 0][v] += bitsf(hb << 16) + bf16_to_f32(lb);
        } else if (a.part) {
          a.part[(size_t)blockIdx.z * a.M * a.N + (size_t)(row0 + m) * a.N + n] = y;
        } else if (a.epi == GG_F32) {
          reinterpret_cast<float *>(a.y)[o] = y;
        } else {
          reinterpret_cast<uint16_t *>(a.y)[o] = (uint16_t)f32_to_bf16_rne(y);
        }
      }
    }
  }
  if constexpr (SW) {
    // the seeds of the planes just written, for the GEMM that reads them as A
    // (in place of a pass over them): per row, the 16 lanes of a DPP row add
    // their columns; a group wider than one wave's 8 NT columns adds its
    // waves' sums through LDS in wave order
    if (a.seeds_out) {
      const int per = a.seeds_gw / (8 * NT);  // waves (wn) per group: 1, 2 or 4
      const int c0 = T0 * 16 + 16 * wn * (NT / 2);  // the wave's first output column
      float t[MS][4];
#pragma unroll
      for (int i = 0; i < MS; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) t[i][v] = row16_sum(rsum[i][v]);
      float *so = a.seeds_out + (size_t)(c0 / a.seeds_gw) * a.seeds_rp + row0;
      if (per == 1) {
        if (lr == 0 && c0 < a.N) {
#pragma unroll
          for (int i = 0; i < MS; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int m = wm * P::RM + 16 * i + 4 * lg + v;
              if (m < mrows) so[m] = -136.f * t[i][v];
            }
        }
      } else {
        __syncthreads();  // every wave is past its last read of the stages
        float *part = reinterpret_cast<float *>(stages);  // [WN][BM]
        if (lr == 0) {
#pragma unroll
          for (int i = 0; i < MS; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) part[wn * P::BM + wm * P::RM + 16 * i + 4 * lg + v] = t[i][v];
        }
        __syncthreads();
        if (wn % per == 0 && lr == 0 && c0 < a.N) {
#pragma unroll
          for (int i = 0; i < MS; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int m = wm * P::RM + 16 * i + 4 * lg + v;
              float sum = part[wn * P::BM + m];
              for (int q = 1; q < per; ++q) sum += part[(wn + q) * P::BM + m];
              if (m < mrows) so[m] = -136.f * sum;
            }
        }
      }
    }
  }
}

// y = sum over the ksplit partials, in slice order; bf16 (RNE) or f32.
__global__ __launch_bounds__(256) void gg_reduce_kernel(const float *part, void *y, int M, int N,
                                                        int ldy, int ksplit, int out_f32) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const size_t n = (size_t)M * N;
  if (i >= n) return;  // n is a multiple of 4
  f32x4_t s = *reinterpret_cast<const f32x4_t *>(part + i);
  // ksplit <= 4: the other slices' loads all issued (clamped to the last
  // slice) before the adds, which go in slice order
  f32x4_t v[3];
#pragma unroll
  for (int z = 1; z < 4; ++z)
    v[z - 1] = *reinterpret_cast<const f32x4_t *>(part + (size_t)min(z, ksplit - 1) * n + i);
#pragma unroll
  for (int z = 1; z < 4; ++z) asm volatile("" : "+v"(v[z - 1]));
#pragma unroll
  for (int z = 1; z < 4; ++z)
    if (z < ksplit) s += v[z - 1];
  const size_t r = i / N, c = i - r * N;  // N % 4 == 0: the four stay in one row
  const size_t o = r * ldy + c;
  if (out_f32) {
    float *yf = reinterpret_cast<float *>(y) + o;
    yf[0] = s.x;
    yf[1] = s.y;
    yf[2] = s.z;
    yf[3] = s.w;
  } else {
    uint16_t *yb = reinterpret_cast<uint16_t *>(y) + o;
    yb[0] = (uint16_t)f32_to_bf16_rne(s.x);
    yb[1] = (uint16_t)f32_to_bf16_rne(s.y);
    yb[2] = (uint16_t)f32_to_bf16_rne(s.z);
    yb[3] = (uint16_t)f32_to_bf16_rne(s.w);
  }
}

// ---------------------------------------------------------------------------
// gg_prep: seeds (and converted activations), one wave per row
// ---------------------------------------------------------------------------

// Sum over groups of L consecutive lanes (L = 4, 8, 16 within a DPP row):
// quad sums, then a half-row mirror (lane i <- 7 - i of its 8 lanes: the other
// quad of the same half), then a row mirror (the other half).
template <int L>
CAI4_DEV float lane_group_sum(float t) {
  t += dpp_f32<0xB1>(t);                          // quad_perm 1,0,3,2
  t += dpp_f32<0x4E>(t);                          // quad_perm 2,3,0,1
  if constexpr (L >= 8) t += dpp_f32<0x141>(t);   // row_half_mirror
  if constexpr (L >= 16) t += dpp_f32<0x140>(t);  // row_mirror
  return t;
}

template <int L>
__global__ __launch_bounds__(256) void gg_prep_kernel(int mode, const void *src, const void *src2,
                                                      const int32_t *row_map, uint16_t *out,
                                                      uint16_t *out2, float *seeds, int rows,
                                                      int rows_pad, int K,
                                                      const int32_t *rows_dev) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (rows_dev) rows = *rows_dev;
  if (r >= rows) return;  // whole waves; no barriers here
  const int gw = 8 * L;   // columns per seed group
  size_t srow = (size_t)r;
  if (mode == 2 && row_map) srow = (size_t)row_map[r];
  for (int c0 = 0; c0 < K; c0 += 512) {
    const int c = c0 + 8 * lane;
    float t = 0.f;
    if (c < K) {
      if (mode <= 1) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t *>(
            reinterpret_cast<const uint16_t *>(src) + srow * K + c);
        t = sum8_bf16(v);
        if (mode == 1)
          t += sum8_bf16(*reinterpret_cast<const u32x4_t *>(
              reinterpret_cast<const uint16_t *>(src2) + srow * K + c));
      } else {
        const float *f = reinterpret_cast<const float *>(src) + srow * K + c;
        const f32x4_t a = *reinterpret_cast<const f32x4_t *>(f);
        const f32x4_t b = *reinterpret_cast<const f32x4_t *>(f + 4);
        if (mode == 2) {
          u32x4_t o;
          o.x = f32_to_bf16_rne(a.x) | (f32_to_bf16_rne(a.y) << 16);
          o.y = f32_to_bf16_rne(a.z) | (f32_to_bf16_rne(a.w) << 16);
          o.z = f32_to_bf16_rne(b.x) | (f32_to_bf16_rne(b.y) << 16);
          o.w = f32_to_bf16_rne(b.z) | (f32_to_bf16_rne(b.w) << 16);
          *reinterpret_cast<u32x4_t *>(out + (size_t)r * K + c) = o;
          t = sum8_bf16(o);
        } else {
          const u32x4_t hi = act_split_f32_nat(a, b, false), lo = act_split_f32_nat(a, b, true);
          *reinterpret_cast<u32x4_t *>(out + (size_t)r * K + c) = hi;
          *reinterpret_cast<u32x4_t *>(out2 + (size_t)r * K + c) = lo;
          t = sum8_bf16(hi) + sum8_bf16(lo);
        }
      }
    }
    t = lane_group_sum<L>(t);
    if ((lane & (L - 1)) == 0 && c < K) seeds[(size_t)(c / gw) * rows_pad + r] = -136.f * t;
  }
}

template <int MS, int NT, int WM, int WN, int GPK, bool HILO, bool SW>
hipError_t gg_launch(const GgArgs &a, dim3 grid, hipStream_t st) {
  if (a.sdt)
    hipLaunchKernelGGL((gg_kernel<MS, NT, WM, WN, GPK, HILO, SW, SCALE_F16>), grid,
                       dim3(64 * WM * WN), 0, st, a);
  else
    hipLaunchKernelGGL((gg_kernel<MS, NT, WM, WN, GPK, HILO, SW, SCALE_BF16>), grid,
                       dim3(64 * WM * WN), 0, st, a);
  return hipGetLastError();
}

template <int MS, int NT, int WM, int WN, bool HILO, bool SW>
hipError_t gg_launch_g(const GgArgs &a, dim3 grid, hipStream_t st) {
  switch (a.G == 32 ? 4 : a.G == 64 ? 2 : 1) {
    case 4: return gg_launch<MS, NT, WM, WN, 4, HILO, SW>(a, grid, st);
    case 2: return gg_launch<MS, NT, WM, WN, 2, HILO, SW>(a, grid, st);
    default: return gg_launch<MS, NT, WM, WN, 1, HILO, SW>(a, grid, st);
  }
}

// Dense tile shapes (rows x output columns): 128 x 256 (8 waves) in up to 4
// slices of K when the tiles alone leave CUs idle, else 128 x 128 or 64 x 128
// (4 waves) -- the choices prefill.hip measured.  Two-plane A: 64 x 256.
int gg_dense_ksplit(int M, int N, int K, int num_cus) {
  const long tiles = (long)((N + 255) / 256) * ((M + 127) / 128);
  const int KB = K / 128;
  for (int s = 1; s <= 4; ++s) {
    if (s > 1 && (KB / s < 6 || N % 4)) break;
    if (8 * tiles * s >= 7L * num_cus) return s;
  }
  return 0;
}

}  // namespace

bool gg_supported(int K, int G, int tiled) {
  return tiled && K % 128 == 0 && (G == 32 || G == 64 || G % 128 == 0) && K % G == 0;
}

int gg_rows_pad(int rows) { return (rows + 255) / 128 * 128; }

hipError_t gg_prep(int mode, const void *src, const void *src2, const int32_t *row_map,
                   uint16_t *out, uint16_t *out2, float *seeds, int rows, int rows_pad, int K,
                   int G, const int32_t *rows_dev, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  const dim3 grid((rows + 3) / 4), block(256);
  const int gw = gg_group_width(G);
  if (gw == 32)
    hipLaunchKernelGGL(gg_prep_kernel<4>, grid, block, 0, st, mode, src, src2, row_map, out, out2,
                       seeds, rows, rows_pad, K, rows_dev);
  else if (gw == 64)
    hipLaunchKernelGGL(gg_prep_kernel<8>, grid, block, 0, st, mode, src, src2, row_map, out, out2,
                       seeds, rows, rows_pad, K, rows_dev);
  else
    hipLaunchKernelGGL(gg_prep_kernel<16>, grid, block, 0, st, mode, src, src2, row_map, out,
                       out2, seeds, rows, rows_pad, K, rows_dev);
  return hipGetLastError();
}

namespace {
size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

size_t gg_dense_workspace(int M, int N, int K, int G, int amode, int epi, int num_cus) {
  const int gw = gg_group_width(G);
  size_t b = al256((size_t)(K / gw) * gg_rows_pad(M) * 4);
  if (amode == GG_A_F32) b += 2 * al256((size_t)M * K * 2);  // the A planes
  const int ks = (amode != GG_A_BF16 || epi == GG_SWIGLU_HILO) ? 1
                                                               : gg_dense_ksplit(M, N, K, num_cus);
  return b + (ks > 1 ? (size_t)ks * M * N * 4 : 0);
}

hipError_t gg_dense(GgArgs a, int amode, void *ws, int num_cus, hipStream_t st) {
  a.rows_pad = gg_rows_pad(a.M);
  a.seeds_out = nullptr;  // (the dense FFN's down makes its own seeds)
  a.row_map = nullptr;
  uint8_t *w = static_cast<uint8_t *>(ws);
  float *seeds = reinterpret_cast<float *>(w);
  a.seeds = seeds;
  w += al256((size_t)(a.K / gg_group_width(a.G)) * a.rows_pad * 4);
  a.tiles = nullptr;
  a.tile_split = 1;
  a.kper = a.K / 128;
  a.part = nullptr;
  a.hilo = amode != GG_A_BF16;
  const bool sw = a.epi == GG_SWIGLU_HILO;
  if (a.hilo) {
    if (amode == GG_A_F32) {
      uint16_t *hi = reinterpret_cast<uint16_t *>(w);
      uint16_t *lo = reinterpret_cast<uint16_t *>(w + al256((size_t)a.M * a.K * 2));
      if (hipError_t e = gg_prep(3, a.x, nullptr, nullptr, hi, lo, seeds, a.M, a.rows_pad, a.K,
                                 a.G, nullptr, st))
        return e;
      a.x = hi;
      a.x2 = lo;
    } else if (hipError_t e = gg_prep(1, a.x, a.x2, nullptr, nullptr, nullptr, seeds, a.M,
                                      a.rows_pad, a.K, a.G, nullptr, st)) {
      return e;
    }
    const dim3 grid((a.N + (sw ? 127 : 255)) / (sw ? 128 : 256), (a.M + 63) / 64, 1);
    if (sw) return gg_launch_g<2, 4, 2, 4, true, true>(a, grid, st);
    return gg_launch_g<2, 4, 2, 4, true, false>(a, grid, st);
  }
  if (hipError_t e = gg_prep(0, a.x, nullptr, nullptr, nullptr, nullptr, seeds, a.M, a.rows_pad,
                             a.K, a.G, nullptr, st))
    return e;
  if (sw)
    return gg_launch_g<4, 4, 2, 4, false, true>(a, dim3((a.N + 127) / 128, (a.M + 127) / 128, 1),
                                                st);
  const int ks = gg_dense_ksplit(a.M, a.N, a.K, num_cus);
  if (ks >= 1) {
    int nsl = 1;
    if (ks > 1) {
      a.kper = (a.K / 128 + ks - 1) / ks;
      nsl = (a.K / 128 + a.kper - 1) / a.kper;
      a.part = reinterpret_cast<float *>(w);
    }
    const dim3 grid((a.N + 255) / 256, (a.M + 127) / 128, nsl);
    if (hipError_t e = gg_launch_g<4, 4, 2, 4, false, false>(a, grid, st)) return e;
    if (nsl > 1) {
      const size_t n = (size_t)a.M * a.N;
      hipLaunchKernelGGL(gg_reduce_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0,
                         st, a.part, a.y, a.M, a.N, a.ldy, nsl, a.epi == GG_F32 ? 1 : 0);
      return hipGetLastError();
    }
    return hipSuccess;
  }
  const long tiles_mid = (long)((a.N + 127) / 128) * ((a.M + 127) / 128);
  if (tiles_mid >= num_cus)
    return gg_launch_g<4, 4, 2, 2, false, false>(a, dim3((a.N + 127) / 128, (a.M + 127) / 128, 1),
                                                 st);
  return gg_launch_g<2, 4, 2, 2, false, false>(a, dim3((a.N + 127) / 128, (a.M + 63) / 64, 1), st);
}

hipError_t gg_grouped(const GgArgs &a0, int max_tiles, hipStream_t st) {
  GgArgs a = a0;
  a.kper = a.K / 128;
  a.part = nullptr;
  if (max_tiles <= 0) return hipSuccess;
  const bool sw = a.epi == GG_SWIGLU_HILO;
  // the epilogue's seeds: SwiGLU only, groups of one, two or four waves' 32 columns
  if (a.seeds_out && (!sw || a.seeds_rp <= 0 ||
                      (a.seeds_gw != 32 && a.seeds_gw != 64 && a.seeds_gw != 128)))
    return hipErrorInvalidValue;
  // rows through a row map: one bf16 plane, x rows addressable in 31 bits
  if (a.row_map && (a.hilo || a.x_rows <= 0 || (size_t)a.x_rows * a.K * 2 > 0x7FFFFFFFu))
    return hipErrorInvalidValue;
  const unsigned gx = sw ? (a.N + 127) / 128 : (a.N + 255) / 256;
  if (a.hilo) {  // 64-row tiles: two per table entry
    a.tile_split = kGgChunkRows / 64;
    const dim3 grid(gx, max_tiles * a.tile_split, 1);
    if (sw) return gg_launch_g<2, 4, 2, 4, true, true>(a, grid, st);
    return gg_launch_g<2, 4, 2, 4, true, false>(a, grid, st);
  }
  a.tile_split = kGgChunkRows / 128;
  const dim3 grid(gx, max_tiles * a.tile_split, 1);
  if (sw) return gg_launch_g<4, 4, 2, 4, false, true>(a, grid, st);
  return gg_launch_g<4, 4, 2, 4, false, false>(a, grid, st);
}

}  // namespace cai4
