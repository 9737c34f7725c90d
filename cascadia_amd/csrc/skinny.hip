// skinny.hip -- decode-regime INT4 weight-only GEMM for gfx950 (M <= 64 per
// pass; larger M loops over M chunks).
//
// y[t, r] = sum_g s[r, g] * sum_{c in g} (nibble[r, c] - 8) * x[t, c]
//
// The GPU counterpart of dequant_gemv_int4 / dequant_gemm_int4_multi_auto
// (crates/cascadia-int4-gemm/src/kernel_avx512.rs:209-297,
// kernel_avx512_multi.rs:66-245) and, with fused epilogues, of the
// gate/up -> SiLU*up -> down chain of expert_forward (kernel.rs:75-136).
//
// Work decomposition.  A workgroup owns a row block (16*NT weight rows; for
// the SwiGLU epilogues one gate tile + one up tile of the same 16 output
// rows) and the whole K range; its waves each take a contiguous run of
// 128-column k-blocks.  Per k-block a lane loads 16 packed bytes of one row
// (lanes 0-15: 16 rows; lane row lane/16: the 16-byte chunk of the 64-byte
// k-block).  Weights, scales and activations of U consecutive k-blocks are in
// flight per wave (a register ring).  All loads are buffer loads: the
// resource descriptor (SGPRs) spans exactly the valid bytes, so rows past N,
// tokens past M, tail chunks and prefetches past the wave's range read 0
// from the hardware range check instead of being clamped, and per-lane
// offsets are 32-bit constants.  Partial sums are reduced across waves
// through LDS in fixed wave order (deterministic; no atomics), then wave 0
// applies the epilogue.
//
// Weight layouts.  CRATE (the crate's row-major bytes) or TILED (layout.hip:
// each 16-row x 128-column block is 1 KB contiguous in lane order, nibbles
// of a dword swizzled so that the decode yields natural column order).
//
// k-slot mapping.  G % 128 == 0 ("contiguous"): MFMA step s of a k-block
// takes dword s of each lane's chunk; all 128 columns share one scale.
// Otherwise ("transposed", G = 32, 64, ...): the chunks are transposed across
// the four lane rows with v_permlane32_swap / v_permlane16_swap so that step
// s covers columns 32s..32s+31 of the block -- inside one group for any G
// that is a multiple of 32.  K must be a multiple of 32 and of G.
//
// Activation modes (token slots of a 16-slot M tile):
//   A_BF16: slot i = token i, bf16 (exact in the MFMA);
//   A_XF32: f32 activations split in-kernel into hi (truncated bf16) and lo
//           (bf16 of the exact remainder): slots 0-7 hi, 8-15 lo of tokens
//           0-7; y = D[hi] + D[lo];
//   A_HILO: the same split, precomputed as two bf16 planes (x and x2; the
//           SwiGLU intermediate is written that way by the gate/up epilogue).
#include <stdlib.h>

#include "int4_common.hpp"
#include "skinny.hpp"

namespace cai4 {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcFlags = 0x00020000;  // gfx9 raw buffer: 32-bit data format
constexpr uint32_t kOOB = 0x80000000u;  // an offset past every descriptor's range

CAI4_DEV rsrc_t make_rsrc(const void *base, size_t bytes) {
  const int n = bytes > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, kRsrcFlags);
}

template <int AM>
struct AModeTraits {
  static constexpr int TPM = AM == A_BF16 ? 16 : 8;  // tokens per M tile
  static constexpr int NA = AM == A_XF32 ? 2 : 1;    // 16-byte loads per step
  static constexpr int ESZ = AM == A_XF32 ? 4 : 2;   // activation element bytes
};

// One k-block of a wave: weights, scales and activations.
template <int NT, int MT, int AM, bool TR>
struct Stage {
  u32x4_t b[NT];
  uint32_t sb[NT][TR ? 4 : 1];
  u32x4_t a[MT][4][AModeTraits<AM>::NA];
};

template <int NT, int MT>
struct WaveSrc {
  rsrc_t wr[NT], sr[NT], ar;
  uint32_t wv[NT], sv[NT], av[MT];  // per-lane byte offsets
  uint32_t wk, sk;                  // bytes per k-block (weights), per group (scales)
};

// 8 consecutive f32 -> hi / lo bf16 in natural order.
CAI4_DEV u32x4_t act_split_f32_nat(const f32x4_t &a, const f32x4_t &b, bool lo) {
  const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float x0 = xs[2 * p], x1 = xs[2 * p + 1];
    if (!lo) {
      w[p] = __builtin_amdgcn_perm(fbits(x1), fbits(x0), 0x07060302u);
    } else {
      const float r0 = x0 - bitsf(fbits(x0) & 0xFFFF0000u);
      const float r1 = x1 - bitsf(fbits(x1) & 0xFFFF0000u);
      f32x2_t v = {r0, r1};
      w[p] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    }
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

template <int NT, int MT, int AM, bool TR>
CAI4_DEV void load_stage(Stage<NT, MT, AM, TR> &S, const WaveSrc<NT, MT> &W, int kb, int G,
                         int glog2) {
  const int kbase = kb * 128;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    S.b[nt] = __builtin_amdgcn_raw_buffer_load_b128(W.wr[nt], W.wv[nt], kb * W.wk, 0);
    if constexpr (TR) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int col = kbase + 32 * s;
        const int g = glog2 >= 0 ? (col >> glog2) : col / G;
        S.sb[nt][s] = __builtin_amdgcn_raw_buffer_load_b16(W.sr[nt], W.sv[nt], g * W.sk, 0);
      }
    } else {
      const int g = glog2 >= 0 ? (kbase >> glog2) : kbase / G;
      S.sb[nt][0] = __builtin_amdgcn_raw_buffer_load_b16(W.sr[nt], W.sv[nt], g * W.sk, 0);
    }
  }
  constexpr int ESZ = AModeTraits<AM>::ESZ;
  const int ks = kbase * ESZ;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // step s sits at a constant column offset from the lane's first column
      const uint32_t off = W.av[mt] + (TR ? 32 * s : 8 * s) * ESZ;
      S.a[mt][s][0] = __builtin_amdgcn_raw_buffer_load_b128(W.ar, off, ks, 0);
      if constexpr (AM == A_XF32)
        S.a[mt][s][1] = __builtin_amdgcn_raw_buffer_load_b128(W.ar, off + 16, ks, 0);
    }
  }
}

template <int AM, bool TILED>
CAI4_DEV u32x4_t act_fragment(const u32x4_t (&r)[AModeTraits<AM>::NA], bool lo_half) {
  if constexpr (AM == A_XF32) {
    const f32x4_t a = __builtin_bit_cast(f32x4_t, r[0]), b = __builtin_bit_cast(f32x4_t, r[1]);
    return TILED ? act_split_f32_nat(a, b, lo_half) : act_split_f32(a, b, lo_half);
  } else {
    return TILED ? r[0] : act_perm_bf16(r[0]);
  }
}

// MFMAs of one k-block.
template <int NT, int MT, int AM, bool TR, bool TILED>
CAI4_DEV void compute_stage(Stage<NT, MT, AM, TR> &S, int kb, int K, int sdt, bool lo_half,
                            f32x4_t (&acc)[MT][NT]) {
  const u32x4_t B136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  u32x4_t af[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < 4; ++s) af[mt][s] = act_fragment<AM, TILED>(S.a[mt][s], lo_half);
  if constexpr (!TR) {
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
      const float sc =
          sdt ? scale_to_f32<SCALE_F16>(S.sb[nt][0]) : scale_to_f32<SCALE_BF16>(S.sb[nt][0]);
      const u32x4_t d0 = decode8(S.b[nt].x), d1 = decode8(S.b[nt].y);
      const u32x4_t d2 = decode8(S.b[nt].z), d3 = decode8(S.b[nt].w);
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
    const int nsteps = min(4, (K - kb * 128) >> 5);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) S.b[nt] = xpose_rows(S.b[nt]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s >= nsteps) break;
      f32x4_t corr[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) corr[mt] = mfma_bf16(af[mt][s], B136, zero4);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float sc = sdt ? scale_to_f32<SCALE_F16>(S.sb[nt][s])
                             : scale_to_f32<SCALE_BF16>(S.sb[nt][s]);
        const uint32_t dw =
            s == 0 ? S.b[nt].x : s == 1 ? S.b[nt].y : s == 2 ? S.b[nt].z : S.b[nt].w;
        const u32x4_t d = decode8(dw);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x4_t p = mfma_bf16(af[mt][s], d, corr[mt]);
          acc[mt][nt] += sc * p;
        }
      }
    }
  }
}

// One wave's k-blocks [kb0, kb1) through a U-deep register ring.
template <int NT, int MT, int AM, bool TR, bool TILED, int U>
CAI4_DEV void skinny_accumulate(const WaveSrc<NT, MT> &W, int K, int G, int glog2, int sdt,
                                int kb0, int kb1, f32x4_t (&acc)[MT][NT]) {
  const bool lo_half = AM != A_BF16 && (threadIdx.x & 15) >= 8;
  Stage<NT, MT, AM, TR> ring[U];
#pragma unroll
  for (int u = 0; u < U; ++u) load_stage<NT, MT, AM, TR>(ring[u], W, kb0 + u, G, glog2);
  for (int kb = kb0; kb < kb1; kb += U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kb + u;
      if (k < kb1) {
        compute_stage<NT, MT, AM, TR, TILED>(ring[u], k, K, sdt, lo_half, acc);
        // past kb1 this prefetch reads other valid bytes or 0; never consumed
        load_stage<NT, MT, AM, TR>(ring[u], W, k + U, G, glog2);
      }
    }
  }
}

// Sum the per-wave accumulators of a workgroup in wave order through LDS.
// Returns true in wave 0, which then holds the totals.
template <int MT, int NT>
CAI4_DEV bool wg_reduce(f32x4_t (&acc)[MT][NT], f32x4_t *red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  constexpr int NI = MT * NT;
  if (nw > 1) {
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          red[((size_t)(wave - 1) * NI + mt * NT + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (wave != 0) return false;
    for (int w = 1; w < nw; ++w) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] += red[((size_t)(w - 1) * NI + mt * NT + nt) * 64 + lane];
    }
  }
  return true;
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

// Threads per workgroup the register file allows for an M-tile count.
constexpr int skinny_max_threads(int mt) { return mt >= 4 ? 256 : (mt == 2 ? 512 : 1024); }

template <int NT, int MT, int AM, bool TR, bool TILED, int EPI, int U>
__global__ __launch_bounds__(skinny_max_threads(MT)) void skinny_kernel(SkinnyArgs a) {
  extern __shared__ f32x4_t red[];
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  constexpr int TPM = AModeTraits<AM>::TPM;
  constexpr int ESZ = AModeTraits<AM>::ESZ;
  constexpr bool SWIGLU = EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_HILO;
  constexpr int NOUT = SWIGLU ? NT / 2 : NT;

  const int out_row0 = blockIdx.x * 16 * NOUT;
  const int m0 = blockIdx.y * TPM * MT;
  const int mcount = min(a.M - m0, TPM * MT);
  const int kb_total = (a.K + 127) / 128;
  const int ngroups = a.K / a.G;

  WaveSrc<NT, MT> W;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const bool up = SWIGLU && nt >= NOUT;
    const int r0 = out_row0 + 16 * (up ? nt - NOUT : nt);  // the tile's first row (uniform)
    const uint8_t *wb = up ? a.w1 : a.w0;
    const uint8_t *sb = up ? a.s1 : a.s0;
    const size_t rows_left = r0 < a.N ? (size_t)(a.N - r0) : 0;
    if (TILED) {
      const size_t T = (size_t)(r0 >> 4);
      const bool live = rows_left > 0;
      W.wr[nt] = make_rsrc(wb + T * kb_total * 1024, live ? (size_t)kb_total * 1024 : 0);
      W.sr[nt] = make_rsrc(sb + T * ngroups * 32, live ? (size_t)ngroups * 32 : 0);
      W.wv[nt] = 16 * lane;
      W.sv[nt] = 2 * lr;
    } else {
      const size_t rb = (size_t)a.K / 2;
      W.wr[nt] = make_rsrc(wb + (size_t)r0 * rb, rows_left * rb);
      W.sr[nt] = make_rsrc(sb + (size_t)r0 * ngroups * 2, rows_left * ngroups * 2);
      W.wv[nt] = lr * (uint32_t)rb + 16 * lg;
      W.sv[nt] = lr * (uint32_t)ngroups * 2;
    }
  }
  W.wk = TILED ? 1024 : 64;
  W.sk = TILED ? 32 : 2;
  // activations: one descriptor over [x, x + M rows) (both planes for A_HILO)
  {
    const size_t plane = (size_t)a.M * a.ldx * ESZ;
    const size_t gap =
        AM == A_HILO ? (size_t)((const uint8_t *)a.x2 - (const uint8_t *)a.x) : (size_t)0;
    W.ar = make_rsrc(a.x, gap + plane);
    const uint32_t plane_off = (AM == A_HILO && lr >= 8) ? (uint32_t)gap : 0u;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int idx = mt * TPM + (AM == A_BF16 ? lr : (lr & 7));
      const int col0 = TR ? 8 * lg : 32 * lg;
      W.av[mt] = idx < mcount
                     ? plane_off + (uint32_t)(((size_t)(m0 + idx) * a.ldx + col0) * ESZ)
                     : kOOB;  // past M: reads 0, never stored
    }
  }

  const int per = (kb_total + nw - 1) / nw;
  const int kb0 = min(wave * per, kb_total), kb1 = min(kb0 + per, kb_total);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (mcount > 0 && kb0 < kb1)
    skinny_accumulate<NT, MT, AM, TR, TILED, U>(W, a.K, a.G, a.glog2, a.sdt, kb0, kb1, acc);

  if (!wg_reduce<MT, NT>(acc, red)) return;
  if (mcount <= 0) return;
  if constexpr (AM != A_BF16) {
    fold_hilo<MT, NT>(acc);
    if (lg >= 2) return;
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NOUT; ++nt) {
      const int row = out_row0 + 16 * nt + lr;
      if (row >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int ti = mt * TPM + 4 * lg + v;
        if (ti >= mcount) continue;
        const size_t o = (size_t)(m0 + ti) * a.ldo + row;
        const float y = acc[mt][nt][v];
        if constexpr (EPI == EPI_F32) {
          reinterpret_cast<float *>(a.out)[o] = y;
        } else if constexpr (EPI == EPI_BF16) {
          reinterpret_cast<uint16_t *>(a.out)[o] = (uint16_t)f32_to_bf16_rne(y);
        } else {
          const float h = silu_f32(y) * acc[mt][nt + NOUT][v];
          if constexpr (EPI == EPI_SWIGLU) {
            reinterpret_cast<float *>(a.out)[o] = h;
          } else {
            // hi = h truncated to bf16, lo = bf16(h - hi): the A_HILO planes
            const uint32_t hb = fbits(h) >> 16;
            const float lo = h - bitsf(hb << 16);
            reinterpret_cast<uint16_t *>(a.out)[o] = (uint16_t)hb;
            reinterpret_cast<uint16_t *>(a.out2)[o] = (uint16_t)f32_to_bf16_rne(lo);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host-side planning and dispatch
// ---------------------------------------------------------------------------

// k-blocks in flight per wave (register ring depth), chosen so that MT = 1
// stays within 128 VGPRs (4 waves per SIMD).
constexpr int skinny_ring_depth(int nt, int mt, int am, bool tr) {
  return mt == 1 ? ((am == A_XF32 || tr) ? 2 : (nt == 1 ? 4 : 3)) : 2;
}

SkinnyPlan skinny_plan(int N, int K, int M, int amode, int epi, int num_cus) {
  SkinnyPlan p{};
  const int tpm = amode == A_BF16 ? 16 : 8;
  int mt = (M + tpm - 1) / tpm;
  if (mt > 4) mt = 4;
  if (mt == 3) mt = 4;
  if (amode == A_XF32 && mt > 2) mt = 2;  // f32 activations: at most 16 tokens per pass
  p.mt = mt;
  p.m_chunks = (M + tpm * mt - 1) / (tpm * mt);
  const bool swiglu = epi == EPI_SWIGLU || epi == EPI_SWIGLU_HILO;
  const int kb_total = (K + 127) / 128;
  const int maxw = (mt >= 4 ? 256 : (mt == 2 ? 512 : 1024)) / 64;
  // aim for ~4 resident waves per SIMD across the chip
  const long target = 16L * num_cus;
  auto rows_per_block = [&](int nt) { return 16 * (swiglu ? nt / 2 : nt); };
  p.nt = 2;
  if (!swiglu) {
    const long rb2 = (N + 31) / 32;
    if (rb2 * p.m_chunks * maxw < target) p.nt = 1;  // too few row blocks: halve them
  }
  p.row_blocks = (N + rows_per_block(p.nt) - 1) / rows_per_block(p.nt);
  long w = target / ((long)p.row_blocks * p.m_chunks);  // never beyond one resident round
  int waves = (int)(w < 1 ? 1 : (w > maxw ? maxw : w));
  // tuning override: CASCADIA_INT4_SKINNY_WAVES=<1..16>
  if (const char *ev = getenv("CASCADIA_INT4_SKINNY_WAVES")) {
    const int v = atoi(ev);
    if (v >= 1 && v <= 16) waves = v;
  }
  if (waves > maxw) waves = maxw;
  if (waves > kb_total) waves = kb_total < 1 ? 1 : kb_total;
  p.waves = waves;
  p.lds_bytes = (size_t)(waves - 1) * p.mt * p.nt * 64 * sizeof(f32x4_t);
  return p;
}

template <int NT, int MT, int AM, bool TR, bool TILED, int EPI>
static hipError_t launch_one(const SkinnyArgs &a, const SkinnyPlan &p, hipStream_t st) {
  dim3 grid(p.row_blocks, p.m_chunks, 1), block(64 * p.waves, 1, 1);
  constexpr int U = skinny_ring_depth(NT, MT, AM, TR);
  hipLaunchKernelGGL((skinny_kernel<NT, MT, AM, TR, TILED, EPI, U>), grid, block, p.lds_bytes, st,
                     a);
  return hipGetLastError();
}

template <int AM, bool TR, bool TILED, int EPI>
static hipError_t launch_mt(const SkinnyArgs &a, const SkinnyPlan &p, hipStream_t st) {
  constexpr bool SW = EPI == EPI_SWIGLU || EPI == EPI_SWIGLU_HILO;
  if constexpr (!SW) {
    if (p.nt == 1) {
      if (p.mt == 1) return launch_one<1, 1, AM, TR, TILED, EPI>(a, p, st);
      if constexpr (AM == A_XF32) return launch_one<1, 2, AM, TR, TILED, EPI>(a, p, st);
      if (p.mt == 2) return launch_one<1, 2, AM, TR, TILED, EPI>(a, p, st);
      if constexpr (AM != A_XF32) return launch_one<1, 4, AM, TR, TILED, EPI>(a, p, st);
    }
  }
  if (p.mt == 1) return launch_one<2, 1, AM, TR, TILED, EPI>(a, p, st);
  if constexpr (AM == A_XF32) return launch_one<2, 2, AM, TR, TILED, EPI>(a, p, st);
  if (p.mt == 2) return launch_one<2, 2, AM, TR, TILED, EPI>(a, p, st);
  if constexpr (AM != A_XF32) return launch_one<2, 4, AM, TR, TILED, EPI>(a, p, st);
  return hipErrorInvalidValue;
}

template <int AM, bool TR, bool TILED>
static hipError_t launch_epi(const SkinnyArgs &a, const SkinnyPlan &p, int epi,
                             hipStream_t st) {
  switch (epi) {
    case EPI_F32: return launch_mt<AM, TR, TILED, EPI_F32>(a, p, st);
    case EPI_BF16: return launch_mt<AM, TR, TILED, EPI_BF16>(a, p, st);
    case EPI_SWIGLU: return launch_mt<AM, TR, TILED, EPI_SWIGLU>(a, p, st);
    default: return launch_mt<AM, TR, TILED, EPI_SWIGLU_HILO>(a, p, st);
  }
}

template <int AM>
static hipError_t launch_tr(const SkinnyArgs &a, const SkinnyPlan &p, int epi, hipStream_t st) {
  const bool tr = (a.G % 128) != 0;
  if (a.tiled)
    return tr ? launch_epi<AM, true, true>(a, p, epi, st)
              : launch_epi<AM, false, true>(a, p, epi, st);
  return tr ? launch_epi<AM, true, false>(a, p, epi, st)
            : launch_epi<AM, false, false>(a, p, epi, st);
}

hipError_t skinny_launch(const SkinnyArgs &a, const SkinnyPlan &p, int amode, int epi,
                         hipStream_t st) {
  switch (amode) {
    case A_BF16: return launch_tr<A_BF16>(a, p, epi, st);
    case A_XF32: return launch_tr<A_XF32>(a, p, epi, st);
    default: return launch_tr<A_HILO>(a, p, epi, st);
  }
}

}  // namespace cai4
