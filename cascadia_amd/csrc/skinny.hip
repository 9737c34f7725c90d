// skinny.hip -- decode-regime INT4 weight-only GEMM for gfx950 (M <= 64).
//
// y[t, r] = sum_g s[r, g] * sum_{c in g} (nibble[r, c] - 8) * x[t, c]
//
// The GPU counterpart of dequant_gemv_int4 / dequant_gemm_int4_multi_auto
// (crates/cascadia-int4-gemm/src/kernel_avx512.rs:209-297,
// kernel_avx512_multi.rs:66-245) and, with fused epilogues, of the
// gate/up -> SiLU*up -> down chain of expert_forward (kernel.rs:75-136).
//
// Work decomposition.  A workgroup owns a row block (16*NT weight rows; for
// the SwiGLU epilogue NT/2 gate tiles + NT/2 up tiles of the same output
// rows) and the whole K range; its WAVES waves each take a contiguous run of
// 128-column k-blocks.  Per k-block a lane loads 16 contiguous packed bytes
// (global_load_dwordx4) of one row: lanes 0-15 cover 16 rows, the 4 lane rows
// (lane/16) the four 16-byte chunks of the 64-byte k-block -- full 64-byte
// row segments per wave instruction.  Partial sums are reduced across waves
// through LDS in fixed wave order (deterministic; no atomics), then one wave
// applies the epilogue.
//
// k-slot mapping.  G % 128 == 0 ("contiguous"): MFMA step s of a k-block
// takes dword s of each lane's chunk; all 128 columns share one scale.
// Otherwise ("transposed", G = 32, 64, ...): the chunks are transposed across
// the four lane rows with v_permlane32_swap / v_permlane16_swap so that step
// s covers columns 32s..32s+31 of the block -- inside one group for any G
// that is a multiple of 32.  K must be a multiple of 32 (tails of a k-block
// are masked) and of G.
//
// Activations: bf16 (exact in the MFMA) or f32, split into hi + lo bf16
// halves that occupy token slots 0-7 and 8-15 of an M tile; y = D[hi] + D[lo].
#include "int4_common.hpp"
#include "skinny.hpp"

namespace cai4 {

template <int NT, int MT, bool XF32, bool TR>
CAI4_DEV void skinny_accumulate(const uint8_t *const (&brow)[NT],
                                const uint8_t *const (&srow)[NT], const bool (&rvalid)[NT],
                                const void *__restrict__ x, int ldx,
                                const int32_t *__restrict__ tok_list, int m0, int mcount,
                                int K, int G, int sdt, int kb0, int kb1,
                                f32x4_t (&acc)[MT][NT]) {
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  constexpr int TPM = XF32 ? 8 : 16;
  const u32x4_t B136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};

  const uint16_t *xb[MT];
  const float *xf[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int idx = mt * TPM + (XF32 ? (lr & 7) : lr);
    avalid[mt] = idx < mcount;
    const int tok = avalid[mt] ? (tok_list ? tok_list[m0 + idx] : m0 + idx) : 0;
    xb[mt] = reinterpret_cast<const uint16_t *>(x) + (size_t)tok * ldx;
    xf[mt] = reinterpret_cast<const float *>(x) + (size_t)tok * ldx;
  }
  const bool lo_half = XF32 && lr >= 8;

  for (int kb = kb0; kb < kb1; ++kb) {
    const int kbase = kb * 128;
    const int nsteps = TR ? min(4, (K - kbase) >> 5) : 4;

    // ---- weights: 16 B per lane per row tile
    u32x4_t b[NT];
    const bool cvalid = TR ? (lg < nsteps) : true;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (rvalid[nt] && cvalid)
        b[nt] = *reinterpret_cast<const u32x4_t *>(brow[nt] + (size_t)kb * 64 + 16 * lg);
      else
        b[nt] = u32x4_t{0u, 0u, 0u, 0u};
    }

    // ---- activation fragments, same k-slot order as decode8
    u32x4_t af[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int col = TR ? kbase + 32 * s + 8 * lg : kbase + 32 * lg + 8 * s;
        const bool ok = avalid[mt] && s < nsteps;
        if constexpr (XF32) {
          if (ok) {
            const f32x4_t v0 = *reinterpret_cast<const f32x4_t *>(xf[mt] + col);
            const f32x4_t v1 = *reinterpret_cast<const f32x4_t *>(xf[mt] + col + 4);
            af[mt][s] = act_split_f32(v0, v1, lo_half);
          } else {
            af[mt][s] = u32x4_t{0u, 0u, 0u, 0u};
          }
        } else {
          if (ok)
            af[mt][s] = act_perm_bf16(*reinterpret_cast<const u32x4_t *>(xb[mt] + col));
          else
            af[mt][s] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }

    if constexpr (!TR) {
      // one group for the whole k-block
      const int g = kbase / G;
      float sc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint32_t bits = reinterpret_cast<const uint16_t *>(srow[nt])[g];
        sc[nt] = sdt ? scale_to_f32<SCALE_F16>(bits) : scale_to_f32<SCALE_BF16>(bits);
      }
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
        const u32x4_t d0 = decode8(b[nt].x), d1 = decode8(b[nt].y);
        const u32x4_t d2 = decode8(b[nt].z), d3 = decode8(b[nt].w);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f32x4_t p = mfma_bf16(af[mt][0], d0, corr[mt]);
          p = mfma_bf16(af[mt][1], d1, p);
          p = mfma_bf16(af[mt][2], d2, p);
          p = mfma_bf16(af[mt][3], d3, p);
          acc[mt][nt] += sc[nt] * p;
        }
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b[nt] = xpose_rows(b[nt]);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if (s >= nsteps) break;
        const int g = (kbase + 32 * s) / G;
        f32x4_t corr[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) corr[mt] = mfma_bf16(af[mt][s], B136, zero4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t bits = reinterpret_cast<const uint16_t *>(srow[nt])[g];
          const float sc =
              sdt ? scale_to_f32<SCALE_F16>(bits) : scale_to_f32<SCALE_BF16>(bits);
          const uint32_t dw = s == 0 ? b[nt].x : s == 1 ? b[nt].y : s == 2 ? b[nt].z : b[nt].w;
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

// Up to 16 waves per workgroup; the MT = 4 tiles need the register file of
// a 4-wave workgroup (the planner keeps them at <= 4 waves).
template <int NT, int MT, bool XF32, bool TR, int EPI>
__global__ __launch_bounds__(MT >= 4 ? 256 : 1024) void skinny_kernel(SkinnyArgs a) {
  extern __shared__ f32x4_t red[];
  const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  constexpr int TPM = XF32 ? 8 : 16;
  constexpr bool SWIGLU = EPI == EPI_SWIGLU;
  constexpr int NOUT = SWIGLU ? NT / 2 : NT;

  const int out_row0 = blockIdx.x * 16 * NOUT;
  const int m0 = blockIdx.y * TPM * MT;
  const int mcount = min(a.M - m0, TPM * MT);
  const size_t row_bytes = (size_t)a.K / 2, srow_bytes = (size_t)(a.K / a.G) * 2;

  const uint8_t *brow[NT];
  const uint8_t *srow[NT];
  bool rvalid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const bool up = SWIGLU && nt >= NOUT;
    const int r = out_row0 + 16 * (up ? nt - NOUT : nt) + lr;
    rvalid[nt] = r < a.N;
    const size_t rr = rvalid[nt] ? (size_t)r : 0;
    brow[nt] = (up ? a.w1 : a.w0) + rr * row_bytes;
    srow[nt] = (up ? a.s1 : a.s0) + rr * srow_bytes;
  }

  const int kb_total = (a.K + 127) / 128;
  const int per = (kb_total + nw - 1) / nw;
  const int kb0 = min(wave * per, kb_total), kb1 = min(kb0 + per, kb_total);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (mcount > 0)
    skinny_accumulate<NT, MT, XF32, TR>(brow, srow, rvalid, a.x, a.ldx, nullptr, m0, mcount,
                                        a.K, a.G, a.sdt, kb0, kb1, acc);

  if (!wg_reduce<MT, NT>(acc, red)) return;
  if (mcount <= 0) return;
  if constexpr (XF32) {
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
          const float u = acc[mt][nt + NOUT][v];
          reinterpret_cast<float *>(a.out)[o] = silu_f32(y) * u;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host-side planning and dispatch
// ---------------------------------------------------------------------------

SkinnyPlan skinny_plan(int N, int K, int M, bool xf32, int epi, int num_cus) {
  SkinnyPlan p{};
  const int tpm = xf32 ? 8 : 16;
  int mt = (M + tpm - 1) / tpm;
  if (mt > 4) mt = 4;
  if (mt == 3) mt = 4;
  p.mt = mt;
  p.nt = (epi == EPI_SWIGLU) ? 2 : (mt >= 4 ? 2 : 2);
  const int nout = epi == EPI_SWIGLU ? p.nt / 2 : p.nt;
  p.row_blocks = (N + 16 * nout - 1) / (16 * nout);
  p.m_chunks = (M + tpm * mt - 1) / (tpm * mt);
  const int kb_total = (K + 127) / 128;
  const long target_waves = 16L * num_cus;
  long w = target_waves / ((long)p.row_blocks * p.m_chunks);
  int waves = 1;
  while (waves * 2 <= w && waves * 2 <= 16) waves *= 2;
  if (waves > kb_total) waves = kb_total < 1 ? 1 : kb_total;
  if (mt >= 4 && waves > 4) waves = 4;
  p.waves = waves;
  p.lds_bytes = (size_t)(waves - 1) * p.mt * p.nt * 64 * sizeof(f32x4_t);
  return p;
}

template <int NT, int MT, bool XF32, bool TR, int EPI>
static hipError_t launch_one(const SkinnyArgs &a, const SkinnyPlan &p, hipStream_t st) {
  dim3 grid(p.row_blocks, p.m_chunks, 1), block(64 * p.waves, 1, 1);
  hipLaunchKernelGGL((skinny_kernel<NT, MT, XF32, TR, EPI>), grid, block, p.lds_bytes, st, a);
  return hipGetLastError();
}

template <int NT, bool XF32, bool TR, int EPI>
static hipError_t launch_mt(const SkinnyArgs &a, const SkinnyPlan &p, hipStream_t st) {
  switch (p.mt) {
    case 1: return launch_one<NT, 1, XF32, TR, EPI>(a, p, st);
    case 2: return launch_one<NT, 2, XF32, TR, EPI>(a, p, st);
    default: return launch_one<NT, 4, XF32, TR, EPI>(a, p, st);
  }
}

template <bool XF32, bool TR>
static hipError_t launch_epi(const SkinnyArgs &a, const SkinnyPlan &p, int epi,
                             hipStream_t st) {
  switch (epi) {
    case EPI_F32: return launch_mt<2, XF32, TR, EPI_F32>(a, p, st);
    case EPI_BF16: return launch_mt<2, XF32, TR, EPI_BF16>(a, p, st);
    default: return launch_mt<2, XF32, TR, EPI_SWIGLU>(a, p, st);
  }
}

hipError_t skinny_launch(const SkinnyArgs &a, const SkinnyPlan &p, bool xf32, int epi,
                         hipStream_t st) {
  const bool tr = (a.G % 128) != 0;
  if (xf32)
    return tr ? launch_epi<true, true>(a, p, epi, st) : launch_epi<true, false>(a, p, epi, st);
  return tr ? launch_epi<false, true>(a, p, epi, st) : launch_epi<false, false>(a, p, epi, st);
}

}  // namespace cai4
