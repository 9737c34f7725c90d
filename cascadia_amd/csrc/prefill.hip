// prefill.hip -- INT4 weight-only GEMM for many tokens (prefill, M >= 64) on
// gfx950: bf16 activations [M, K], MFMA-tiled INT4 weights [N, K], f32
// accumulation, bf16 (RNE) or f32 output [M, N].
//
// The crate runs prefill as M GEMVs (kernel_avx512_multi.rs:240-244); the
// result per element is the same sum, y[t, r] = sum_g s[r, g] * sum_{c in g}
// (nibble - 8) * x[t, c], with products exact and f32 accumulation.
//
// Tiling.  A workgroup of 2 x NW waves computes a BM x 64 NW output tile; each
// wave a (BM / 2) x 64 sub-tile as 16 x 16 MFMA tiles.  K advances one
// 128-column k-block (one scale group, G a multiple of 128) per stage.
//
// Data movement.  Everything a stage needs -- the BM x 128 bf16 activation
// tile, the workgroup's 16-row weight tiles of the k-block (1 KB each in the
// MFMA-tiled layout) and their scales -- goes global -> LDS by buffer loads
// with an LDS destination (no registers; out-of-range rows read 0), two
// k-blocks ahead, into three static LDS stages.  Each stage: wait for this
// wave's loads of the stage (vmcnt), barrier (then every wave's have landed),
// issue the loads two stages ahead (into the buffer last read one stage ago,
// which the barrier has freed), then read the fragments and run the MFMAs.
// The loop is unrolled over the three buffers so each access names its own
// LDS array.
//
// Activation rows are stored 256 bytes apart with the 16-byte chunk index
// XOR-swizzled by the row (chunk q of row r at slot q ^ (r & 15)): a load
// instruction fills 1 KB of LDS in lane order, and the fragment reads of 16
// rows at one column hit 16 different bank groups.
//
// Arithmetic per k-block: each weight fragment is decoded once into bf16
// (128 + nibble) and used for every M sub-tile of the wave; one MFMA chain of
// the activations against the constant bf16 -136 seeds each 16 x 16 partial;
// the group scale is applied in f32, acc += s * p.
#include "int4_common.hpp"
#include "prefill.hpp"

namespace cai4 {

namespace {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kFlags = 0x00020000;

CAI4_DEV rsrc_t rsrc(const void *base, size_t bytes) {
  const int n = bytes > 0x7FFFFFFFu ? 0x7FFFFFFF : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, kFlags);
}

// Wait until at most n of this wave's vector-memory loads are outstanding,
// then barrier.  Inline asm with a memory clobber: neither the compiler's
// LDS reads nor the LDS-destination loads may move across it (the barrier
// builtin alone is no compiler memory barrier, and __syncthreads' fences
// would wait for every load in flight, the prefetch included).
template <int n>
CAI4_DEV void pf_wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(n) : "memory");
}

struct PfArgs {
  const uint8_t *w;   // MFMA-tiled packed weights
  const uint8_t *s;   // tiled scales [T][NG][16] u16
  const uint16_t *x;  // bf16 [M, K]
  void *y;            // [M, N] bf16 or f32
  int M, N, K, G, sdt, out_f32;
};

// LDS of one stage: activations [BM][256 B] swizzled, weight tiles [NT16][1 KB],
// scales [NT16][16] u16.
template <int BM, int NW>
struct Stage {
  static constexpr int NT16 = 4 * NW;  // 16-row weight tiles of the workgroup
  static constexpr int A = 0, B = BM * 256, S = B + NT16 * 1024, BYTES = S + NT16 * 32;
};

template <int BM, int NW>
struct Pf {
  static constexpr int MS = BM / 32;                      // 16-row sub-tiles per wave
  static constexpr int AI = BM * 256 / 1024 / (2 * NW);   // activation loads per wave per stage
  static constexpr int LOADS = AI + 2 + 1;                // + two weight tiles + the scales
};

// Issue wave `wave`'s loads of k-block kb into stage buffer `buf`.
template <int BM, int NW>
CAI4_DEV void pf_issue(uint8_t *buf, rsrc_t xr, rsrc_t wr, rsrc_t sr, int K, int KB, int NG,
                       int G, int kb, int wave, int lane) {
  using P = Pf<BM, NW>;
  using S = Stage<BM, NW>;
  // activations: load t fills LDS bytes [(wave AI + t) KB, +1 KB): rows
  // 4 (wave AI + t) + lane / 16, slot lane & 15 holding chunk slot ^ (row & 15)
#pragma unroll
  for (int t = 0; t < P::AI; ++t) {
    const int blk = wave * P::AI + t;
    const int row = 4 * blk + (lane >> 4);
    const int q = (lane & 15) ^ (row & 15);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *)(buf + S::A + blk * 1024), 16,
                                         (uint32_t)(row * K + kb * 128 + 8 * q) * 2, 0, 0, 0);
  }
  // weights: tiles 2 wave, 2 wave + 1 of the workgroup, 1 KB each in lane order
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int tile = 2 * wave + j;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void *)(buf + S::B + tile * 1024), 16,
                                         (uint32_t)(tile * KB + kb) * 1024 + 16 * lane, 0, 0, 0);
  }
  // scales of those two tiles: 2 x 32 bytes, four bytes from each of lanes
  // 0-15 (lane i writes LDS slot i: the other lanes must not run the load,
  // or their slots would overwrite the neighbouring waves' scales)
  const int g = (kb * 128) / G;
  const int tile = 2 * wave + ((lane >> 3) & 1);
  if (lane < 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void *)(buf + S::S + 2 * wave * 32), 4,
                                         (uint32_t)((tile * NG + g) * 16 * 2 + 4 * (lane & 7)),
                                         0, 0, 0);
}

template <int BM, int NW>
CAI4_DEV void pf_compute(const uint8_t *buf, int wm, int wn, int lane, int sdt,
                         f32x4_t (&acc)[BM / 32][4]) {
  using P = Pf<BM, NW>;
  using S = Stage<BM, NW>;
  const int lr = lane & 15, lg = lane >> 4;
  const u32x4_t B136 = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  u32x4_t af[P::MS][4];
#pragma unroll
  for (int i = 0; i < P::MS; ++i) {
    const int row = wm * (BM / 2) + 16 * i + lr;  // row & 15 == lr
#pragma unroll
    for (int s = 0; s < 4; ++s)
      af[i][s] = *reinterpret_cast<const u32x4_t *>(buf + S::A + row * 256 +
                                                    16 * ((4 * lg + s) ^ lr));
  }
  u32x4_t b[4];
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tile = 4 * wn + j;
    b[j] = *reinterpret_cast<const u32x4_t *>(buf + S::B + tile * 1024 + 16 * lane);
    const uint32_t bits = *reinterpret_cast<const uint16_t *>(buf + S::S + tile * 32 + 2 * lr);
    sc[j] = sdt ? scale_to_f32<SCALE_F16>(bits) : scale_to_f32<SCALE_BF16>(bits);
  }
  f32x4_t corr[P::MS];
#pragma unroll
  for (int i = 0; i < P::MS; ++i) {
    corr[i] = mfma_bf16(af[i][0], B136, zero4);
    corr[i] = mfma_bf16(af[i][1], B136, corr[i]);
    corr[i] = mfma_bf16(af[i][2], B136, corr[i]);
    corr[i] = mfma_bf16(af[i][3], B136, corr[i]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4_t d0 = decode8(b[j].x), d1 = decode8(b[j].y);
    const u32x4_t d2 = decode8(b[j].z), d3 = decode8(b[j].w);
#pragma unroll
    for (int i = 0; i < P::MS; ++i) {
      f32x4_t p = mfma_bf16(af[i][0], d0, corr[i]);
      p = mfma_bf16(af[i][1], d1, p);
      p = mfma_bf16(af[i][2], d2, p);
      p = mfma_bf16(af[i][3], d3, p);
      acc[i][j] += sc[j] * p;
    }
  }
}

// One stage: k-block kb from `cur`; the loads of kb + 2 go into `nxt2`.
template <int BM, int NW>
CAI4_DEV void pf_stage(uint8_t *cur, uint8_t *nxt2, rsrc_t xr, rsrc_t wr, rsrc_t sr,
                       const PfArgs &a, int KB, int NG, int kb, int wave, int wm, int wn,
                       int lane, f32x4_t (&acc)[BM / 32][4]) {
  using P = Pf<BM, NW>;
  if (kb >= KB) return;  // uniform
  // this wave's loads of kb are done once only kb + 1's may still be in
  // flight; after the barrier every wave's have landed
  if (kb + 1 < KB)
    pf_wait_barrier<P::LOADS>();
  else
    pf_wait_barrier<0>();
  if (kb + 2 < KB) pf_issue<BM, NW>(nxt2, xr, wr, sr, a.K, KB, NG, a.G, kb + 2, wave, lane);
  pf_compute<BM, NW>(cur, wm, wn, lane, a.sdt, acc);
}

template <int BM, int NW>
__global__ __launch_bounds__(128 * NW) void pf_gemm_kernel(PfArgs a) {
  using P = Pf<BM, NW>;
  using S = Stage<BM, NW>;
  __shared__ __attribute__((aligned(16))) uint8_t st0[S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t st1[S::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t st2[S::BYTES];
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  // wave index as a scalar: descriptors built from it must be uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * 64 * NW;
  const int KB = a.K >> 7, NG = a.K / a.G;
  const int ntiles = (a.N + 15) >> 4;
  const int T0 = n0 >> 4;
  const int tv =
      __builtin_amdgcn_readfirstlane(ntiles - T0 > S::NT16 ? S::NT16 : ntiles - T0);
  const rsrc_t wr = rsrc(a.w + (size_t)T0 * KB * 1024, (size_t)tv * KB * 1024);
  const rsrc_t sr = rsrc(a.s + (size_t)T0 * NG * 32, (size_t)tv * NG * 32);
  const rsrc_t xr = rsrc(a.x + (size_t)m0 * a.K, (size_t)(a.M - m0) * a.K * 2);

  f32x4_t acc[P::MS][4];
#pragma unroll
  for (int i = 0; i < P::MS; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  pf_issue<BM, NW>(st0, xr, wr, sr, a.K, KB, NG, a.G, 0, wave, lane);
  if (KB > 1) pf_issue<BM, NW>(st1, xr, wr, sr, a.K, KB, NG, a.G, 1, wave, lane);
  for (int kb = 0; kb < KB; kb += 3) {
    pf_stage<BM, NW>(st0, st2, xr, wr, sr, a, KB, NG, kb, wave, wm, wn, lane, acc);
    pf_stage<BM, NW>(st1, st0, xr, wr, sr, a, KB, NG, kb + 1, wave, wm, wn, lane, acc);
    pf_stage<BM, NW>(st2, st1, xr, wr, sr, a, KB, NG, kb + 2, wave, wm, wn, lane, acc);
  }

  // epilogue: D lane l holds column l % 16 and rows 4 * (l / 16) + v
#pragma unroll
  for (int i = 0; i < P::MS; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + lr;
      if (n >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * (BM / 2) + 16 * i + 4 * lg + v;
        if (m >= a.M) continue;
        const size_t o = (size_t)m * a.N + n;
        if (a.out_f32)
          reinterpret_cast<float *>(a.y)[o] = acc[i][j][v];
        else
          reinterpret_cast<uint16_t *>(a.y)[o] = (uint16_t)f32_to_bf16_rne(acc[i][j][v]);
      }
    }
  }
}

}  // namespace

bool prefill_supported(int M, int N, int K, int G, int tiled) {
  return tiled && M >= 64 && K % 128 == 0 && G % 128 == 0 && N >= 16;
}

hipError_t prefill_gemm(const uint8_t *w, const uint8_t *s, const uint16_t *x, void *y, int M,
                        int N, int K, int G, int sdt, int out_f32, int num_cus, hipStream_t st) {
  PfArgs a{w, s, x, y, M, N, K, G, sdt, out_f32};
  const long tiles_big = (long)((N + 255) / 256) * ((M + 127) / 128);
  const long tiles_mid = (long)((N + 127) / 128) * ((M + 127) / 128);
  if (tiles_big >= num_cus) {  // 128 x 256 tiles, 8 waves
    hipLaunchKernelGGL((pf_gemm_kernel<128, 4>), dim3((N + 255) / 256, (M + 127) / 128),
                       dim3(512), 0, st, a);
  } else if (tiles_mid >= num_cus) {  // 128 x 128 tiles, 4 waves
    hipLaunchKernelGGL((pf_gemm_kernel<128, 2>), dim3((N + 127) / 128, (M + 127) / 128),
                       dim3(256), 0, st, a);
  } else {  // 64 x 128 tiles
    hipLaunchKernelGGL((pf_gemm_kernel<64, 2>), dim3((N + 127) / 128, (M + 63) / 64), dim3(256),
                       0, st, a);
  }
  return hipGetLastError();
}

}  // namespace cai4
