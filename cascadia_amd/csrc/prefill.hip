// prefill.hip -- INT4 weight-only GEMM for many tokens (prefill, M >= 64) on
// gfx950: bf16 activations [M, K], MFMA-tiled INT4 weights [N, K], f32
// accumulation, bf16 (RNE) or f32 output [M, N].
//
// The crate runs prefill as M GEMVs (kernel_avx512_multi.rs:240-244); the
// result per element is the same sum, y[t, r] = sum_g s[r, g] * sum_{c in g}
// (nibble - 8) * x[t, c], with products exact and f32 accumulation.
//
// Arithmetic.  Weights enter the MFMAs as the bf16 value 128 + nibble; the
// offset 136 (128 + the zero point 8) is removed by seeding each k-block's
// partial with xs = -136 * sum(x) over the block's 128 columns, which a
// pre-pass computes once per (row, k-block) in f32; the group scale is applied
// in f32 per k-block, acc += s * p.  (G is a multiple of 128, so a k-block
// lies in one group.)
//
// Tiling.  A workgroup of WM x WN waves computes a 16 MS WM x 16 NT WN output
// tile, each wave a 16 MS x 16 NT sub-tile as 16 x 16 MFMA tiles.  K advances
// one 128-column k-block per stage, in four 32-column steps: a step's
// activation fragments are read from LDS one step ahead, so the MFMAs of a
// step never wait on LDS; each decoded weight fragment serves MS MFMAs.
//
// Data movement.  Everything a stage needs -- the BM x 128 bf16 activation
// tile, the workgroup's 16-row weight tiles of the k-block (1 KB each in the
// MFMA-tiled layout), their scales and the BM seeds -- goes global -> LDS by
// buffer loads with an LDS destination (no registers; out-of-range rows read
// 0), two k-blocks ahead, into three static LDS stages.  Each stage: wait for
// this wave's loads of the stage (vmcnt), barrier (then every wave's have
// landed), then the four steps, issuing the loads two stages ahead in eight
// parts over the steps (into the buffer read one stage ago, which the barrier
// has freed).  The loop is unrolled over the three buffers so each access
// names its own LDS array.  (Measured on gfx950: an LDS-destination load costs
// the LDS several times what a ds_write_b128 of the same bytes does, but
// staging through registers leaves too few of them for a two-stage lead with
// this wave tile, and was slower.)
//
// Activation rows are stored 256 bytes apart with the 16-byte chunk index
// XOR-swizzled by the row (chunk q of row r at slot q ^ (r & 15)): a load
// instruction fills 1 KB of LDS in lane order, and the fragment reads of 16
// rows at one column hit 16 different bank groups.
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

// The LDS address (M0) of an LDS pointer, as a wave-uniform scalar.
CAI4_DEV uint32_t lds_addr(const uint8_t *p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)p);
}

// One global -> LDS buffer load of `bytes` (16 or 4) per lane; lane i's data
// lands at M0 + bytes * i.  Written as asm: the compiler cannot tell the stage
// buffers apart, and would make every later LDS read of any stage wait for
// this load (the prefetch two stages ahead) to land.  The stage waits count
// these loads themselves.
template <int bytes>
CAI4_DEV void pf_dma(rsrc_t r, uint32_t lds, uint32_t voff) {
  if constexpr (bytes == 16)
    asm volatile("buffer_load_dwordx4 %1, %2, 0 offen lds" ::"{m0}"(lds), "v"(voff), "s"(r)
                 : "memory");
  else
    asm volatile("buffer_load_dword %1, %2, 0 offen lds" ::"{m0}"(lds), "v"(voff), "s"(r)
                 : "memory");
}

struct PfArgs {
  const uint8_t *w;   // MFMA-tiled packed weights
  const uint8_t *s;   // tiled scales [T][NG][16] u16
  const uint16_t *x;  // bf16 [M, K]
  const float *xs;    // seeds [KB][Mp]: -136 * sum of x over each k-block
  void *y;            // [M, N] bf16 or f32
  int M, N, K, G, sdt, out_f32, Mp;
  int kper;           // k-blocks per workgroup slice of K (blockIdx.z)
  float *part;        // ksplit > 1: f32 partial sums [ksplit][M][N], else null
};

// Seeds: xs[kb][m] = -136 * sum_{c < 128} x[m, 128 kb + c] (f32, fixed order:
// eight columns per lane, then the 16 lanes of a DPP row, which hold one
// k-block); rows M .. Mp - 1 are 0.  One wave per row and kPfXsumPasses passes
// of four k-blocks (blockIdx.y: which), all loads issued before summing: the
// pass is latency-bound, so it is spread over as many waves as possible.
constexpr int kPfXsumPasses = 2;

template <int CTRL>
CAI4_DEV float dpp_row_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__global__ __launch_bounds__(256) void pf_xsum_kernel(const uint16_t *x, float *xs, int M, int K,
                                                      int Mp) {
  constexpr int P = kPfXsumPasses;
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= Mp) return;
  const int KB = K >> 7, p0 = blockIdx.y * P;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(x + (size_t)(m < M ? m : 0) * K), (short)0, m < M ? K * 2 : 0,
      0x00020000);
  u32x4_t v[P];
#pragma unroll
  for (int q = 0; q < P; ++q)  // columns 512 (p0 + q) + 8 lane; past K reads 0
    v[q] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                           xr, (uint32_t)(512 * (p0 + q) + 8 * lane) * 2, 0, 0));
#pragma unroll
  for (int q = 0; q < P; ++q) {
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) t += bf16_to_f32(v[q][e] & 0xFFFFu) + bf16_to_f32(v[q][e] >> 16);
    t = dpp_row_add<0xB1>(t);   // quad_perm 1,0,3,2
    t = dpp_row_add<0x4E>(t);   // quad_perm 2,3,0,1
    t = dpp_row_add<0x124>(t);  // row_ror 4
    t = dpp_row_add<0x128>(t);  // row_ror 8
    const int kb = 4 * (p0 + q) + (lane >> 4);
    if ((lane & 15) == 0 && kb < KB) xs[(size_t)kb * Mp + m] = -136.f * t;
  }
}

// Workgroup geometry and the LDS of one stage: activations [BM][256 B]
// swizzled, weight tiles [NT16][1 KB], scales [NT16][16] u16, seeds [BM] f32.
template <int MS, int NT, int WM, int WN>
struct Pf {
  static constexpr int W = WM * WN;                 // waves
  static constexpr int BM = 16 * MS * WM, BN = 16 * NT * WN;
  static constexpr int RM = 16 * MS;                // rows per wave
  static constexpr int NT16 = NT * WN;              // 16-row weight tiles per workgroup
  static constexpr int A = 0, B = BM * 256, S = B + NT16 * 1024, X = S + NT16 * 32,
                       BYTES = X + BM * 4;
  static constexpr int AL = BM / (4 * W);           // 1 KB activation loads per wave
  static constexpr int BL = NT16 / W;               // weight tiles loaded per wave
  static constexpr int SL = NT16 * 8 / W;           // lanes loading 4 scale bytes each
  static constexpr int XL = BM / (4 * W);           // lanes loading 4 seeds each
  static constexpr int LOADS = AL + BL + 2;
  static_assert(AL >= 1 && BL >= 1 && SL <= 64 && XL >= 1, "workgroup shape");
};

// Load `l` (0 .. LOADS-1) of wave `wave`'s share of k-block kb into stage
// buffer `buf`: activation blocks, weight tiles, scales, seeds.
template <class P>
CAI4_DEV void pf_load(int l, uint8_t *buf, rsrc_t xr, rsrc_t wr, rsrc_t sr, rsrc_t qr, int K,
                      int KB, int NG, int G, int Mp, int kb, int wave, int lane) {
  if (l < P::AL) {
    // activation block b = 1 KB of LDS in lane order: rows 4 b + lane / 16,
    // slot lane & 15 holding chunk slot ^ (row & 15)
    const int blk = wave * P::AL + l;
    const int row = 4 * blk + (lane >> 4);
    const int q = (lane & 15) ^ (row & 15);
    pf_dma<16>(xr, lds_addr(buf + P::A + blk * 1024), (uint32_t)(row * K + kb * 128 + 8 * q) * 2);
  } else if (l < P::AL + P::BL) {
    const int tile = wave * P::BL + (l - P::AL);  // 1 KB in lane order
    pf_dma<16>(wr, lds_addr(buf + P::B + tile * 1024), (uint32_t)(tile * KB + kb) * 1024 + 16 * lane);
  } else if (l == P::AL + P::BL) {
    // scales of the wave's BL tiles, 32 bytes each, four bytes per lane (lane
    // i writes LDS slot i: lanes past SL must not run the load, or they would
    // overwrite the next wave's slots)
    const int g = (kb * 128) / G;
    const int tile = wave * P::BL + (lane >> 3);
    if (lane < P::SL)
      pf_dma<4>(sr, lds_addr(buf + P::S + wave * P::SL * 4),
                (uint32_t)((tile * NG + g) * 16 * 2 + 4 * (lane & 7)));
  } else {
    // seeds of rows 4 (wave XL + lane) .. +3, 16 bytes per lane
    if (lane < P::XL)
      pf_dma<16>(qr, lds_addr(buf + P::X + wave * P::XL * 16),
                 (uint32_t)(kb * Mp + 4 * (wave * P::XL + lane)) * 4);
  }
}

// The loads one stage issues, for k-block kb two ahead (none past the end).
struct PfNext {
  uint8_t *buf;
  rsrc_t xr, wr, sr, qr;
  int K, KB, NG, G, Mp, kb, wave, lane;
  int KE;  // end of the workgroup's k-blocks (KB: the tile stride of the weights)
};

// Issue the loads of part `part` (of 8): loads [part L / 8, (part + 1) L / 8).
template <class P>
CAI4_DEV void pf_issue_part(const PfNext &n, int part) {
  if (n.kb < n.KE) {
#pragma unroll
    for (int l = 0; l < P::LOADS; ++l)
      if (l >= part * P::LOADS / 8 && l < (part + 1) * P::LOADS / 8)
        pf_load<P>(l, n.buf, n.xr, n.wr, n.sr, n.qr, n.K, n.KB, n.NG, n.G, n.Mp, n.kb, n.wave,
                   n.lane);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Activation fragments of step s: rows wm BM / WM + 16 i + (lane & 15), the
// 8 columns of chunk 4 (lane / 16) + s.
template <class P, int MS>
CAI4_DEV void pf_read_a(const uint8_t *buf, int wm, int lane, int s, u32x4_t (&af)[MS]) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < MS; ++i) {
    const int row = wm * P::RM + 16 * i + lr;  // row & 15 == lr
    af[i] = *reinterpret_cast<const u32x4_t *>(buf + P::A + row * 256 + 16 * ((4 * lg + s) ^ lr));
  }
}

template <class P, int MS, int NT, int SDT>
CAI4_DEV void pf_compute(const uint8_t *buf, int wm, int wn, int lane, const PfNext &nx,
                         f32x4_t (&acc)[MS][NT]) {
  const int lr = lane & 15, lg = lane >> 4;
  u32x4_t b[NT];
  float sc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int tile = NT * wn + j;
    b[j] = *reinterpret_cast<const u32x4_t *>(buf + P::B + tile * 1024 + 16 * lane);
    const uint32_t bits = *reinterpret_cast<const uint16_t *>(buf + P::S + tile * 32 + 2 * lr);
    sc[j] = scale_to_f32<SDT>(bits);
  }
  f32x4_t p[MS][NT];
  u32x4_t af[MS], an[MS];
  pf_read_a<P, MS>(buf, wm, lane, 0, af);
  f32x4_t seed[MS];
#pragma unroll
  for (int i = 0; i < MS; ++i)
    // D layout: lane holds rows 4 (lane / 16) + v of the 16-row tile
    seed[i] = *reinterpret_cast<const f32x4_t *>(buf + P::X + 4 * (wm * P::RM + 16 * i + 4 * lg));
  // half a step at a time: decode NT / 2 weight fragments, then their MS x NT / 2
  // MFMAs (the first step's take the seeds as their accumulator input)
  static_assert(NT % 2 == 0, "weight tiles per wave");
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s < 3) pf_read_a<P, MS>(buf, wm, lane, s + 1, an);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4_t d[NT / 2];
#pragma unroll
      for (int j = 0; j < NT / 2; ++j) d[j] = decode8(b[h * NT / 2 + j][s]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < NT / 2; ++j)
#pragma unroll
        for (int i = 0; i < MS; ++i)
          p[i][h * NT / 2 + j] = mfma_bf16(af[i], d[j], s == 0 ? seed[i] : p[i][h * NT / 2 + j]);
      __builtin_amdgcn_sched_barrier(0);
      pf_issue_part<P>(nx, 2 * s + h);
    }
#pragma unroll
    for (int i = 0; i < MS; ++i) af[i] = an[i];
  }
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] += sc[j] * p[i][j];
}

// One stage: k-block kb from `cur`; the loads of kb + 2 go into `nxt2`.
template <class P, int MS, int NT, int SDT>
CAI4_DEV void pf_stage(uint8_t *cur, uint8_t *nxt2, rsrc_t xr, rsrc_t wr, rsrc_t sr, rsrc_t qr,
                       const PfArgs &a, int KB, int KE, int NG, int kb, int wave, int wm, int wn,
                       int lane, f32x4_t (&acc)[MS][NT]) {
  if (kb >= KE) return;  // uniform
  // this wave's loads of kb are done once only kb + 1's may still be in
  // flight (loads complete in order); after the barrier every wave's have
  // landed
  if (kb + 1 < KE)
    pf_wait_barrier<P::LOADS>();
  else
    pf_wait_barrier<0>();
  const PfNext nx{nxt2, xr, wr, sr, qr, a.K, KB, NG, a.G, a.Mp, kb + 2, wave, lane, KE};
  pf_compute<P, MS, NT, SDT>(cur, wm, wn, lane, nx, acc);
}

template <int MS, int NT, int WM, int WN, int SDT>
__global__ __launch_bounds__(64 * WM * WN) void pf_gemm_kernel(PfArgs a) {
  using P = Pf<MS, NT, WM, WN>;
  __shared__ __attribute__((aligned(16))) uint8_t st0[P::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t st1[P::BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t st2[P::BYTES];
  const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  // wave index as a scalar: descriptors built from it must be uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave % WM, wn = wave / WM;
  const int m0 = blockIdx.y * P::BM, n0 = blockIdx.x * P::BN;
  const int KB = a.K >> 7, NG = a.K / a.G;
  const int ntiles = (a.N + 15) >> 4;
  const int T0 = n0 >> 4;
  const int tv =
      __builtin_amdgcn_readfirstlane(ntiles - T0 > P::NT16 ? P::NT16 : ntiles - T0);
  const rsrc_t wr = rsrc(a.w + (size_t)T0 * KB * 1024, (size_t)tv * KB * 1024);
  const rsrc_t sr = rsrc(a.s + (size_t)T0 * NG * 32, (size_t)tv * NG * 32);
  const rsrc_t xr = rsrc(a.x + (size_t)m0 * a.K, (size_t)(a.M - m0) * a.K * 2);
  const rsrc_t qr = rsrc(a.xs + m0, ((size_t)(KB - 1) * a.Mp + P::BM) * 4);

  f32x4_t acc[MS][NT];
#pragma unroll
  for (int i = 0; i < MS; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // this workgroup's k-blocks [kb0, KE): all of K, or slice blockIdx.z of it
  const int kb0 = blockIdx.z * a.kper, KE = min(KB, kb0 + a.kper);
#pragma unroll
  for (int l = 0; l < P::LOADS; ++l)
    pf_load<P>(l, st0, xr, wr, sr, qr, a.K, KB, NG, a.G, a.Mp, kb0, wave, lane);
  if (kb0 + 1 < KE) {
#pragma unroll
    for (int l = 0; l < P::LOADS; ++l)
      pf_load<P>(l, st1, xr, wr, sr, qr, a.K, KB, NG, a.G, a.Mp, kb0 + 1, wave, lane);
  }
  for (int kb = kb0; kb < KE; kb += 3) {
    pf_stage<P, MS, NT, SDT>(st0, st2, xr, wr, sr, qr, a, KB, KE, NG, kb, wave, wm, wn, lane, acc);
    pf_stage<P, MS, NT, SDT>(st1, st0, xr, wr, sr, qr, a, KB, KE, NG, kb + 1, wave, wm, wn, lane, acc);
    pf_stage<P, MS, NT, SDT>(st2, st1, xr, wr, sr, qr, a, KB, KE, NG, kb + 2, wave, wm, wn, lane, acc);
  }

  // epilogue: D lane l holds column l % 16 and rows 4 * (l / 16) + v
#pragma unroll
  for (int i = 0; i < MS; ++i) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int n = n0 + 16 * (NT * wn + j) + lr;
      if (n >= a.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * P::RM + 16 * i + 4 * lg + v;
        if (m >= a.M) continue;
        const size_t o = (size_t)m * a.N + n;
        if (a.part)  // a slice of K: the f32 partial, summed by pf_reduce_kernel
          a.part[(size_t)blockIdx.z * a.M * a.N + o] = acc[i][j][v];
        else if (a.out_f32)
          reinterpret_cast<float *>(a.y)[o] = acc[i][j][v];
        else
          reinterpret_cast<uint16_t *>(a.y)[o] = (uint16_t)f32_to_bf16_rne(acc[i][j][v]);
      }
    }
  }
}

// y = sum over the ksplit partials, in slice order; bf16 (RNE) or f32.
__global__ __launch_bounds__(256) void pf_reduce_kernel(const float *part, void *y, size_t n,
                                                        int ksplit, int out_f32) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
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
  if (out_f32) {
    *reinterpret_cast<f32x4_t *>(reinterpret_cast<float *>(y) + i) = s;
  } else {
    u32x2_t o;
    o.x = f32_to_bf16_rne(s.x) | (f32_to_bf16_rne(s.y) << 16);
    o.y = f32_to_bf16_rne(s.z) | (f32_to_bf16_rne(s.w) << 16);
    *reinterpret_cast<u32x2_t *>(reinterpret_cast<uint16_t *>(y) + i) = o;
  }
}

template <int MS, int NT, int WM, int WN>
hipError_t pf_launch(const PfArgs &a, int ksplit, hipStream_t st) {
  using P = Pf<MS, NT, WM, WN>;
  const dim3 grid((a.N + P::BN - 1) / P::BN, (a.M + P::BM - 1) / P::BM, ksplit), block(64 * P::W);
  if (a.sdt == SCALE_F16)
    hipLaunchKernelGGL((pf_gemm_kernel<MS, NT, WM, WN, SCALE_F16>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((pf_gemm_kernel<MS, NT, WM, WN, SCALE_BF16>), grid, block, 0, st, a);
  if (hipError_t e = hipGetLastError()) return e;
  if (ksplit > 1) {
    const size_t n = (size_t)a.M * a.N;
    hipLaunchKernelGGL(pf_reduce_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, st,
                       a.part, a.y, n, ksplit, a.out_f32);
    return hipGetLastError();
  }
  return hipSuccess;
}

// K slices for the 128 x 256 tile: enough workgroups to cover 7/8 of the CUs,
// at most 4 slices of at least 6 k-blocks (the three-stage pipeline); 0: none
// fits (smaller tiles instead).  1: no split.
int pf_ksplit(int M, int N, int K, int num_cus) {
  const long tiles = (long)((N + 255) / 256) * ((M + 127) / 128);
  const int KB = K / 128;
  for (int s = 1; s <= 4; ++s) {
    if (s > 1 && (KB / s < 6 || (long)M * N % 4)) break;
    if (8 * tiles * s >= 7L * num_cus) return s;
  }
  return 0;
}

int pf_rows_padded(int M) { return (M + 127) / 128 * 128; }

}  // namespace

bool prefill_supported(int M, int N, int K, int G, int tiled) {
  return tiled && M >= 64 && K % 128 == 0 && G % 128 == 0 && N >= 16;
}

size_t prefill_workspace_bytes(int M, int N, int K, int num_cus) {
  const int ks = pf_ksplit(M, N, K, num_cus);
  const size_t seeds = (((size_t)(K / 128) * pf_rows_padded(M) * 4) + 255) & ~(size_t)255;
  return seeds + (ks > 1 ? (size_t)ks * M * N * 4 : 0);
}

hipError_t prefill_gemm(const uint8_t *w, const uint8_t *s, const uint16_t *x, void *y, int M,
                        int N, int K, int G, int sdt, int out_f32, void *ws, int num_cus,
                        hipStream_t st) {
  const int Mp = pf_rows_padded(M);
  float *xs = static_cast<float *>(ws);
  const int passes = (K / 128 + 3) / 4;
  hipLaunchKernelGGL(pf_xsum_kernel, dim3(Mp / 4, (passes + kPfXsumPasses - 1) / kPfXsumPasses),
                     dim3(256), 0, st, x, xs, M, K, Mp);
  PfArgs a{w, s, x, xs, y, M, N, K, G, sdt, out_f32, Mp, K / 128, nullptr};
  const int ks = pf_ksplit(M, N, K, num_cus);
  if (ks >= 1) {  // 128 x 256, 8 waves (in ks slices of K)
    if (ks > 1) {
      a.kper = (K / 128 + ks - 1) / ks;
      const size_t seeds = (((size_t)(K / 128) * Mp * 4) + 255) & ~(size_t)255;
      a.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + seeds);
    }
    return pf_launch<4, 4, 2, 4>(a, (K / 128 + a.kper - 1) / a.kper, st);
  }
  const long tiles_mid = (long)((N + 127) / 128) * ((M + 127) / 128);
  if (tiles_mid >= num_cus) return pf_launch<4, 4, 2, 2>(a, 1, st);  // 128 x 128, 4 waves
  return pf_launch<2, 4, 2, 2>(a, 1, st);                            // 64 x 128, 4 waves
}

}  // namespace cai4
