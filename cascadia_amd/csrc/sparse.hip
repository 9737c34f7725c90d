// sparse.hip -- the activation-sparse (tau > 0) expert FFN after its gate/up
// GEMM (ffn_sparsity.rs:131-179 build_active_mask_mode, :499-537 the sparse
// branch of the GEMV form, :638-740 the AXPY form; ffn_axpy.rs:82-160).
//
// Per token the mask needs the max |silu| over every intermediate lane, so the
// gate/up GEMM comes first and leaves, next to its f32 gate and up rows, one
// slot per workgroup: that workgroup's max |silu| (the f32 bits; every value
// is >= 0 and a NaN counts as 0) with bit 31 set when one of its lanes has a
// per-channel threshold > 0.  The one-token GEMV writes them from its
// epilogue (one per 16-row tile); after any other GEMM sparse_slots_kernel
// does (one per 256 lanes).  Every slot is written on every call, so nothing
// has to be cleared first.
//
// The up GEMM reads every row, as the dense FFN does: at one token on MI355X a
// rows-subset pass costs two dependent memory round trips and a launch more
// than the fused gate/up stream takes to read the inactive rows, and the
// intermediate of the active lanes is the same either way.  What the mask
// saves is the AXPY form's down: only the active rows of the transposed down
// are read.
//
//   sparse_mask_kernel   (GEMV form) a lane per thread: the token's max and
//                        flag from its slots, the test |silu| >= cutoff * max
//                        (every lane when the max is 0 or the mode is dense),
//                        inter = silu * up or 0, and the group's count.
//   sparse_axpy_kernel   (AXPY form) workgroup (512-column block, group of
//                        256 lanes, token): the same test, the active lanes
//                        listed in ascending order (ballot + mbcnt), then
//                        sum over them of inter * W_t[lane, block] into the
//                        group's partial output row.
//   sparse_axpy_reduce_kernel  the partial rows added in group order
//                        (deterministic), and the groups' counts.
#include "int4_common.hpp"
#include "layout.hpp"
#include "sparse.hpp"
#include "tuning.hpp"

namespace cai4 {

namespace {

__global__ void fill_u32_kernel(uint32_t *p, int n, uint32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

CAI4_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float t = __shfl_xor(v, o, 64);
    v = t > v ? t : v;
  }
  return v;
}

CAI4_DEV uint32_t wave_rank(uint64_t b) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
}

// |silu| of one lane as a slot contribution (NaN -> 0).
CAI4_DEV float slot_mag(float s) {
  const float m = fabsf(s);
  return m > 0.0f ? m : 0.0f;
}

// The slots of a gate [T, I] computed by any GEMM: one per 256 lanes.
template <bool STABLE>
__global__ void __launch_bounds__(256)
    sparse_slots_kernel(const float *__restrict__ gate, int I, const float *__restrict__ thr,
                        uint32_t *__restrict__ slots, int n_slots) {
  __shared__ float s_m[4], s_p[4];
  const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m = 0.0f, pos = 0.0f;
  if (i < I) {
    const float g = gate[(size_t)t * I + i];
    m = slot_mag(STABLE ? silu_stable(g) : silu_plain(g));
    if (thr) pos = thr[i] <= 0.0f ? 0.0f : 1.0f;
  }
  m = wave_max(m);
  pos = wave_max(pos);
  if (lane == 0) {
    s_m[wave] = m;
    s_p[wave] = pos;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) {
      m = fmaxf(m, s_m[w]);
      pos = fmaxf(pos, s_p[w]);
    }
    slots[(size_t)t * n_slots + blockIdx.x] = fbits(m) | (pos > 0.0f ? 0x80000000u : 0u);
  }
}

constexpr int kSlotLoads = 8;  // slot words per thread in one round of loads

// The mask of lane i (this thread) of token t: every independent load issued
// first (the token's slots, the lane's gate / up / threshold), the slots
// folded across the workgroup (one barrier).  Returns whether the lane is
// active; *v = silu * up.  STABLE && sparse: build_active_mask_mode's SiLU.
template <bool STABLE>
CAI4_DEV bool lane_mask(const SparseMaskArgs &a, int t, int i, float *v, float *s_red,
                        uint32_t *s_flag) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t *sl = a.slots + (size_t)t * a.n_slots;
  uint32_t sv[kSlotLoads];
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    const int k = tid + 256 * u;
    sv[u] = k < a.n_slots ? sl[k] : 0u;
  }
  const bool in = i < a.I;
  const float g = in ? a.gate[(size_t)t * a.I + i] : 0.0f;
  const float up = in ? a.up[(size_t)t * a.I + i] : 0.0f;
  const float th = in && a.thr ? a.thr[i] : 0.0f;
  float m = 0.0f;
  uint32_t f = 0u;
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    m = fmaxf(m, bitsf(sv[u] & 0x7FFFFFFFu));
    f |= sv[u] >> 31;
  }
  for (int k = tid + 256 * kSlotLoads; k < a.n_slots; k += 256) {  // past 2048 slots
    const uint32_t u = sl[k];
    m = fmaxf(m, bitsf(u & 0x7FFFFFFFu));
    f |= u >> 31;
  }
  m = wave_max(m);
  const bool fw = __ballot(f != 0u) != 0ull;
  if (lane == 0) {
    s_red[wave] = m;
    s_flag[wave] = fw ? 1u : 0u;
  }
  __syncthreads();
  float mx = 0.0f;
  bool any = false;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mx = fmaxf(mx, s_red[w]);
    any = any || s_flag[w] != 0u;
  }
  // SparsityMode::is_dense (ffn_sparsity.rs:85-90): tau <= 0, or no
  // per-channel threshold > 0; then, or when the max is 0, every lane is on
  const bool sparse = a.thr ? any : !(a.tau <= 0.0f);
  const bool all = !sparse || mx == 0.0f;
  const float s = STABLE && sparse ? silu_stable(g) : silu_plain(g);
  // inter[r] = silu_gate[r] * up[r] (ffn_sparsity.rs:527, 711-716)
  *v = s * up;
  return in && (all || fabsf(s) >= (a.thr ? th : a.tau) * mx);
}

template <bool STABLE>
__global__ void __launch_bounds__(256) sparse_mask_kernel(SparseMaskArgs a) {
  __shared__ float s_red[4];
  __shared__ uint32_t s_flag[4], s_wn[4];
  const int t = blockIdx.y, i = blockIdx.x * kSparseGroup + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float v;
  const bool on = lane_mask<STABLE>(a, t, i, &v, s_red, s_flag);
  if (i < a.I) a.inter[(size_t)t * a.I + i] = on ? v : 0.0f;
  const uint64_t b = __ballot(on);
  if (lane == 0) s_wn[wave] = (uint32_t)__popcll(b);
  __syncthreads();
  if (threadIdx.x == 0)
    a.cnt[(size_t)t * gridDim.x + blockIdx.x] = ((s_wn[0] + s_wn[1]) + s_wn[2]) + s_wn[3];
}

// The AXPY form: workgroup (column block, group, token).  The group's active
// lanes are listed in ascending order; wave w takes entries w, w + 4, ...
// kAxBatch at a time, all of a batch's loads issued before any is used
// (entries past the list read its first row with weight 0); a lane owns 8
// columns (4 bytes of each transposed-down row, one bf16 scale);
// combined = inter * scale, acc += combined * n, the -8 of q = n - 8 applied
// once at the end (ffn_axpy.rs:118-134); the four waves' sums are added in
// wave order.
constexpr int kAxBatch = 16;

__global__ void __launch_bounds__(256) sparse_axpy_kernel(SparseMaskArgs a) {
  __shared__ float s_red[4];
  __shared__ uint32_t s_flag[4], s_wn[4];
  __shared__ uint32_t s_id[kSparseGroup];
  __shared__ float s_val[kSparseGroup];
  __shared__ float s_acc[3][8][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.y, tl = blockIdx.z, t = a.t0 + tl;
  const int i = g * kSparseGroup + tid;
  float v;
  const bool on = lane_mask<false>(a, t, i, &v, s_red, s_flag);
  const uint64_t b = __ballot(on);
  const uint32_t rank = wave_rank(b);
  if (lane == 0) s_wn[wave] = (uint32_t)__popcll(b);
  __syncthreads();
  uint32_t off = 0u, n = 0u;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (w < wave) off += s_wn[w];
    n += s_wn[w];
  }
  if (on) {
    s_id[off + rank] = (uint32_t)i;
    s_val[off + rank] = v;
  }
  if (blockIdx.x == 0 && tid == 0) a.cnt[(size_t)t * gridDim.y + g] = n;
  __syncthreads();

  const int c0 = blockIdx.x * kSparseAxCols + 8 * lane;  // this lane's 8 columns
  const bool cok = c0 < a.H;
  const int cc = cok ? c0 : 0;  // a lane past the columns reads column 0 and adds nothing
  const int GD = a.H / 32;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  float csum = 0.0f;
  for (int f0 = wave; f0 < (int)n; f0 += 4 * kAxBatch) {
    uint32_t q[kAxBatch], sc[kAxBatch];
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const int f = f0 + 4 * u;
      const uint32_t r = s_id[f < (int)n ? f : f0];
      q[u] = *reinterpret_cast<const uint32_t *>(a.dt + (size_t)r * (a.H / 2) + cc / 2);
      sc[u] = a.dt_s[(size_t)r * GD + cc / 32];
    }
#pragma unroll
    for (int u = 0; u < kAxBatch; ++u) {
      const int f = f0 + 4 * u;
      const float comb = f < (int)n && cok ? s_val[f] * bf16_to_f32(sc[u]) : 0.0f;
      const uint32_t lo = q[u] & 0x0F0F0F0Fu, hi = (q[u] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int k = 0; k < 4; ++k) {  // byte k: columns 2k (low nibble) and 2k + 1
        acc[2 * k] = fmaf(comb, (float)((lo >> (8 * k)) & 0xFFu), acc[2 * k]);
        acc[2 * k + 1] = fmaf(comb, (float)((hi >> (8 * k)) & 0xFFu), acc[2 * k + 1]);
      }
      csum += comb;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = fmaf(-8.0f, csum, acc[e]);
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_acc[wave - 1][e][lane] = acc[e];
  }
  __syncthreads();
  if (wave == 0 && cok) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      acc[e] = ((acc[e] + s_acc[0][e][lane]) + s_acc[1][e][lane]) + s_acc[2][e][lane];
    float *prow = a.partial + ((size_t)tl * gridDim.y + g) * a.H + c0;
    *reinterpret_cast<f32x4_t *>(prow) = f32x4_t{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<f32x4_t *>(prow + 4) = f32x4_t{acc[4], acc[5], acc[6], acc[7]};
  }
}

// Sum of the token's n group counts, by one wave (eight loads in flight).
CAI4_DEV uint32_t wave_count_sum(const uint32_t *__restrict__ cnt, int n, int lane) {
  uint32_t s = 0u;
  for (int k0 = lane; k0 < n; k0 += 64 * 8) {
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = k0 + 64 * j < n ? cnt[k0 + 64 * j] : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  return s;
}

// out[t0 + y][h] = sum over groups of partial[y][group][h], in group order
// per wave (groups w, w + 16, ...; eight loads in flight) and the sixteen
// wave sums in wave order: deterministic.  Block (0, y) also sums the token's
// group counts.
__global__ void __launch_bounds__(1024)
    sparse_axpy_reduce_kernel(const float *__restrict__ partial, int n_groups, int H,
                              float *__restrict__ out, const uint32_t *__restrict__ cnt,
                              uint32_t *__restrict__ counts, int t0) {
  __shared__ float s_sum[16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tl = blockIdx.y, t = t0 + tl, h = blockIdx.x * 64 + lane;
  const float *p = partial + (size_t)tl * n_groups * H;
  float s = 0.0f;
  if (h < H) {
    // 16 loads in flight per thread: up to 256 groups in one round
    for (int k = wave; k < n_groups; k += 16 * 16) {
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kk = k + 16 * j;
        v[j] = p[(size_t)(kk < n_groups ? kk : k) * H + h];
      }
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (k + 16 * j < n_groups) s += v[j];
    }
  }
  s_sum[wave][lane] = s;
  if (counts && blockIdx.x == 0 && wave == 15) {
    const uint32_t c = wave_count_sum(cnt + (size_t)t * n_groups, n_groups, lane);
    if (lane == 0) counts[t] = c;
  }
  __syncthreads();
  if (wave == 0 && h < H) {
    float v = s_sum[0][lane];
#pragma unroll
    for (int w = 1; w < 16; ++w) v += s_sum[w][lane];
    out[(size_t)t * H + h] = v;
  }
}

__global__ void __launch_bounds__(64)
    sparse_counts_kernel(const uint32_t *__restrict__ cnt, int n_groups,
                         uint32_t *__restrict__ counts) {
  const uint32_t c = wave_count_sum(cnt + (size_t)blockIdx.x * n_groups, n_groups, threadIdx.x);
  if (threadIdx.x == 0) counts[blockIdx.x] = c;
}

// ---------------------------------------------------------------------------
// rows-subset GEMV (ffn_sparsity.rs:187-348) and the sparse forms over it
// ---------------------------------------------------------------------------
//
// A row is read in 16-byte chunks, chunk c holding columns 32c .. 32c + 31
// (inside one scale group: G is a multiple of 32); lane l of a wave takes
// chunks l, l + 64, ...  Crate layout: chunk c is the row's bytes 16c ..
// 16c + 15 (byte b = columns 2b | 2b + 1).  Tiled layout (layout.hip): part
// c % 4 of the row's k-block c / 4 (its four dwords 256 bytes apart when the
// groups are narrower than 128 columns), each dword's byte b holding columns
// b | b + 4.  Per chunk a lane forms sum((128 + n) * x) over the nibble codes n
// (nib128) and takes the offset off with the chunk's sum of x (q = n - 8, so
// 136 x sum); the chunk's scale
// multiplies that, the lane adds its chunks, and the wave adds its lanes:
// f32 throughout (the crate's per-row sum in another order).

CAI4_DEV size_t rm_chunk(const RowsMatrix &w, int r, int c) {
  if (!w.tiled) return (size_t)r * (size_t)(w.K / 2) + 16 * (size_t)c;
  const size_t KB = (size_t)(w.K + 127) / 128;
  return ((size_t)(r >> 4) * KB + (size_t)(c >> 2)) * 1024 + 16 * (size_t)((r & 15) + 16 * (c & 3));
}
// Chunk c of row r, dword d = its columns 8 d .. 8 d + 7.  A tiled matrix
// whose groups are narrower than 128 columns stores its blocks with the
// dwords transposed across the lane rows (layout.hip): dword d of lane row
// c % 4 sits at dword c % 4 of lane row d, 256 bytes apart.
CAI4_DEV u32x4_t rm_load(const RowsMatrix &w, int r, int c) {
  if (!w.tiled || !tiled_xposed(w.G))
    return *reinterpret_cast<const u32x4_t *>(w.packed + rm_chunk(w, r, c));
  const size_t KB = (size_t)(w.K + 127) / 128;
  const uint32_t *p = reinterpret_cast<const uint32_t *>(
      w.packed + ((size_t)(r >> 4) * KB + (size_t)(c >> 2)) * 1024 + 16 * (size_t)(r & 15) +
      4 * (size_t)(c & 3));
  return u32x4_t{p[0], p[64], p[128], p[192]};
}
CAI4_DEV size_t rm_scale(const RowsMatrix &w, int r, int c) {
  const int NG = w.K / w.G, g = (32 * c) / w.G;
  if (!w.tiled) return (size_t)r * NG + g;
  return ((size_t)(r >> 4) * NG + g) * 16 + (r & 15);
}

// The f32 value 128 + n of byte k of a dword whose bytes hold nibble codes n
// (0..15): one v_perm placing the byte under the exponent byte 0x43 (the
// f32 128 is 0x43000000 and its unit in the last place 2^-16, so the byte at
// bits 16..19 adds n exactly).
template <int K>
CAI4_DEV float nib128(uint32_t t) {
  return bitsf(__builtin_amdgcn_perm(0x43000000u, t, 0x07000C0Cu | ((uint32_t)K << 16)));
}

// sum over the chunk's 32 columns of (128 + nibble) * x, x the chunk's 32
// values; the caller removes the 136 = 128 + 8 offset with the chunk's sum
// of x (q = n - 8).
template <bool TILED>
CAI4_DEV float chunk_nx(const u32x4_t v, const float *xc) {
  float s0 = 0.f, s1 = 0.f;
  const uint32_t dw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const f32x4_t xa = *reinterpret_cast<const f32x4_t *>(xc + 8 * d);
    const f32x4_t xb = *reinterpret_cast<const f32x4_t *>(xc + 8 * d + 4);
    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    const uint32_t t = dw[d] & 0x0F0F0F0Fu, u = (dw[d] >> 4) & 0x0F0F0F0Fu;
    const float a[4] = {nib128<0>(t), nib128<1>(t), nib128<2>(t), nib128<3>(t)};
    const float b[4] = {nib128<0>(u), nib128<1>(u), nib128<2>(u), nib128<3>(u)};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (TILED) {  // byte k: columns k (low nibble) and k + 4 (high)
        s0 = fmaf(a[k], xv[k], s0);
        s1 = fmaf(b[k], xv[k + 4], s1);
      } else {  // byte k: columns 2k and 2k + 1
        s0 = fmaf(a[k], xv[2 * k], s0);
        s1 = fmaf(b[k], xv[2 * k + 1], s1);
      }
    }
  }
  return s0 + s1;
}

CAI4_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// x in LDS: chunk c's 32 values at xs + kXPad * c (a 16-byte pad after every
// chunk): the lanes of a wave read 32 consecutive values each, chunks apart,
// and with an unpadded 128-byte stride every lane would hit the same banks.
constexpr int kXPad = 36;

// Stage one row of x (K values, f32 or bf16 bits) into xs as f32, chunk c at
// xs + XS * c, and each 32-column chunk's sum into sxs, by all 256 threads:
// rounds of kStageLoads 4-value loads per thread, all of a round issued
// before any is used (a load per step would cost a memory round trip each),
// then the LDS stores and the chunk sums (the 8 threads of a chunk add their
// partial sums by shuffles).
constexpr int kStageLoads = 8;
template <int XS, int NT = 256>  // NT: the workgroup's threads
CAI4_DEV void stage_x(const void *x, int x_bf16, int K, float *xs, float *sxs) {
  const int n4 = K / 4;  // 4-value items; K is a multiple of 32, so n4 of 8
  for (int i0 = 0; i0 < n4; i0 += NT * kStageLoads) {
    f32x4_t v[kStageLoads];
#pragma unroll
    for (int u = 0; u < kStageLoads; ++u) {
      const int i = i0 + NT * u + threadIdx.x;
      const int ic = i < n4 ? i : n4 - 1;  // past the row: a valid item, unused
      if (x_bf16) {
        const u32x2_t b = reinterpret_cast<const u32x2_t *>(x)[ic];
        v[u] = f32x4_t{bitsf(b.x << 16), bitsf(b.x & 0xFFFF0000u), bitsf(b.y << 16),
                       bitsf(b.y & 0xFFFF0000u)};
      } else {
        v[u] = reinterpret_cast<const f32x4_t *>(x)[ic];
      }
    }
#pragma unroll
    for (int u = 0; u < kStageLoads; ++u) {
      const int i = i0 + NT * u + threadIdx.x;
      // uniform per 8-thread chunk: n4 and NT are multiples of 8
      if (i0 + NT * u >= n4) break;
      if (i < n4) *reinterpret_cast<f32x4_t *>(xs + XS * (i >> 3) + 4 * (i & 7)) = v[u];
      float p = (v[u].x + v[u].y) + (v[u].z + v[u].w);
      p += __shfl_xor(p, 1, 64);
      p += __shfl_xor(p, 2, 64);
      p += __shfl_xor(p, 4, 64);
      if ((i & 7) == 0 && i < n4) sxs[i >> 3] = p;
    }
  }
}

// One batch of rows-subset loads: row r[u]'s chunk (j0 + j) * 64 + lane and
// its scale, for RB rows and JB chunk slots, issued unconditionally: a dead
// slot (row not ok, chunk past K) reads a valid chunk (row r[u], the last
// chunk) whose value rows_dot does not use -- a select between a load and a
// constant would make the wave wait for each load in turn.  r[u] must be a
// valid row for every u.
template <int RB, int JB>
struct RowsBatch {
  u32x4_t v[RB][JB];
  uint32_t sb[RB][JB];
};
// live: how many of the RB rows are in use, uniform over the wave (the rest
// load nothing: a scalar branch skips them).
template <int RB, int JB>
CAI4_DEV void rows_load(const RowsMatrix &w, const int (&r)[RB], int j0, int lane,
                        RowsBatch<RB, JB> &b, int live = RB) {
  const int nch = w.K >> 5;
  const uint16_t *sc = reinterpret_cast<const uint16_t *>(w.scales);
#pragma unroll
  for (int u = 0; u < RB; ++u)
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      if (u >= live) continue;
      const int c0 = (j0 + j) * 64 + lane, c = c0 < nch ? c0 : nch - 1;
      b.v[u][j] = rm_load(w, r[u], c);
      b.sb[u][j] = (uint32_t)sc[rm_scale(w, r[u], c)];
    }
}

// acc[u] += the dot products of the batch's rows (ok[u]) over its chunks.
template <int RB, int JB, bool TILED, int SDT, int XS>
CAI4_DEV void rows_dot(const RowsMatrix &w, const RowsBatch<RB, JB> &b, const bool (&ok)[RB],
                       int j0, int lane, const float *xs, const float *sxs, float (&acc)[RB]) {
  const int nch = w.K >> 5;
#pragma unroll
  for (int u = 0; u < RB; ++u)
#pragma unroll
    for (int j = 0; j < JB; ++j) {
      const int c = (j0 + j) * 64 + lane;
      if (ok[u] && c < nch) {
        const float d = fmaf(-136.0f, sxs[c], chunk_nx<TILED>(b.v[u][j], xs + XS * c));
        acc[u] = fmaf(scale_to_f32<SDT>(b.sb[u][j]), d, acc[u]);
      }
    }
}

// The standalone rows-subset GEMV: each wave takes RB listed rows at a time.
template <bool TILED, int SDT, bool XL>
__global__ void __launch_bounds__(256)
    rows_subset_kernel(RowsMatrix w, const void *x, int x_bf16, const uint32_t *__restrict__ rows,
                       int n, float *__restrict__ y, float *__restrict__ xg) {
  constexpr int RB = 4, JB = 2;
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];  // read as f32x4
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *xs, *sxs;
  if (XL) {
    stage_x<kXPad>(x, x_bf16, w.K, s_dyn, s_dyn + (w.K / 32) * kXPad);
    __syncthreads();
    xs = s_dyn;
    sxs = s_dyn + (w.K / 32) * kXPad;
  } else {  // x and its chunk sums staged once in global memory by the host's launch
    xs = xg;
    sxs = xg + w.K;
  }
  const int nch = w.K >> 5, jmax = (nch + 63) / 64;
  for (int f0 = (blockIdx.x * 4 + wave) * RB; f0 < n; f0 += gridDim.x * 4 * RB) {
    int r[RB];
    bool ok[RB];
    float acc[RB];
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int f = f0 + u;
      const uint32_t rr = f < n ? rows[f] : 0xFFFFFFFFu;
      ok[u] = rr < (uint32_t)w.N;
      r[u] = ok[u] ? (int)rr : 0;
      acc[u] = 0.f;
    }
    for (int j0 = 0; j0 < jmax; j0 += JB) {
      RowsBatch<RB, JB> bt;
      rows_load<RB, JB>(w, r, j0, lane, bt);
      rows_dot<RB, JB, TILED, SDT, XL ? kXPad : 32>(w, bt, ok, j0, lane, xs, sxs, acc);
    }
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const float s = wave_sum(acc[u]);
      if (lane == 0 && ok[u]) y[r[u]] = s;
    }
  }
}

// x (f32 or bf16) of one row -> f32 copy and chunk sums in global memory, for
// a rows-subset GEMV whose K does not fit LDS.
__global__ void __launch_bounds__(256)
    stage_x_global_kernel(const void *x, int x_bf16, int K, float *__restrict__ xg) {
  // one workgroup per 8192 columns: stage_x over that slice
  const int c0 = blockIdx.x * 8192, k = K - c0 < 8192 ? K - c0 : 8192;
  const void *xs = x_bf16 ? (const void *)(reinterpret_cast<const uint16_t *>(x) + c0)
                          : (const void *)(reinterpret_cast<const float *>(x) + c0);
  stage_x<32>(xs, x_bf16, k, xg + c0, xg + K + c0 / 32);
}

// f32 slots before the chunk sums in the fused kernels' LDS: the padded x,
// which the AXPY's padded wave rows (NW waves x 64 C rows of kXPad) reuse
// afterwards.
__host__ __device__ inline int subset_x_floats(int H, int C, int NW, bool axpy) {
  const int xf = (H / 32) * kXPad, rf = axpy ? NW * 64 * C * kXPad : 0;  // x, the waves' rows
  return xf > rf ? xf : rf;
}

// Waves per workgroup of the fused kernels: a group's active rows spread over
// 8 waves, so that a group with many active lanes has fewer rows per wave,
// except where the AXPY form's 8 output rows per lane would not fit the LDS
// (C = 4).  Measured (config 1, one token, tau 0.1 / 0.3): AXPY form 34.4 /
// 26.6 -> 29.7 / 24.7 us, GEMV form 34.2 / 28.6 -> 30.4 / 26.9 us.
constexpr int subset_waves(bool axpy, int C) { return !axpy || C <= 2 ? 8 : 4; }

// The fused sparse forms: workgroup (group g of a.lanes lanes, 16 to
// kSubsetGroup, token).  Threads 0 .. a.lanes - 1 each test one lane; the
// active lanes are listed in ascending order (ballot + mbcnt); wave w of NW takes entries w,
// w + NW, ... RB at a time, reading their up rows (and, AXPY, their
// transposed-down rows) in one round of loads.  C: chunk slots per lane (K and
// H <= 2048 C).  AXPY: lane l owns columns 32(l + 64 j) .. + 31 of the output
// (j < C): combined = inter * scale, acc += combined * (128 + n), the offset
// (-136 per unit of combined) applied once per chunk slot at the end (the -8
// of ffn_axpy.rs:118-134, plus nib128's 128); the waves' rows are added in
// wave order (0, 1, ..., NW - 1) into the group's partial row.  LDS (dynamic):
// subset_x_floats + H / 32 floats, up to 148 KB (gfx950: 160 KB per CU).
template <bool AXPY, bool TILED, int SDT, int C, int NW>
__global__ void __launch_bounds__(64 * NW) sparse_subset_kernel(SparseSubsetArgs a) {
  // rows per wave per round: 32 per workgroup round at C <= 2 (8 waves
  // hold half the rows each within 256 VGPRs)
  constexpr int RB = C <= 2 && NW == 4 ? 8 : 4, NT = 64 * NW;
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];  // read as f32x4
  __shared__ float s_red[NW];
  __shared__ uint32_t s_flag[NW], s_wn[2];
  __shared__ uint32_t s_id[kSubsetGroup];
  __shared__ float s_val[kSubsetGroup];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x, tl = blockIdx.y, t = a.t0 + tl;
  const int H = a.H;
  // [subset_x_floats] f32: x (padded chunks), then the AXPY's wave rows;
  // then [H / 32] chunk sums
  float *xs = s_dyn;
  float *sxs = s_dyn + subset_x_floats(H, C, NW, AXPY);
  // the token's slots: every thread folds its share (loads issued first)
  const uint32_t *sl = a.slots + (size_t)t * a.n_slots;
  uint32_t sv[kSlotLoads];
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    const int k = tid + NT * u;
    sv[u] = k < a.n_slots ? sl[k] : 0u;
  }
  const int i = g * a.lanes + tid;
  const bool in = tid < a.lanes && i < a.I;
  const float gv = in ? a.gate[(size_t)t * a.I + i] : 0.0f;
  const float th = in && a.thr ? a.thr[i] : 0.0f;
  stage_x<kXPad, NT>(a.x_bf16 ? (const void *)(reinterpret_cast<const uint16_t *>(a.x) + (size_t)t * H)
                          : (const void *)(reinterpret_cast<const float *>(a.x) + (size_t)t * H),
                 a.x_bf16, H, xs, sxs);
  float m = 0.0f;
  uint32_t f = 0u;
#pragma unroll
  for (int u = 0; u < kSlotLoads; ++u) {
    m = fmaxf(m, bitsf(sv[u] & 0x7FFFFFFFu));
    f |= sv[u] >> 31;
  }
  for (int k = tid + NT * kSlotLoads; k < a.n_slots; k += NT) {
    const uint32_t u = sl[k];
    m = fmaxf(m, bitsf(u & 0x7FFFFFFFu));
    f |= u >> 31;
  }
  m = wave_max(m);
  const bool fw = __ballot(f != 0u) != 0ull;
  if (lane == 0) {
    s_red[wave] = m;
    s_flag[wave] = fw ? 1u : 0u;
  }
  __syncthreads();
  float mx = 0.0f;
  bool any = false;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mx = fmaxf(mx, s_red[w]);
    any = any || s_flag[w] != 0u;
  }
  // SparsityMode::is_dense (ffn_sparsity.rs:85-90); the GEMV form's mask uses
  // build_active_mask_mode's stable SiLU, the AXPY form the plain one
  const bool sparse = a.thr ? any : !(a.tau <= 0.0f);
  const bool all = !sparse || mx == 0.0f;
  const float sg = !AXPY && sparse ? silu_stable(gv) : silu_plain(gv);
  const bool on = in && (all || fabsf(sg) >= (a.thr ? th : a.tau) * mx);
  if (!AXPY && in && !on) a.inter[(size_t)t * a.I + i] = 0.0f;
  const uint64_t b = __ballot(on);
  const uint32_t rank = wave_rank(b);
  if (lane == 0 && wave < 2) s_wn[wave] = (uint32_t)__popcll(b);
  __syncthreads();
  const uint32_t n = s_wn[0] + s_wn[1];
  if (on) {
    const uint32_t at = (wave == 0 ? 0u : s_wn[0]) + rank;
    s_id[at] = (uint32_t)i;
    s_val[at] = sg;
  }
  if (tid == 0) a.cnt[(size_t)t * gridDim.x + g] = n;
  __syncthreads();

  const int nhc = H >> 5;
  float acc[AXPY ? C : 1][AXPY ? 32 : 1];
  float csum[AXPY ? C : 1];
  if (AXPY) {
#pragma unroll
    for (int j = 0; j < C; ++j) {
      csum[j] = 0.0f;
#pragma unroll
      for (int k = 0; k < 32; ++k) acc[j][k] = 0.0f;
    }
  }
  // the list length and the wave index as scalars: rows past the list are
  // skipped by scalar branches, not loaded
  const int ns = __builtin_amdgcn_readfirstlane((int)n);
  const int ws = __builtin_amdgcn_readfirstlane(wave);
  for (int f0 = ws; f0 < ns; f0 += NW * RB) {
    int r[RB];
    bool ok[RB];
    float up[RB];
    const int live = (ns - f0 + NW - 1) / NW < RB ? (ns - f0 + NW - 1) / NW : RB;
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      const int fe = f0 + NW * u;
      ok[u] = u < live;
      r[u] = (int)s_id[ok[u] ? fe : f0];
      up[u] = 0.0f;
    }
    // the up rows, then the transposed down's rows of the batch: one round
    // of loads (unconditional, from valid addresses, as rows_load's).  The
    // scheduling barrier keeps every load ahead of the arithmetic; waiting
    // for the up rows then leaves the down rows in flight.
    RowsBatch<RB, C> ub;
    rows_load<RB, C>(a.up, r, 0, lane, ub, live);
    u32x4_t dq[AXPY ? RB : 1][AXPY ? C : 1];
    uint32_t ds[AXPY ? RB : 1][AXPY ? C : 1];
    if (AXPY) {
#pragma unroll
      for (int u = 0; u < RB; ++u)
#pragma unroll
        for (int j = 0; j < C; ++j) {
          if (u >= live) continue;
          const int c0 = j * 64 + lane, c = c0 < nhc ? c0 : nhc - 1;
          dq[u][j] = *reinterpret_cast<const u32x4_t *>(a.dt + (size_t)r[u] * (H / 2) + 16 * c);
          ds[u][j] = (uint32_t)a.dt_s[(size_t)r[u] * nhc + c];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    rows_dot<RB, C, TILED, SDT, kXPad>(a.up, ub, ok, 0, lane, xs, sxs, up);
#pragma unroll
    for (int u = 0; u < RB; ++u) {
      if (u >= live) continue;
      const int fe = f0 + NW * u;
      // inter[r] = silu_gate[r] * up[r] (ffn_sparsity.rs:527, 711-716)
      const float v = s_val[fe] * wave_sum(up[u]);
      if (!AXPY) {
        if (lane == 0) a.inter[(size_t)t * a.I + r[u]] = v;
      } else {
#pragma unroll
        for (int j = 0; j < C; ++j) {
          // a chunk slot past the row adds nothing
          const float comb = j * 64 + lane < nhc ? v * bf16_to_f32(ds[u][j]) : 0.0f;
          const uint32_t dw[4] = {dq[u][j].x, dq[u][j].y, dq[u][j].z, dq[u][j].w};
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t lo = dw[d] & 0x0F0F0F0Fu, hi = (dw[d] >> 4) & 0x0F0F0F0Fu;
            // byte k of dword d: columns 8d + 2k (low nibble), 8d + 2k + 1
            const float a4[4] = {nib128<0>(lo), nib128<1>(lo), nib128<2>(lo), nib128<3>(lo)};
            const float b4[4] = {nib128<0>(hi), nib128<1>(hi), nib128<2>(hi), nib128<3>(hi)};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              acc[j][8 * d + 2 * k] = fmaf(comb, a4[k], acc[j][8 * d + 2 * k]);
              acc[j][8 * d + 2 * k + 1] = fmaf(comb, b4[k], acc[j][8 * d + 2 * k + 1]);
            }
          }
          csum[j] += comb;
        }
      }
    }
  }
  if (!AXPY) return;
#pragma unroll
  for (int j = 0; j < C; ++j)
#pragma unroll
    for (int k = 0; k < 32; ++k) acc[j][k] = fmaf(-136.0f, csum[j], acc[j][k]);
  // every wave stores its rows in an LDS region of its own (x is no longer
  // read; rows kXPad floats apart, as x's chunks, so the lanes' 16-byte
  // stores fall in different banks); after one barrier each thread adds the
  // NW waves' values of 32 C / NW columns in wave order and stores them
  __syncthreads();
  {
    float *mine = xs + (size_t)wave * (64 * C * kXPad);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      float *row = mine + (size_t)(j * 64 + lane) * kXPad;
#pragma unroll
      for (int k4 = 0; k4 < 8; ++k4)
        *reinterpret_cast<f32x4_t *>(row + 4 * k4) =
            f32x4_t{acc[j][4 * k4], acc[j][4 * k4 + 1], acc[j][4 * k4 + 2], acc[j][4 * k4 + 3]};
    }
  }
  __syncthreads();
  {
    constexpr int PER = 32 * C / NW;  // columns per thread: 64 C rows of 32 over NT threads
    static_assert(PER % 4 == 0, "whole f32x4 per thread");
    const int q = (tid * PER) / 32, k0 = (tid * PER) % 32;  // row, first column in it
    float *prow = a.partial + ((size_t)tl * gridDim.x + g) * H + 32 * q + k0;
    if (32 * q < H) {
#pragma unroll
      for (int k4 = 0; k4 < PER / 4; ++k4) {
        f32x4_t v = *reinterpret_cast<const f32x4_t *>(xs + (size_t)q * kXPad + k0 + 4 * k4);
#pragma unroll
        for (int w = 1; w < NW; ++w) {
          const f32x4_t p = *reinterpret_cast<const f32x4_t *>(
              xs + (size_t)w * (64 * C * kXPad) + (size_t)q * kXPad + k0 + 4 * k4);
          v = f32x4_t{v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w};
        }
        *reinterpret_cast<f32x4_t *>(prow + 4 * k4) = v;
      }
    }
  }
}

// build_active_mask_mode (ffn_sparsity.rs:131-179) over one row, one
// workgroup of 1024 threads: the stable SiLU of every lane and the max |silu|
// (a NaN never raises it, as `m > max_abs` in the crate), then the active
// lanes in ascending order, 1024 at a time (ballot, wave counts, a scan of the
// 16 wave counts).
__global__ void __launch_bounds__(1024)
    build_mask_kernel(const float *__restrict__ gate, int n, float tau,
                      const float *__restrict__ thr, float *__restrict__ silu,
                      uint32_t *__restrict__ active, uint32_t *__restrict__ n_active) {
  __shared__ float s_m[16];
  __shared__ uint32_t s_f[16], s_c[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float m = 0.0f;
  uint32_t pos = 0u;
  for (int i = tid; i < n; i += 1024) {
    const float v = silu_stable(gate[i]);
    silu[i] = v;
    const float a = fabsf(v);
    m = a > m ? a : m;
    if (thr && !(thr[i] <= 0.0f)) pos = 1u;
  }
  m = wave_max(m);
  const bool pw = __ballot(pos != 0u) != 0ull;
  if (lane == 0) {
    s_m[wave] = m;
    s_f[wave] = pw ? 1u : 0u;
  }
  __syncthreads();
  float mx = 0.0f;
  bool any = false;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    mx = s_m[w] > mx ? s_m[w] : mx;
    any = any || s_f[w] != 0u;
  }
  // SparsityMode::is_dense (ffn_sparsity.rs:85-90), or a zero max: every lane
  const bool all = mx == 0.0f || (thr ? !any : tau <= 0.0f);
  uint32_t base = 0u;
  for (int i0 = 0; i0 < n; i0 += 1024) {
    const int i = i0 + tid;
    bool on = false;
    if (i < n) {
      const float cut = (thr ? thr[i] : tau) * mx;
      on = all || fabsf(silu[i]) >= cut;
    }
    const uint64_t b = __ballot(on);
    if (lane == 0) s_c[wave] = (uint32_t)__popcll(b);
    __syncthreads();
    uint32_t off = base, tot = 0u;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      if (w < wave) off += s_c[w];
      tot += s_c[w];
    }
    if (on) active[off + wave_rank(b)] = (uint32_t)i;
    base += tot;
    __syncthreads();
  }
  if (tid == 0) *n_active = base;
}

__global__ void f32_to_bf16_kernel(const float *__restrict__ x, uint16_t *__restrict__ y,
                                   size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (uint16_t)f32_to_bf16_rne(x[i]);
}

__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ x, float *__restrict__ y,
                                   size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = bf16_to_f32(x[i]);
}

}  // namespace

hipError_t sparse_slots(const float *gate, int I, int T, const float *thr, bool stable,
                        uint32_t *slots, hipStream_t st) {
  const int n = sparse_slots_per_token(I, false);
  const dim3 grid((unsigned)n, (unsigned)T);
  if (stable)
    hipLaunchKernelGGL(sparse_slots_kernel<true>, grid, dim3(256), 0, st, gate, I, thr, slots, n);
  else
    hipLaunchKernelGGL(sparse_slots_kernel<false>, grid, dim3(256), 0, st, gate, I, thr, slots,
                       n);
  return hipGetLastError();
}

hipError_t sparse_mask(const SparseMaskArgs &a, int T, bool stable, hipStream_t st) {
  const dim3 grid((unsigned)sparse_groups(a.I), (unsigned)T);
  if (stable)
    hipLaunchKernelGGL(sparse_mask_kernel<true>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(sparse_mask_kernel<false>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t sparse_axpy_ffn(const SparseMaskArgs &a, int n_tokens, float *out, uint32_t *counts,
                           hipStream_t st) {
  const int ng = sparse_groups(a.I);
  hipLaunchKernelGGL(sparse_axpy_kernel,
                     dim3((unsigned)((a.H + kSparseAxCols - 1) / kSparseAxCols), (unsigned)ng,
                          (unsigned)n_tokens),
                     dim3(256), 0, st, a);
  hipLaunchKernelGGL(sparse_axpy_reduce_kernel,
                     dim3((unsigned)((a.H + 63) / 64), (unsigned)n_tokens), dim3(1024), 0, st,
                     a.partial, ng, a.H, out, a.cnt, counts, a.t0);
  return hipGetLastError();
}

hipError_t sparse_counts(const uint32_t *cnt, int n_groups, int T, uint32_t *counts,
                         hipStream_t st) {
  hipLaunchKernelGGL(sparse_counts_kernel, dim3((unsigned)T), dim3(64), 0, st, cnt, n_groups,
                     counts);
  return hipGetLastError();
}

hipError_t fill_u32(uint32_t *p, int n, uint32_t v, hipStream_t st) {
  hipLaunchKernelGGL(fill_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n, v);
  return hipGetLastError();
}

namespace {

template <bool TILED, int SDT, bool XL>
hipError_t rows_subset_launch(const RowsMatrix &w, const void *x, bool x_bf16,
                              const uint32_t *rows, int n, float *y, int grid, size_t lds,
                              float *xg, hipStream_t st) {
  auto k = rows_subset_kernel<TILED, SDT, XL>;
  hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, st, w, x, x_bf16 ? 1 : 0, rows, n, y, xg);
  return hipGetLastError();
}

template <bool AXPY, bool TILED, int SDT, int C>
hipError_t subset_launch(const SparseSubsetArgs &a, int T, hipStream_t st) {
  constexpr int NW = subset_waves(AXPY, C);
  const size_t lds = ((size_t)subset_x_floats(a.H, C, NW, AXPY) + a.H / 32) * 4;
  auto k = sparse_subset_kernel<AXPY, TILED, SDT, C, NW>;
  hipLaunchKernelGGL(k, dim3((unsigned)subset_groups(a.I, a.lanes), (unsigned)T), dim3(64 * NW),
                     lds, st, a);
  return hipGetLastError();
}

template <bool AXPY>
hipError_t subset_dispatch(const SparseSubsetArgs &a, int T, hipStream_t st) {
  const int c = a.H <= 2048 && a.up.K <= 2048 ? 1 : a.H <= 4096 && a.up.K <= 4096 ? 2 : 4;
  const bool tiled = a.up.tiled != 0, f16 = a.up.sdt != 0;
#define CAI4_SUBSET(CC)                                                            \
  if (c == CC) {                                                                   \
    if (tiled)                                                                     \
      return f16 ? subset_launch<AXPY, true, SCALE_F16, CC>(a, T, st)              \
                 : subset_launch<AXPY, true, SCALE_BF16, CC>(a, T, st);            \
    return f16 ? subset_launch<AXPY, false, SCALE_F16, CC>(a, T, st)               \
               : subset_launch<AXPY, false, SCALE_BF16, CC>(a, T, st);             \
  }
  CAI4_SUBSET(1)
  CAI4_SUBSET(2)
  CAI4_SUBSET(4)
#undef CAI4_SUBSET
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t rows_subset(const RowsMatrix &w, const void *x, bool x_bf16, const uint32_t *rows,
                       int n, float *y, size_t max_lds, int num_cus, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const size_t lds = ((size_t)(w.K / 32) * kXPad + (size_t)w.K / 32) * 4;
  const bool xl = lds <= max_lds;
  const size_t gbytes = ((size_t)w.K + (size_t)w.K / 32) * 4;  // x in global memory: unpadded
  float *xg = nullptr;
  if (!xl) {
    // x too long for LDS: its f32 copy and chunk sums in global memory, freed
    // once the stream has used them
    if (hipMallocAsync(reinterpret_cast<void **>(&xg), gbytes, st) != hipSuccess)
      return hipErrorOutOfMemory;
    hipLaunchKernelGGL(stage_x_global_kernel, dim3((unsigned)((w.K + 8191) / 8192)), dim3(256), 0,
                       st, x, x_bf16 ? 1 : 0, w.K, xg);
    if (hipError_t e = hipGetLastError()) return e;
  }
  // 16 rows per workgroup per round, at most two rounds of workgroups per CU
  int grid = (n + 15) / 16;
  if (grid > 2 * num_cus) grid = 2 * num_cus;
  hipError_t e;
  const bool tiled = w.tiled != 0, f16 = w.sdt != 0;
  const size_t l = xl ? lds : 0;
  if (xl) {
    e = tiled ? (f16 ? rows_subset_launch<true, SCALE_F16, true>(w, x, x_bf16, rows, n, y, grid, l, xg, st)
                     : rows_subset_launch<true, SCALE_BF16, true>(w, x, x_bf16, rows, n, y, grid, l, xg, st))
              : (f16 ? rows_subset_launch<false, SCALE_F16, true>(w, x, x_bf16, rows, n, y, grid, l, xg, st)
                     : rows_subset_launch<false, SCALE_BF16, true>(w, x, x_bf16, rows, n, y, grid, l, xg, st));
  } else {
    e = tiled ? (f16 ? rows_subset_launch<true, SCALE_F16, false>(w, x, x_bf16, rows, n, y, grid, l, xg, st)
                     : rows_subset_launch<true, SCALE_BF16, false>(w, x, x_bf16, rows, n, y, grid, l, xg, st))
              : (f16 ? rows_subset_launch<false, SCALE_F16, false>(w, x, x_bf16, rows, n, y, grid, l, xg, st)
                     : rows_subset_launch<false, SCALE_BF16, false>(w, x, x_bf16, rows, n, y, grid, l, xg, st));
    const hipError_t f = hipFreeAsync(xg, st);
    if (e == hipSuccess) e = f;
  }
  return e;
}

int subset_lanes(int I, int num_cus, bool axpy) {
  const int ev = tuning_env("CASCADIA_INT4_SUBSET_LANES", 0);
  if (subset_lanes_ok(ev)) return ev;
  if (subset_groups(I, kSubsetGroup) >= num_cus) return kSubsetGroup;
  // Smaller groups for small intermediates (2048 lanes in 64-lane groups left
  // 224 CUs idle).  The GEMV form halves its group while the groups number
  // fewer than the CUs, to 8 lanes; the AXPY form, whose workgroups each add
  // a partial row and hold the LDS of a CU, while they cover under half the
  // CUs, to 16.  Measured (one token, tau 0.1 / 0.3): H 7168, I 2048 GEMV
  // form 32.0 / 26.3 us at 64 lanes, 21.2 / 19.7 at 16, 19.3 / 18.8 at 8;
  // H 4096, I 14336 GEMV form 30.4 / 26.9 at 64, 29.6 / 26.8 at 32, the AXPY
  // form 29.7 / 24.7 at 64 against 35.9 / 31.5 at 32.
  int lanes = 64;
  if (axpy)
    while (lanes > 16 && subset_groups(I, lanes) < num_cus / 2) lanes /= 2;
  else
    while (lanes > 8 && subset_groups(I, lanes) < num_cus) lanes /= 2;
  return lanes;
}

hipError_t sparse_subset_mask(const SparseSubsetArgs &a, int T, hipStream_t st) {
  if (!subset_lanes_ok(a.lanes)) return hipErrorInvalidValue;
  return subset_dispatch<false>(a, T, st);
}

hipError_t sparse_subset_axpy(const SparseSubsetArgs &a, int n_tokens, float *out,
                              uint32_t *counts, hipStream_t st) {
  if (!subset_lanes_ok(a.lanes)) return hipErrorInvalidValue;
  if (hipError_t e = subset_dispatch<true>(a, n_tokens, st)) return e;
  const int ng = subset_groups(a.I, a.lanes);
  hipLaunchKernelGGL(sparse_axpy_reduce_kernel,
                     dim3((unsigned)((a.H + 63) / 64), (unsigned)n_tokens), dim3(1024), 0, st,
                     a.partial, ng, a.H, out, a.cnt, counts, a.t0);
  return hipGetLastError();
}

hipError_t build_active_mask(const float *gate, int n, float tau, const float *thr, float *silu,
                             uint32_t *active, uint32_t *n_active, hipStream_t st) {
  hipLaunchKernelGGL(build_mask_kernel, dim3(1), dim3(1024), 0, st, gate, n, tau, thr, silu,
                     active, n_active);
  return hipGetLastError();
}

namespace {
unsigned conv_grid(size_t n) {
  const size_t g = (n + 255) / 256;
  return (unsigned)(g > 4096 ? 4096 : g);
}
}  // namespace

hipError_t f32_to_bf16_n(const float *x, uint16_t *out, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(conv_grid(n)), dim3(256), 0, st, x, out, n);
  return hipGetLastError();
}

hipError_t bf16_to_f32_n(const uint16_t *x, float *out, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(conv_grid(n)), dim3(256), 0, st, x, out, n);
  return hipGetLastError();
}

}  // namespace cai4
