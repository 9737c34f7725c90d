// abi.hip -- the extern "C" boundary (include/cascadia_int4.h).
//
// Argument validation mirrors the crate's assert_eq! length checks
// (kernel.rs:39-43, kernel_avx512_multi.rs:75-80) but returns
// CASCADIA_INT4_ERR_ARG instead of panicking; nothing throws across the ABI.
#include <stdlib.h>

#include <mutex>
#include <new>

#include "../../include/cascadia_int4.h"
#include "axpy.hpp"
#include "int4_common.hpp"
#include "layout.hpp"
#include "moe.hpp"
#include "ov.hpp"
#include "gemv.hpp"
#include "grouped.hpp"
#include "prefill.hpp"
#include "quant.hpp"
#include "skinny.hpp"
#include "sparse.hpp"
#include "synth.hpp"
#include "tuning.hpp"

namespace {

constexpr int kMaxDevices = 64;

struct DeviceState {
  int num_cus = 0;
  size_t max_lds = 0;
  void *ws = nullptr;  // library-owned workspace (grow-only)
  size_t ws_bytes = 0;
  void **retired = nullptr;  // earlier, smaller workspaces: held, never freed
  size_t n_retired = 0;
  hipStream_t side = nullptr;  // second stream for independent work (default priority)
  hipEvent_t fork = nullptr, join = nullptr;
};

std::mutex g_mu;
std::mutex g_side_mu;  // held from a fork onto the side stream to the join
DeviceState g_dev[kMaxDevices];

// Scratch of cascadia_int4_expert_forward_noalloc: a file-scope device array,
// one copy per GPU, held until the process ends.  In host code `scratch`
// names a host-side stand-in; its device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
constexpr size_t kNoAllocScratchBytes = CASCADIA_INT4_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on device `dev` (which must be current).
int noalloc_scratch(int dev, void **out) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
      return CASCADIA_INT4_ERR_DEVICE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CASCADIA_INT4_OK;
}

int current_device(int *dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kMaxDevices)
    return CASCADIA_INT4_ERR_DEVICE;
  return CASCADIA_INT4_OK;
}

// CU count and per-workgroup LDS limit of a device (queried once).
cai4::SkinnyDevice device_props(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &d = g_dev[dev];
  if (d.num_cus == 0) {
    int n = 0, l = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    if (hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
            hipSuccess ||
        l <= 0)
      l = 64 * 1024;
    d.num_cus = n;
    d.max_lds = (size_t)l;
  }
  return cai4::SkinnyDevice{d.num_cus, d.max_lds};
}

// The side stream of a device and the events that fork work onto it and
// join it back (created once; non-blocking, default priority, no timing).
int side_stream(int dev, hipStream_t *side, hipEvent_t *fork, hipEvent_t *join) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &d = g_dev[dev];
  if (!d.side) {
    hipStream_t s = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess)
      return CASCADIA_INT4_ERR_DEVICE;
    if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
      if (f) (void)hipEventDestroy(f);
      (void)hipStreamDestroy(s);
      return CASCADIA_INT4_ERR_DEVICE;
    }
    d.side = s;
    d.fork = f;
    d.join = j;
  }
  *side = d.side;
  *fork = d.fork;
  *join = d.join;
  return CASCADIA_INT4_OK;
}

// Library workspace of at least `bytes` on the current device.  Growing it
// allocates a larger buffer (at least twice the old size) and RETIRES the old
// one without freeing it: a graph captured while the old buffer was current
// keeps its address in its kernel arguments and stays valid to replay.
// Retired buffers are held until the process ends (their total stays below
// the current buffer's size, since each growth at least doubles).  A growth
// cannot be recorded by a stream capture: while `st` is capturing, a call that
// would grow the workspace is refused with ERR_ARG (pass a workspace of the
// *_workspace_bytes size instead).
int lib_workspace(int dev, size_t bytes, void **out, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState &d = g_dev[dev];
  if (d.ws_bytes < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return CASCADIA_INT4_ERR_ARG;
    size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
    if (sz < 2 * d.ws_bytes) sz = 2 * d.ws_bytes;
    void *p = nullptr;
    if (hipMalloc(&p, sz) != hipSuccess) {
      (void)hipGetLastError();
      // the doubling is a preference, the request is the requirement
      p = nullptr;
      sz = bytes;
      if (hipMalloc(&p, sz) != hipSuccess) {
        (void)hipGetLastError();
        return CASCADIA_INT4_ERR_NOMEM;
      }
    }
    if (d.ws) {
      // kept alive, never reused: captured graphs may still address it
      void **grown = static_cast<void **>(realloc(d.retired, (d.n_retired + 1) * sizeof(void *)));
      if (!grown) {
        (void)hipFree(p);
        return CASCADIA_INT4_ERR_NOMEM;
      }
      d.retired = grown;
      d.retired[d.n_retired++] = d.ws;
    }
    d.ws = p;
    d.ws_bytes = sz;
  }
  *out = d.ws;
  return CASCADIA_INT4_OK;
}

inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_layout(const cascadia_int4_layout *L) {
  if (!L) return CASCADIA_INT4_ERR_NULL;
  if (L->n_rows == 0 || L->k_cols == 0 || L->group_size == 0) return CASCADIA_INT4_ERR_ARG;
  if (L->group_size % 32 != 0 || L->k_cols % L->group_size != 0) return CASCADIA_INT4_ERR_ARG;
  if (L->scale_dtype > CASCADIA_INT4_SCALE_F16) return CASCADIA_INT4_ERR_ARG;
  if (L->tiling > CASCADIA_INT4_TILING_MFMA) return CASCADIA_INT4_ERR_ARG;
  if (L->n_rows > (1u << 30) || L->k_cols > (1u << 30)) return CASCADIA_INT4_ERR_ARG;
  return CASCADIA_INT4_OK;
}

int check_weights(const uint8_t *packed, const uint8_t *scales) {
  if (!packed || !scales) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(packed, 16) || !aligned(scales, 2)) return CASCADIA_INT4_ERR_ARG;
  return CASCADIA_INT4_OK;
}

int hip_status(hipError_t e) { return e == hipSuccess ? CASCADIA_INT4_OK : CASCADIA_INT4_ERR_DEVICE; }

int glog2_of(int G) { return (G & (G - 1)) == 0 ? __builtin_ctz((unsigned)G) : -1; }

// Activation bytes a skinny GEMM addresses with 32-bit offsets.
bool act_fits(int M, int K, int amode) {
  return (size_t)M * K * (amode == cai4::A_XF32 ? 4 : 2) < 0x7FFFFFFFu;
}

// One skinny GEMM (any M), f32 output or fused epilogue.  `partials` is
// workspace for split-K partial sums (null: the library's own workspace,
// unless `may_alloc` is false, when a plan that needs partials is an error).
int run_gemm(const uint8_t *w0, const uint8_t *s0, const uint8_t *w1, const uint8_t *s1,
             int N, int K, int G, int sdt, int tiled, const void *x, const void *x2, int amode,
             int M, void *out, void *out2, int epi, hipStream_t st, void *partials = nullptr,
             bool may_alloc = true, int ldo = 0) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  if (!act_fits(M, K, amode)) return CASCADIA_INT4_ERR_ARG;
  const cai4::SkinnyDevice d = device_props(dev);
  {  // one token over tiled weights: the streaming GEMV kernel
    cai4::SkinnyArgs g{};
    g.w0 = w0;
    g.s0 = s0;
    g.w1 = w1;
    g.s1 = s1;
    g.x = x;
    g.x2 = x2;
    g.out = out;
    g.out2 = out2;
    g.N = N;
    g.K = K;
    g.G = G;
    g.M = M;
    g.sdt = sdt;
    g.tiled = tiled;
    if ((M == 1 || ldo == 0 || ldo == N) && cai4::gemv_supported(g, amode, epi, d.num_cus))
      return hip_status(cai4::gemv_launch(g, amode, epi, d.num_cus, 0, st));
  }
  const cai4::SkinnyPlan p = cai4::skinny_plan(N, K, G, M, amode, epi, d);
  if (p.partial_bytes && !partials) {
    if (!may_alloc) return CASCADIA_INT4_ERR_ARG;
    if (int rc = lib_workspace(dev, p.partial_bytes, &partials, st)) return rc;
  }
  cai4::SkinnyArgs a{};
  a.partials = partials;
  a.w0 = w0;
  a.s0 = s0;
  a.w1 = w1;
  a.s1 = s1;
  a.x = x;
  a.x2 = x2;
  a.out = out;
  a.out2 = out2;
  a.N = N;
  a.K = K;
  a.G = G;
  a.M = M;
  a.ldx = K;
  a.ldo = ldo ? ldo : N;
  a.sdt = sdt;
  a.glog2 = glog2_of(G);
  a.tiled = tiled;
  return hip_status(cai4::skinny_launch(a, p, amode, epi, st));
}

// Tokens from which an expert FFN runs on the MFMA-tile GEMMs (grouped.hip)
// rather than the skinny kernel's 64-row passes (measured: the tiles win from
// 512 rows at the K2.6 and Llama-3-8B FFN shapes; below, too few workgroups).
// CASCADIA_INT4_FFN_TILE_TOKENS overrides.
uint32_t ffn_tile_tokens() {
  const int n = cai4::tuning_env("CASCADIA_INT4_FFN_TILE_TOKENS", 0);
  return n > 0 ? (uint32_t)n : 512u;
}

bool ffn_tile_shape(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t n_tokens) {
  return n_tokens >= ffn_tile_tokens() && cai4::gg_supported((int)hidden, (int)group, 1) &&
         cai4::gg_supported((int)inter, (int)group, 1);
}

// Workspace of an expert FFN: the SwiGLU intermediate as two bf16 planes,
// then the split-K partials of whichever of its two GEMMs needs more; or, for
// many tokens, the planes and the MFMA-tile GEMMs' seeds / split activations.
struct FfnWorkspace {
  size_t planes, partials, tile;
  size_t total() const { return planes + partials > tile ? planes + partials : tile; }
};
size_t ffn_tile_workspace(int num_cus, uint32_t hidden, uint32_t inter, uint32_t group,
                          uint32_t n_tokens, bool x_f32, bool out_bf16) {
  const size_t planes = 2 * (((size_t)n_tokens * inter * 2 + 255) & ~(size_t)255);
  const size_t a = cai4::gg_dense_workspace((int)n_tokens, (int)inter, (int)hidden, (int)group,
                                            x_f32 ? cai4::GG_A_F32 : cai4::GG_A_BF16,
                                            cai4::GG_SWIGLU_HILO, num_cus);
  const size_t b = cai4::gg_dense_workspace((int)n_tokens, (int)hidden, (int)inter, (int)group,
                                            cai4::GG_A_PLANES,
                                            out_bf16 ? cai4::GG_BF16 : cai4::GG_F32, num_cus);
  return planes + (a > b ? a : b);
}
FfnWorkspace ffn_workspace(int dev, uint32_t hidden, uint32_t inter, uint32_t group,
                           uint32_t n_tokens, bool x_f32) {
  const cai4::SkinnyDevice d = device_props(dev);
  size_t tile = 0;
  if (ffn_tile_shape(hidden, inter, group, n_tokens)) {
    const size_t t0 = ffn_tile_workspace(d.num_cus, hidden, inter, group, n_tokens, x_f32, false);
    const size_t t1 = ffn_tile_workspace(d.num_cus, hidden, inter, group, n_tokens, x_f32, true);
    tile = t0 > t1 ? t0 : t1;
  }
  const cai4::SkinnyPlan gu =
      cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens,
                        x_f32 ? cai4::A_XF32 : cai4::A_BF16, cai4::EPI_SWIGLU_HILO, d);
  const cai4::SkinnyPlan dn = cai4::skinny_plan((int)hidden, (int)inter, (int)group,
                                                (int)n_tokens, cai4::A_HILO, cai4::EPI_F32, d);
  const size_t planes = ((size_t)n_tokens * inter * 2 * sizeof(uint16_t) + 255) & ~(size_t)255;
  return FfnWorkspace{planes,
                      gu.partial_bytes > dn.partial_bytes ? gu.partial_bytes : dn.partial_bytes,
                      tile};
}

// The expert FFN on the MFMA-tile GEMMs: gate/up with the SwiGLU epilogue
// into hi / lo planes, then down over the planes (grouped.hip, dense mode).
int ffn_tiles(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t sdt,
              const cascadia_int4_expert *e, const void *x, bool x_f32, uint32_t n_tokens,
              void *out, bool out_bf16, void *ws, int num_cus, hipStream_t st) {
  const size_t plane = ((size_t)n_tokens * inter * 2 + 255) & ~(size_t)255;
  uint16_t *hi = static_cast<uint16_t *>(ws);
  uint16_t *lo = reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(ws) + plane);
  void *rest = static_cast<uint8_t *>(ws) + 2 * plane;
  cai4::GgArgs g{};
  g.w0 = e->gate_packed;
  g.s0 = e->gate_scale;
  g.w1 = e->up_packed;
  g.s1 = e->up_scale;
  g.x = static_cast<const uint16_t *>(x);
  g.y = hi;
  g.y2 = lo;
  g.M = (int)n_tokens;
  g.N = (int)inter;
  g.K = (int)hidden;
  g.G = (int)group;
  g.sdt = (int)sdt;
  g.ldy = (int)inter;
  g.epi = cai4::GG_SWIGLU_HILO;
  if (hipError_t err =
          cai4::gg_dense(g, x_f32 ? cai4::GG_A_F32 : cai4::GG_A_BF16, rest, num_cus, st))
    return hip_status(err);
  cai4::GgArgs dn{};
  dn.w0 = e->down_packed;
  dn.s0 = e->down_scale;
  dn.x = hi;
  dn.x2 = lo;
  dn.y = out;
  dn.M = (int)n_tokens;
  dn.N = (int)hidden;
  dn.K = (int)inter;
  dn.G = (int)group;
  dn.sdt = (int)sdt;
  dn.ldy = (int)hidden;
  dn.epi = out_bf16 ? cai4::GG_BF16 : cai4::GG_F32;
  return hip_status(cai4::gg_dense(dn, cai4::GG_A_PLANES, rest, num_cus, st));
}

void expert_sections(uint32_t hidden, uint32_t inter, uint32_t group, size_t off[6]) {
  const size_t gp = (size_t)inter * hidden / 2, gs = (size_t)inter * (hidden / group) * 2;
  const size_t dp = (size_t)hidden * inter / 2;
  off[0] = 0;
  off[1] = gp;
  off[2] = gp + gs;
  off[3] = 2 * gp + gs;
  off[4] = 2 * (gp + gs);
  off[5] = off[4] + dp;
}

// up_rows: the caller accepts CASCADIA_INT4_TILING_MFMA_UP_ROWS (the sparse
// forms, which read up one row at a time).
int check_expert(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t sdt,
                 const cascadia_int4_expert *e, bool up_rows = false) {
  if (!e) return CASCADIA_INT4_ERR_NULL;
  if (!e->gate_packed || !e->gate_scale || !e->up_packed || !e->up_scale || !e->down_packed ||
      !e->down_scale)
    return CASCADIA_INT4_ERR_NULL;
  if (hidden == 0 || inter == 0 || group == 0 || group % 32) return CASCADIA_INT4_ERR_ARG;
  if (hidden % group || inter % group || sdt > 1) return CASCADIA_INT4_ERR_ARG;
  if (e->tiling > (up_rows ? CASCADIA_INT4_TILING_MFMA_UP_ROWS : CASCADIA_INT4_TILING_MFMA))
    return CASCADIA_INT4_ERR_ARG;
  if (!aligned(e->gate_packed, 16) || !aligned(e->up_packed, 16) ||
      !aligned(e->down_packed, 16))
    return CASCADIA_INT4_ERR_ARG;
  if (!aligned(e->gate_scale, 2) || !aligned(e->up_scale, 2) || !aligned(e->down_scale, 2))
    return CASCADIA_INT4_ERR_ARG;
  return CASCADIA_INT4_OK;
}

int ffn_common(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t sdt,
               const cascadia_int4_expert *e, const void *x, bool x_f32, uint32_t n_tokens,
               void *out, bool out_bf16, void *workspace, hipStream_t st) {
  if (int rc = check_expert(hidden, inter, group, sdt, e)) return rc;
  if (n_tokens == 0) return CASCADIA_INT4_OK;
  if (!x || !out) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x, 16)) return CASCADIA_INT4_ERR_ARG;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  if (!act_fits((int)n_tokens, (int)hidden, x_f32 ? cai4::A_XF32 : cai4::A_BF16) ||
      !act_fits((int)n_tokens, (int)inter, cai4::A_HILO))
    return CASCADIA_INT4_ERR_ARG;
  const FfnWorkspace need = ffn_workspace(dev, hidden, inter, group, n_tokens, x_f32);
  void *ws = workspace;
  if (!ws) {
    if (int rc = lib_workspace(dev, need.total(), &ws, st)) return rc;
  } else if (!aligned(ws, 16)) {
    return CASCADIA_INT4_ERR_ARG;
  }
  if (need.tile && e->tiling == CASCADIA_INT4_TILING_MFMA) {
    return ffn_tiles(hidden, inter, group, sdt, e, x, x_f32, n_tokens, out, out_bf16, ws,
                     device_props(dev).num_cus, st);
  }
  // the SwiGLU intermediate as two bf16 planes (hi, lo): [n_tokens, inter] each
  uint16_t *hi = reinterpret_cast<uint16_t *>(ws);
  uint16_t *lo = hi + (size_t)n_tokens * inter;
  void *part = need.partials ? static_cast<uint8_t *>(ws) + need.planes : nullptr;
  // a caller's workspace (or the static scratch) is never supplemented by an allocation
  const bool may_alloc = workspace == nullptr;
  int rc = run_gemm(e->gate_packed, e->gate_scale, e->up_packed, e->up_scale, (int)inter,
                    (int)hidden, (int)group, (int)sdt, (int)e->tiling, x, nullptr,
                    x_f32 ? cai4::A_XF32 : cai4::A_BF16, (int)n_tokens, hi, lo,
                    cai4::EPI_SWIGLU_HILO, st, part, may_alloc);
  if (rc) return rc;
  return run_gemm(e->down_packed, e->down_scale, nullptr, nullptr, (int)hidden, (int)inter,
                  (int)group, (int)sdt, (int)e->tiling, hi, lo, cai4::A_HILO, (int)n_tokens,
                  out, nullptr, out_bf16 ? cai4::EPI_BF16 : cai4::EPI_F32, st, part, may_alloc);
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Max-|silu| slot words of n_tokens tokens: the one-token GEMV writes one per
// 16-row tile, sparse_slots one per 256 lanes of each token.
size_t sparse_slot_bytes(uint32_t inter, uint32_t n_tokens) {
  const size_t a = (size_t)cai4::sparse_slots_per_token((int)inter, true);
  const size_t b = (size_t)n_tokens * cai4::sparse_slots_per_token((int)inter, false);
  return align256((a > b ? a : b) * 4);
}

// Workspace of the activation-sparse FFN (GEMV form): gate, up and the
// intermediate ([n_tokens, inter] f32 each), the slots, the groups' active
// counts, then split-K partials of the largest of its GEMMs; at least what the
// dense branch needs.
struct SparseWorkspace {
  size_t lanes, slots, cnt, partials, total;
};
SparseWorkspace sparse_workspace(int dev, uint32_t hidden, uint32_t inter, uint32_t group,
                                 uint32_t n_tokens) {
  const cai4::SkinnyDevice d = device_props(dev);
  size_t part = 0;
  const cai4::SkinnyPlan plans[6] = {
      cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens, cai4::A_XF32,
                        cai4::EPI_PAIR_F32, d),
      cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens, cai4::A_BF16,
                        cai4::EPI_PAIR_F32, d),
      cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens, cai4::A_XF32,
                        cai4::EPI_F32, d),
      cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens, cai4::A_BF16,
                        cai4::EPI_F32, d),
      cai4::skinny_plan((int)hidden, (int)inter, (int)group, (int)n_tokens, cai4::A_XF32,
                        cai4::EPI_F32, d),
      cai4::skinny_plan((int)hidden, (int)inter, (int)group, (int)n_tokens, cai4::A_XF32,
                        cai4::EPI_BF16, d)};
  for (const cai4::SkinnyPlan &p : plans) part = p.partial_bytes > part ? p.partial_bytes : part;
  SparseWorkspace w;
  w.lanes = align256((size_t)n_tokens * inter * 4);
  w.slots = sparse_slot_bytes(inter, n_tokens);
  w.cnt = align256((size_t)n_tokens *
                   cai4::subset_groups((int)inter, cai4::subset_lanes((int)inter, d.num_cus, false)) *
                   4);
  w.partials = part;
  w.total = 3 * w.lanes + w.slots + w.cnt + part;
  const FfnWorkspace f = ffn_workspace(dev, hidden, inter, group, n_tokens, true);
  const FfnWorkspace b = ffn_workspace(dev, hidden, inter, group, n_tokens, false);
  const size_t dense = f.total() > b.total() ? f.total() : b.total();
  if (dense > w.total) w.total = dense;
  return w;
}

// The gate and up GEMMs of a sparse form, f32 out (not combined), with the
// mask's max-|silu| slots: one fused gate/up GEMV whose epilogue writes them
// when it serves the shape, else the skinny kernel's gate/up pair and
// sparse_slots.  *n_slots: slot words per token.
int sparse_gate_up(const cascadia_int4_expert *e, uint32_t hidden, uint32_t inter,
                   uint32_t group, uint32_t sdt, const void *x, int amode, uint32_t n_tokens,
                   float *gate, float *up, const float *thr, bool stable, uint32_t *slots,
                   int *n_slots, void *part, bool may_alloc, hipStream_t st) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const cai4::SkinnyDevice d = device_props(dev);
  cai4::SkinnyArgs g{};
  g.w0 = e->gate_packed;
  g.s0 = e->gate_scale;
  g.w1 = e->up_packed;
  g.s1 = e->up_scale;
  g.x = x;
  g.out = gate;
  g.out2 = up;
  g.N = (int)inter;
  g.K = (int)hidden;
  g.G = (int)group;
  g.M = (int)n_tokens;
  g.sdt = (int)sdt;
  g.tiled = (int)e->tiling;
  g.slots = slots;
  g.thr = thr;
  g.silu_slot = stable ? 2 : 1;
  if (n_tokens == 1 && cai4::gemv_supported(g, amode, cai4::EPI_SWIGLU, d.num_cus)) {
    *n_slots = cai4::sparse_slots_per_token((int)inter, true);
    return hip_status(cai4::gemv_launch(g, amode, cai4::EPI_SWIGLU, d.num_cus, 0, st));
  }
  int rc = run_gemm(e->gate_packed, e->gate_scale, e->up_packed, e->up_scale, (int)inter,
                    (int)hidden, (int)group, (int)sdt, (int)e->tiling, x, nullptr, amode,
                    (int)n_tokens, gate, up, cai4::EPI_PAIR_F32, st, part, may_alloc);
  if (rc) return rc;
  *n_slots = cai4::sparse_slots_per_token((int)inter, false);
  return hip_status(cai4::sparse_slots(gate, (int)inter, (int)n_tokens, thr, stable, slots, st));
}

// The gate GEMM alone, f32 out, with the mask's max-|silu| slots (the
// rows-subset forms, whose up is read later for the active lanes only): the
// one-token GEMV's slot epilogue when it serves the shape, else any GEMM and
// sparse_slots.  *n_slots: slot words per token.
int sparse_gate(const uint8_t *gp, const uint8_t *gs, uint32_t tiling, uint32_t hidden,
                uint32_t inter, uint32_t group, uint32_t sdt, const void *x, int amode,
                uint32_t n_tokens, float *gate, const float *thr, bool stable, uint32_t *slots,
                int *n_slots, void *part, bool may_alloc, hipStream_t st) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const cai4::SkinnyDevice d = device_props(dev);
  cai4::SkinnyArgs g{};
  g.w0 = gp;
  g.s0 = gs;
  g.x = x;
  g.out = gate;
  g.N = (int)inter;
  g.K = (int)hidden;
  g.G = (int)group;
  g.M = (int)n_tokens;
  g.sdt = (int)sdt;
  g.tiled = (int)tiling;
  g.slots = slots;
  g.thr = thr;
  g.silu_slot = stable ? 2 : 1;
  if (n_tokens == 1 && cai4::gemv_supported(g, amode, cai4::EPI_F32, d.num_cus)) {
    *n_slots = cai4::sparse_slots_per_token((int)inter, true);
    return hip_status(cai4::gemv_launch(g, amode, cai4::EPI_F32, d.num_cus, 0, st));
  }
  int rc = run_gemm(gp, gs, nullptr, nullptr, (int)inter, (int)hidden, (int)group, (int)sdt,
                    (int)tiling, x, nullptr, amode, (int)n_tokens, gate, nullptr, cai4::EPI_F32,
                    st, part, may_alloc);
  if (rc) return rc;
  *n_slots = cai4::sparse_slots_per_token((int)inter, false);
  return hip_status(cai4::sparse_slots(gate, (int)inter, (int)n_tokens, thr, stable, slots, st));
}

// The up matrix of an expert as rows for the rows-subset kernels.
cai4::RowsMatrix up_rows(const cascadia_int4_expert *e, uint32_t hidden, uint32_t inter,
                         uint32_t group, uint32_t sdt) {
  cai4::RowsMatrix u{};
  u.packed = e->up_packed;
  u.scales = e->up_scale;
  u.N = (int)inter;
  u.K = (int)hidden;
  u.G = (int)group;
  u.sdt = (int)sdt;
  u.tiled = e->tiling == CASCADIA_INT4_TILING_MFMA ? 1 : 0;
  return u;
}

// Whether a sparse form reads up through the rows subset: every shape whose
// hidden size the fused kernels take (a multiple of 32 up to 8192); the
// mixed layout needs it.
bool subset_path(uint32_t hidden) { return cai4::subset_supported((int)hidden); }

// Gate and down layout of an expert (the mixed layout's are MFMA-tiled).
int gd_tiling(const cascadia_int4_expert *e) {
  return e->tiling == CASCADIA_INT4_TILING_CRATE ? 0 : 1;
}

// ffn_forward_sparse_f32_mode / expert_forward_sparse_mode
// (ffn_sparsity.rs:438-538, 756-867): thresholds == nullptr is the global
// tau, dense (the ordinary FFN) when tau <= 0.  Gate/up GEMM with the slots ->
// the mask and the intermediate -> the down GEMM over it.
int sparse_common(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t sdt,
                  const cascadia_int4_expert *e, const void *x, bool x_f32, uint32_t n_tokens,
                  float tau, const float *thr, void *out, bool out_bf16, uint32_t *counts,
                  void *workspace, hipStream_t st) {
  if (int rc = check_expert(hidden, inter, group, sdt, e, true)) return rc;
  const bool rows_up = e->tiling == CASCADIA_INT4_TILING_MFMA_UP_ROWS;
  if (rows_up && !subset_path(hidden)) return CASCADIA_INT4_ERR_ARG;
  if (n_tokens == 0) return CASCADIA_INT4_OK;
  if (!x || !out) return CASCADIA_INT4_ERR_NULL;
  if (n_tokens > 65535 || !aligned(x, 16) || (thr && !aligned(thr, 4)) ||
      (counts && !aligned(counts, 4)) || (workspace && !aligned(workspace, 16)))
    return CASCADIA_INT4_ERR_ARG;
  if (!thr && tau <= 0.0f && !rows_up) {
    int rc = ffn_common(hidden, inter, group, sdt, e, x, x_f32, n_tokens, out, out_bf16,
                        workspace, st);
    if (rc || !counts) return rc;
    return hip_status(cai4::fill_u32(counts, (int)n_tokens, inter, st));
  }
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const int amode = x_f32 ? cai4::A_XF32 : cai4::A_BF16;
  if (!act_fits((int)n_tokens, (int)hidden, amode) ||
      !act_fits((int)n_tokens, (int)inter, cai4::A_XF32))
    return CASCADIA_INT4_ERR_ARG;
  const SparseWorkspace w = sparse_workspace(dev, hidden, inter, group, n_tokens);
  void *ws = workspace;
  if (!ws) {
    if (int rc = lib_workspace(dev, w.total, &ws, st)) return rc;
  }
  uint8_t *b = static_cast<uint8_t *>(ws);
  float *gate = reinterpret_cast<float *>(b);
  float *upv = reinterpret_cast<float *>(b + w.lanes);
  float *mid = reinterpret_cast<float *>(b + 2 * w.lanes);
  uint32_t *slots = reinterpret_cast<uint32_t *>(b + 3 * w.lanes);
  uint32_t *cnt = reinterpret_cast<uint32_t *>(b + 3 * w.lanes + w.slots);
  void *part = w.partials ? b + 3 * w.lanes + w.slots + w.cnt : nullptr;
  int n_slots = 0;
  if (subset_path(hidden)) {
    // gate in full, then per 128-lane group the mask and the up rows of the
    // active lanes only (ffn_sparsity.rs:499-527), then the down in full
    (void)upv;
    int rc = sparse_gate(e->gate_packed, e->gate_scale, gd_tiling(e), hidden, inter, group, sdt,
                         x, amode, n_tokens, gate, thr, true, slots, &n_slots, part, true, st);
    if (rc) return rc;
    cai4::SparseSubsetArgs a{};
    a.gate = gate;
    a.slots = slots;
    a.n_slots = n_slots;
    a.thr = thr;
    a.tau = tau;
    a.up = up_rows(e, hidden, inter, group, sdt);
    a.x = x;
    a.x_bf16 = x_f32 ? 0 : 1;
    a.I = (int)inter;
    a.H = (int)hidden;
    a.lanes = cai4::subset_lanes((int)inter, device_props(dev).num_cus, false);
    a.cnt = cnt;
    a.inter = mid;
    if ((rc = hip_status(cai4::sparse_subset_mask(a, (int)n_tokens, st)))) return rc;
    if (counts && (rc = hip_status(cai4::sparse_counts(cnt, cai4::subset_groups((int)inter, a.lanes),
                                                       (int)n_tokens, counts, st))))
      return rc;
    return run_gemm(e->down_packed, e->down_scale, nullptr, nullptr, (int)hidden, (int)inter,
                    (int)group, (int)sdt, gd_tiling(e), mid, nullptr, cai4::A_XF32,
                    (int)n_tokens, out, nullptr, out_bf16 ? cai4::EPI_BF16 : cai4::EPI_F32, st,
                    part);
  }
  int rc = sparse_gate_up(e, hidden, inter, group, sdt, x, amode, n_tokens, gate, upv, thr, true,
                          slots, &n_slots, part, true, st);
  if (rc) return rc;
  cai4::SparseMaskArgs m{};
  m.gate = gate;
  m.up = upv;
  m.slots = slots;
  m.thr = thr;
  m.tau = tau;
  m.n_slots = n_slots;
  m.I = (int)inter;
  m.H = (int)hidden;
  m.cnt = cnt;
  m.inter = mid;
  if ((rc = hip_status(cai4::sparse_mask(m, (int)n_tokens, true, st)))) return rc;
  if (counts && (rc = hip_status(cai4::sparse_counts(cnt, cai4::sparse_groups((int)inter),
                                                     (int)n_tokens, counts, st))))
    return rc;
  return run_gemm(e->down_packed, e->down_scale, nullptr, nullptr, (int)hidden, (int)inter,
                  (int)group, (int)sdt, (int)e->tiling, mid, nullptr, cai4::A_XF32,
                  (int)n_tokens, out, nullptr, out_bf16 ? cai4::EPI_BF16 : cai4::EPI_F32, st,
                  part);
}

// Workspace of the AXPY-form sparse FFN: gate and up ([n_tokens, inter] f32
// each), the slots, the groups' counts [n_tokens, groups], the GEMMs' split-K
// partials, then the groups' partial output rows of up to `chunk` tokens.
struct AxpyFfnWorkspace {
  size_t lanes, slots, cnt, part_gemm, rows, total;
  uint32_t chunk;  // tokens per AXPY launch pair
};
AxpyFfnWorkspace axpy_ffn_workspace(int dev, uint32_t hidden, uint32_t inter, uint32_t group,
                                    uint32_t n_tokens) {
  const cai4::SkinnyDevice d = device_props(dev);
  AxpyFfnWorkspace w;
  // one token's partial rows: one per lane group (128 lanes on the
  // rows-subset path, 256 on the other)
  const int groups = subset_path(hidden)
                         ? cai4::subset_groups((int)inter,
                                               cai4::subset_lanes((int)inter, d.num_cus, true))
                         : cai4::sparse_groups((int)inter);
  const size_t row_set = (size_t)groups * hidden * 4;
  // at most ~32 MB of partial rows per launch pair
  const size_t fit = ((size_t)32 << 20) / row_set;
  w.chunk = (uint32_t)(fit < 1 ? 1 : fit < n_tokens ? fit : n_tokens);
  w.lanes = align256((size_t)n_tokens * inter * 4);
  w.slots = sparse_slot_bytes(inter, n_tokens);
  w.cnt = align256((size_t)n_tokens * groups * 4);
  const size_t pp = cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens,
                                      cai4::A_XF32, cai4::EPI_PAIR_F32, d)
                        .partial_bytes;
  const size_t pg = cai4::skinny_plan((int)inter, (int)hidden, (int)group, (int)n_tokens,
                                      cai4::A_XF32, cai4::EPI_F32, d)
                        .partial_bytes;  // the gate alone (rows-subset path)
  w.part_gemm = align256(pp > pg ? pp : pg);
  w.rows = align256((size_t)w.chunk * row_set);
  w.total = 2 * w.lanes + w.slots + w.cnt + w.part_gemm + w.rows;
  return w;
}

// ffn_forward_sparse_axpy_f32_mode (ffn_sparsity.rs:638-740) for n_tokens
// rows: gate/up GEMM (f32 x) with the slots, then per chunk of tokens the
// mask (plain SiLU) and the AXPY of the transposed down's active rows (e->
// down_* hold transpose_requantize_down's codes and bf16 scales) into the
// groups' partial rows, and their reduction into out (overwritten) with the
// active counts.
int axpy_ffn(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t sdt,
             const cascadia_int4_expert *e, const float *x, uint32_t n_tokens, float tau,
             const float *thr, float *out, uint32_t *counts_out, void *workspace,
             hipStream_t st) {
  if (int rc = check_expert(hidden, inter, group, sdt, e, true)) return rc;
  if (e->tiling == CASCADIA_INT4_TILING_MFMA_UP_ROWS && !subset_path(hidden))
    return CASCADIA_INT4_ERR_ARG;
  if (n_tokens == 0) return CASCADIA_INT4_OK;
  if (!x || !out) return CASCADIA_INT4_ERR_NULL;
  if (hidden % 32 || n_tokens > 65535 || !aligned(x, 16) || !aligned(out, 16) ||
      (thr && !aligned(thr, 4)) || (counts_out && !aligned(counts_out, 4)) ||
      (workspace && !aligned(workspace, 16)))
    return CASCADIA_INT4_ERR_ARG;
  if (!act_fits((int)n_tokens, (int)hidden, cai4::A_XF32) ||
      !act_fits((int)n_tokens, (int)inter, cai4::A_XF32))
    return CASCADIA_INT4_ERR_ARG;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const AxpyFfnWorkspace w = axpy_ffn_workspace(dev, hidden, inter, group, n_tokens);
  void *ws = workspace;
  if (!ws) {
    if (int rc = lib_workspace(dev, w.total, &ws, st)) return rc;
  }
  uint8_t *b = static_cast<uint8_t *>(ws);
  float *gate = reinterpret_cast<float *>(b);
  float *upv = reinterpret_cast<float *>(b + w.lanes);
  b += 2 * w.lanes;
  uint32_t *slots = reinterpret_cast<uint32_t *>(b);
  b += w.slots;
  uint32_t *cnt = reinterpret_cast<uint32_t *>(b);
  b += w.cnt;
  void *part_gemm = w.part_gemm ? b : nullptr;
  b += w.part_gemm;
  float *rows = reinterpret_cast<float *>(b);
  int n_slots = 0;
  if (subset_path(hidden)) {
    // gate in full; per 128-lane group the mask, the up rows and the
    // transposed-down rows of the active lanes only, into the group's
    // partial row; the partial rows added in group order
    (void)upv;
    int rc = sparse_gate(e->gate_packed, e->gate_scale, gd_tiling(e), hidden, inter, group, sdt,
                         x, cai4::A_XF32, n_tokens, gate, thr, false, slots, &n_slots, part_gemm,
                         workspace == nullptr, st);
    if (rc) return rc;
    cai4::SparseSubsetArgs a{};
    a.gate = gate;
    a.slots = slots;
    a.n_slots = n_slots;
    a.thr = thr;
    a.tau = tau;
    a.up = up_rows(e, hidden, inter, group, sdt);
    a.x = x;
    a.x_bf16 = 0;
    a.I = (int)inter;
    a.H = (int)hidden;
    a.lanes = cai4::subset_lanes((int)inter, device_props(dev).num_cus, true);
    a.cnt = cnt;
    a.dt = e->down_packed;
    a.dt_s = reinterpret_cast<const uint16_t *>(e->down_scale);
    a.partial = rows;
    hipError_t err = hipSuccess;
    for (uint32_t t0 = 0; t0 < n_tokens && err == hipSuccess; t0 += w.chunk) {
      const uint32_t nt = n_tokens - t0 < w.chunk ? n_tokens - t0 : w.chunk;
      a.t0 = (int)t0;
      err = cai4::sparse_subset_axpy(a, (int)nt, out, counts_out, st);
    }
    return hip_status(err);
  }
  int rc = sparse_gate_up(e, hidden, inter, group, sdt, x, cai4::A_XF32, n_tokens, gate, upv,
                          thr, false, slots, &n_slots, part_gemm, workspace == nullptr, st);
  if (rc) return rc;
  cai4::SparseMaskArgs m{};
  m.gate = gate;
  m.up = upv;
  m.slots = slots;
  m.thr = thr;
  m.tau = tau;
  m.n_slots = n_slots;
  m.I = (int)inter;
  m.H = (int)hidden;
  m.cnt = cnt;
  m.dt = e->down_packed;
  m.dt_s = reinterpret_cast<const uint16_t *>(e->down_scale);
  m.partial = rows;
  hipError_t err = hipSuccess;
  for (uint32_t t0 = 0; t0 < n_tokens && err == hipSuccess; t0 += w.chunk) {
    const uint32_t nt = n_tokens - t0 < w.chunk ? n_tokens - t0 : w.chunk;
    m.t0 = (int)t0;
    err = cai4::sparse_axpy_ffn(m, (int)nt, out, counts_out, st);
  }
  return hip_status(err);
}

// offsets of the six sections of a tiled expert blob
void tiled_expert_sections(uint32_t hidden, uint32_t inter, uint32_t group, size_t off[7]) {
  size_t gp, gs, dp, ds;
  cai4::tiled_sizes((int)inter, (int)hidden, (int)group, &gp, &gs);
  cai4::tiled_sizes((int)hidden, (int)inter, (int)group, &dp, &ds);
  const size_t sz[6] = {gp, gs, gp, gs, dp, ds};
  off[0] = 0;
  for (int i = 0; i < 6; ++i) off[i + 1] = off[i] + align256(sz[i]);
}
size_t expert_blob_bytes(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t tiling) {
  if (tiling) {
    size_t off[7];
    tiled_expert_sections(hidden, inter, group, off);
    return off[6];
  }
  size_t off[6];
  expert_sections(hidden, inter, group, off);
  return off[5] + (size_t)hidden * (inter / group) * 2;
}

void expert_blob_sections(uint32_t hidden, uint32_t inter, uint32_t group, uint32_t tiling,
                          size_t off[6]) {
  if (tiling) {
    size_t o[7];
    tiled_expert_sections(hidden, inter, group, o);
    for (int i = 0; i < 6; ++i) off[i] = o[i];
  } else {
    expert_sections(hidden, inter, group, off);
  }
}

// Which prefill kernel: prefill.hip's (K and G multiples of 128), or the
// MFMA-tile GEMM of grouped.hip (any G of 32, 64, 128k; CASCADIA_INT4_PREFILL_TILES=1
// takes it for every shape).
bool prefill_tiles(const cascadia_int4_layout *L) {
  return cai4::tuning_env("CASCADIA_INT4_PREFILL_TILES", 0) > 0 || L->group_size % 128 != 0;
}

// Prefill GEMM (M >= 64 tokens, MFMA-tiled weights).
int run_prefill(const cascadia_int4_layout *L, const uint8_t *packed, const uint8_t *scales,
                const uint16_t *x, uint32_t M, void *y, bool out_f32, hipStream_t st) {
  int dev;
  if (int rc = current_device(&dev)) return rc;
  if ((size_t)M * L->k_cols * 2 >= 0x7FFFFFFFu) return CASCADIA_INT4_ERR_ARG;
  if (prefill_tiles(L)) {
    const int cus = device_props(dev).num_cus;
    void *ws = nullptr;
    if (int rc = lib_workspace(
            dev,
            cai4::gg_dense_workspace((int)M, (int)L->n_rows, (int)L->k_cols, (int)L->group_size,
                                     cai4::GG_A_BF16, out_f32 ? cai4::GG_F32 : cai4::GG_BF16, cus),
            &ws, st))
      return rc;
    cai4::GgArgs a{};
    a.w0 = packed;
    a.s0 = scales;
    a.x = x;
    a.y = y;
    a.M = (int)M;
    a.N = (int)L->n_rows;
    a.K = (int)L->k_cols;
    a.G = (int)L->group_size;
    a.sdt = (int)L->scale_dtype;
    a.ldy = (int)L->n_rows;
    a.epi = out_f32 ? cai4::GG_F32 : cai4::GG_BF16;
    return hip_status(cai4::gg_dense(a, cai4::GG_A_BF16, ws, cus, st));
  }
  void *ws = nullptr;
  if (int rc = lib_workspace(dev,
                             cai4::prefill_workspace_bytes((int)M, (int)L->n_rows, (int)L->k_cols,
                                                           device_props(dev).num_cus),
                             &ws, st))
    return rc;
  return hip_status(cai4::prefill_gemm(packed, scales, x, y, (int)M, (int)L->n_rows,
                                       (int)L->k_cols, (int)L->group_size, (int)L->scale_dtype,
                                       out_f32 ? 1 : 0, ws, device_props(dev).num_cus, st));
}

// Many tokens over MFMA-tiled weights: one of the prefill GEMMs.
bool prefill_shape(const cascadia_int4_layout *L, uint32_t seq) {
  if (!L->tiling || seq < 64 || L->n_rows < 16) return false;
  if (L->group_size % 128 == 0 && !prefill_tiles(L))
    return cai4::prefill_supported((int)seq, (int)L->n_rows, (int)L->k_cols, (int)L->group_size,
                                   (int)L->tiling);
  return cai4::gg_supported((int)L->k_cols, (int)L->group_size, 1);
}

// ---- sparse-MoE layer ----

bool has_shared(const cascadia_int4_moe_layer *L) {
  const cascadia_int4_expert &e = L->shared;
  return e.gate_packed || e.gate_scale || e.up_packed || e.up_scale || e.down_packed ||
         e.down_scale;
}

int moe_check(const cascadia_int4_moe_layer *L, uint32_t top_k, uint32_t T) {
  if (!L || !L->experts) return CASCADIA_INT4_ERR_NULL;
  const uint32_t H = L->hidden, I = L->inter, G = L->group_size;
  if (G == 0 || G % 32 || H == 0 || I == 0 || H % G || I % G) return CASCADIA_INT4_ERR_ARG;
  if (L->scale_dtype > 1 || L->tiling > 1) return CASCADIA_INT4_ERR_ARG;
  if (L->n_experts == 0 || L->n_experts > (uint32_t)cai4::kMoeMaxExperts) return CASCADIA_INT4_ERR_ARG;
  if (top_k == 0 || top_k > (uint32_t)cai4::kMoeMaxTopK || top_k > L->n_experts)
    return CASCADIA_INT4_ERR_ARG;
  if (T == 0 || (size_t)T * top_k > 65535) return CASCADIA_INT4_ERR_ARG;
  if (!aligned(L->experts, 256) || L->expert_stride % 256 ||
      L->expert_stride < expert_blob_bytes(H, I, G, L->tiling))
    return CASCADIA_INT4_ERR_ARG;
  const size_t rows = (size_t)T * top_k;
  if (rows * H * 2 >= 0x7FFFFFFFu || rows * I * 2 >= 0x7FFFFFFFu ||
      (size_t)T * H * 4 >= 0x7FFFFFFFu)
    return CASCADIA_INT4_ERR_ARG;
  if (has_shared(L)) {
    if (L->shared_inter == 0 || L->shared_inter % G) return CASCADIA_INT4_ERR_ARG;
    if (int rc = check_expert(H, L->shared_inter, G, L->scale_dtype, &L->shared)) return rc;
  }
  return CASCADIA_INT4_OK;
}

struct MoePlan {
  cai4::SkinnyPlan gu, dn;
  cai4::MoeWorkspace ws;
  bool tiles;  // the MFMA-tile GEMMs (grouped.hip) over 128-row chunks
  int rows_pad;
};

// Many tokens per layer: experts receive enough rows that 16-row chunks would
// stream each hot expert's weights many times over; 128-row MFMA tiles read
// them about once per 128 rows.
bool moe_tiles(const cascadia_int4_moe_layer *L, uint32_t T) {
  return L->tiling == CASCADIA_INT4_TILING_MFMA && T >= (uint32_t)cai4::moe_tile_tokens() &&
         cai4::gg_supported((int)L->hidden, (int)L->group_size, 1) &&
         cai4::gg_supported((int)L->inter, (int)L->group_size, 1);
}

MoePlan moe_plan(int dev, const cascadia_int4_moe_layer *L, uint32_t top_k, uint32_t T,
                 bool given_ids) {
  const cai4::SkinnyDevice d = device_props(dev);
  const int H = (int)L->hidden, I = (int)L->inter, G = (int)L->group_size;
  MoePlan m{};
  m.tiles = moe_tiles(L, T);
  size_t sh = 0, sh_ws = 0;
  if (has_shared(L)) {
    const FfnWorkspace f = ffn_workspace(dev, L->hidden, L->shared_inter, L->group_size, T, true);
    sh = (size_t)T * H * sizeof(float);
    sh_ws = f.total();
  }
  if (m.tiles) {
    // hot experts in 128-row MFMA tiles; the others in 16-row skinny chunks
    const int C = cai4::kGgChunkRows, C2 = 16;
    const int n = (int)(T * top_k);
    m.rows_pad = cai4::gg_rows_pad(n);
    const int gw = cai4::gg_group_width(G);
    const int maxc2 = cai4::moe_max_chunks((int)T, (int)L->n_experts, (int)top_k, C2);
    m.gu = cai4::skinny_plan_grouped(I, H, G, C2, maxc2, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO,
                                     d);
    m.dn = cai4::skinny_plan_grouped(H, I, G, C2, maxc2, cai4::A_HILO, cai4::EPI_BF16, d);
    const size_t part =
        m.gu.partial_bytes > m.dn.partial_bytes ? m.gu.partial_bytes : m.dn.partial_bytes;
    // the token rows as bf16 and their seeds (per token), the down's seeds
    // (per grouped row)
    m.ws = cai4::moe_workspace((int)T, H, I, (int)L->n_experts, (int)top_k, C, part, sh, sh_ws,
                               (size_t)T * H * 2,
                               (size_t)(H / gw) * cai4::gg_rows_pad((int)T) * 4,
                               (size_t)(I / gw) * m.rows_pad * 4, C2);
    return m;
  }
  // routing picks distinct experts per token; given ids may repeat one
  const int C = cai4::moe_chunk_rows((int)T, given_ids ? (int)(T * top_k) : (int)T,
                                     L->tiling == CASCADIA_INT4_TILING_MFMA);
  const int maxc = cai4::moe_max_chunks((int)T, (int)L->n_experts, (int)top_k, C);
  m.gu = cai4::skinny_plan_grouped(I, H, G, C, maxc, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO, d);
  m.dn = cai4::skinny_plan_grouped(H, I, G, C, maxc, cai4::A_HILO, cai4::EPI_BF16, d);
  const size_t part = m.gu.partial_bytes > m.dn.partial_bytes ? m.gu.partial_bytes
                                                              : m.dn.partial_bytes;
  m.ws = cai4::moe_workspace((int)T, H, I, (int)L->n_experts, (int)top_k, C, part, sh, sh_ws);
  return m;
}

int moe_forward(const cascadia_int4_moe_layer *L, const cascadia_int4_routing *R, const float *x,
                const float *residual, uint32_t T, float *out, int32_t *ids_out,
                float *weights_out, void *workspace, hipStream_t st) {
  if (!R || !x || !out) return CASCADIA_INT4_ERR_NULL;
  if (int rc = moe_check(L, R->top_k, T)) return rc;
  if (R->mode > CASCADIA_INT4_ROUTE_SOFTMAX_TOPK) return CASCADIA_INT4_ERR_ARG;
  if (R->mode == CASCADIA_INT4_ROUTE_IDS ? (!R->ids || !R->weights) : !R->logits)
    return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x, 16) || !aligned(out, 16) || (residual && !aligned(residual, 16)))
    return CASCADIA_INT4_ERR_ARG;
  if ((ids_out && !aligned(ids_out, 4)) || (weights_out && !aligned(weights_out, 4)))
    return CASCADIA_INT4_ERR_ARG;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const MoePlan m = moe_plan(dev, L, R->top_k, T, R->mode == CASCADIA_INT4_ROUTE_IDS);
  void *ws = workspace;
  if (!ws) {
    if (int rc = lib_workspace(dev, m.ws.total, &ws, st)) return rc;
  } else if (!aligned(ws, 256)) {
    return CASCADIA_INT4_ERR_ARG;
  }
  uint8_t *W = static_cast<uint8_t *>(ws);
  const int H = (int)L->hidden, I = (int)L->inter, E = (int)L->n_experts, k = (int)R->top_k;
  const size_t n = (size_t)T * k;
  int32_t *ids = ids_out ? ids_out : reinterpret_cast<int32_t *>(W + m.ws.ids);
  float *wts = weights_out ? weights_out : reinterpret_cast<float *>(W + m.ws.weights);
  cai4::MoeRouting r{};
  r.mode = (int)R->mode;
  r.top_k = k;
  r.logits = R->logits;
  r.bias = R->bias;
  r.scale = R->scale;
  r.normalize = (int)R->normalize;
  r.ids = R->ids;
  r.weights = R->weights;
  r.threshold = R->threshold;
  int32_t *pos = reinterpret_cast<int32_t *>(W + m.ws.pos);
  int32_t *row_map = reinterpret_cast<int32_t *>(W + m.ws.row_map);
  cai4::SkinnyChunk *chunks = reinterpret_cast<cai4::SkinnyChunk *>(W + m.ws.chunks);
  int32_t *counts = reinterpret_cast<int32_t *>(W + m.ws.counts);
  uint16_t *hi = reinterpret_cast<uint16_t *>(W + m.ws.hi);
  uint16_t *lo = reinterpret_cast<uint16_t *>(W + m.ws.lo);
  uint16_t *y = reinterpret_cast<uint16_t *>(W + m.ws.y);
  void *part = W + m.ws.part;  // used only when a grouped GEMM splits K
  // The shared expert depends only on x: unless it runs as a slot of the
  // one-token launches, it runs on the side stream, forked below and joined
  // before the combine, so it fills the routed path's gaps.  The guard
  // enqueues the join on every return path once the fork is made.
  struct Join {
    hipStream_t st = nullptr;
    hipEvent_t ev = nullptr;
    std::unique_lock<std::mutex> lk;
    hipError_t wait() {
      hipError_t e = hipSuccess;
      if (ev) e = hipStreamWaitEvent(st, ev, 0);
      ev = nullptr;
      if (lk.owns_lock()) lk.unlock();
      return e;
    }
    ~Join() { (void)wait(); }
  } join_guard;
  size_t off[6];
  expert_blob_sections(L->hidden, L->inter, L->group_size, L->tiling, off);
  const int G = (int)L->group_size;
  const cai4::SkinnyDevice d = device_props(dev);
  // one token: the grouped down of one-row chunks (when the fused down + combine
  // does not fit one round of workgroups)
  cai4::SkinnyArgs dn1{};
  dn1.w0 = L->experts + off[4];
  dn1.s0 = L->experts + off[5];
  dn1.x = hi;
  dn1.x2 = lo;
  dn1.out = y;
  dn1.chunks = chunks;
  dn1.expert_stride = L->expert_stride;
  dn1.N = H;
  dn1.K = I;
  dn1.G = G;
  dn1.M = k;
  dn1.ldx = I;
  dn1.ldo = H;
  dn1.sdt = (int)L->scale_dtype;
  dn1.glog2 = glog2_of(G);
  dn1.tiled = (int)L->tiling;
  const bool fused1 = T == 1 && cai4::gemv_moe1_down_fused(H, I, G, k, d.num_cus);
  const bool one_tok =
      T == 1 && L->tiling == CASCADIA_INT4_TILING_MFMA &&
      cai4::gemv_moe1_supported(H, I, G, k, E, d.num_cus) &&
      (fused1 || cai4::gemv_supported(dn1, cai4::A_HILO, cai4::EPI_BF16, d.num_cus, 1, k));
  // One token whose shared expert has the routed experts' shape (and layout):
  // its down runs as an always-on slot (f32 out) of the grouped down launch,
  // its gate/up as a slot of the routed gate/up launch too (sh_mode 1, the
  // default: no side stream), or as a GEMV beside the routed one writing the
  // spare hi / lo row (2); CASCADIA_INT4_MOE1_SHARED = 0 / 1 / 2 chooses,
  // 0 = its own FFN beside.
  int sh_mode = 0;
  if (one_tok && !fused1 && has_shared(L) && L->shared_inter == L->inter &&
      L->shared.tiling == CASCADIA_INT4_TILING_MFMA &&
      cai4::gemv_supported(dn1, cai4::A_HILO, cai4::EPI_BF16, d.num_cus, 1, k + 1)) {
    sh_mode = cai4::tuning_env("CASCADIA_INT4_MOE1_SHARED", 1);
    if (sh_mode < 0 || sh_mode > 2) sh_mode = 1;
  }
  const bool sh_slot = sh_mode != 0;
  float *sh = nullptr;
  if (has_shared(L)) sh = reinterpret_cast<float *>(W + m.ws.shared);
  if (has_shared(L) && sh_mode != 1) {
    // the shared FFN (or, sh_mode 2, its gate/up into the spare hi / lo row)
    auto shared_work = [&](hipStream_t on) {
      if (sh_mode == 2)
        return run_gemm(L->shared.gate_packed, L->shared.gate_scale, L->shared.up_packed,
                        L->shared.up_scale, I, H, (int)L->group_size, (int)L->scale_dtype,
                        (int)L->shared.tiling, x, nullptr, cai4::A_XF32, 1,
                        hi + (size_t)k * I, lo + (size_t)k * I, cai4::EPI_SWIGLU_HILO, on);
      return ffn_common(L->hidden, L->shared_inter, L->group_size, L->scale_dtype, &L->shared,
                        x, true, T, sh, false, W + m.ws.shared_ws, on);
    };
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    if (side_stream(dev, &side, &fork, &join) == CASCADIA_INT4_OK) {
      join_guard.lk = std::unique_lock<std::mutex>(g_side_mu);
      if (hipEventRecord(fork, st) != hipSuccess ||
          hipStreamWaitEvent(side, fork, 0) != hipSuccess)
        return CASCADIA_INT4_ERR_DEVICE;
      const int rc = shared_work(side);
      if (hipEventRecord(join, side) != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
      join_guard.st = st;
      join_guard.ev = join;
      if (rc) return rc;
    } else if (int rc = shared_work(st)) {
      return rc;  // no side stream (e.g. first call inside a stream capture): in order on st
    }
  }
  if (one_tok) {
    // one token: routing inside the gate/up GEMV, the combine inside the down GEMV
    cai4::Moe1Args q{};
    q.gate = L->experts + off[0];
    q.gate_s = L->experts + off[1];
    q.up = L->experts + off[2];
    q.up_s = L->experts + off[3];
    q.down = L->experts + off[4];
    q.down_s = L->experts + off[5];
    q.expert_stride = L->expert_stride;
    q.x = x;
    q.route = r;
    q.E = E;
    q.top_k = k;
    q.ids = ids;
    q.wts = wts;
    q.pos = pos;
    q.hi = hi;
    q.lo = lo;
    q.residual = residual;
    q.shared = sh;
    q.out = out;
    q.H = H;
    q.I = I;
    q.G = G;
    q.sdt = (int)L->scale_dtype;
    if (sh_slot) {
      q.sh = sh_mode;
      q.sh_gate = L->shared.gate_packed;
      q.sh_gate_s = L->shared.gate_scale;
      q.sh_up = L->shared.up_packed;
      q.sh_up_s = L->shared.up_scale;
    }
    if (R->mode != CASCADIA_INT4_ROUTE_IDS && !cai4::gemv_moe1_routes(r, E)) {
      // many experts: route in a launch of its own, the GEMV reads the result
      if (cai4::moe_route(r, 1, E, ids, wts, st) != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
      q.route.mode = cai4::ROUTE_IDS;
      q.route.ids = ids;
      q.route.weights = wts;
    }
    const bool fused = fused1;
    if (!fused) {  // the gate/up launch also leaves one-row chunks for the grouped down
      q.chunks = chunks;
      q.row_map = row_map;
    }
    if (cai4::gemv_moe1_gate_up(q, d.num_cus, st) != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
    if (fused) {
      if (!sh) return hip_status(cai4::gemv_moe1_down(q, st));  // combine included
      // a shared expert: the routed down runs beside it, the sum is finished after the join
      q.moe_sum = reinterpret_cast<float *>(y);  // [H] f32 fits the [k, H] bf16 region
      if (cai4::gemv_moe1_down(q, st) != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
      if (join_guard.wait() != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
      return hip_status(cai4::moe_finish(residual, sh, q.moe_sum, H, out, st));
    }
    // the grouped down over the slots' one-row chunks (and the shared slot's,
    // f32 into sh; its gate/up rows joined first), then the combine
    if (sh_mode == 2 && join_guard.wait() != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
    const cai4::GemvSharedSlot shs{L->shared.down_packed, L->shared.down_scale, sh};
    if (cai4::gemv_launch(dn1, cai4::A_HILO, cai4::EPI_BF16, d.num_cus, k + (sh_slot ? 1 : 0),
                          st, sh_slot ? &shs : nullptr) != hipSuccess)
      return CASCADIA_INT4_ERR_DEVICE;
    if (join_guard.wait() != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
    return hip_status(cai4::moe_combine(residual, sh, y, pos, wts, 1, H, k, out, st));
  }
  hipError_t e = hipSuccess;
  if (m.tiles) {
    // many tokens: route, group into 128-row chunks, the token rows as bf16
    // with their seeds, then the grouped MFMA-tile gate/up (SwiGLU -> hi / lo
    // planes, reading its rows through the row map) and down (-> bf16 per
    // (token, slot)) over all experts at once
    if (R->mode == CASCADIA_INT4_ROUTE_IDS) {
      e = hipMemcpyAsync(ids, R->ids, n * 4, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync(wts, R->weights, n * 4, hipMemcpyDeviceToDevice, st);
    } else {
      e = cai4::moe_route(r, (int)T, E, ids, wts, st);
    }
    cai4::SkinnyChunk *chunks2 = reinterpret_cast<cai4::SkinnyChunk *>(W + m.ws.chunks2);
    if (e == hipSuccess)
      e = cai4::moe_group(ids, wts, R->threshold, (int)T, E, k, m.ws.chunk_rows,
                          m.ws.max_chunks, pos, row_map, chunks, counts, st, m.ws.chunk_rows2,
                          cai4::moe_tile_rows(), chunks2, m.ws.max_chunks2);
    // the skinny kernels' share: experts with few rows, 16-row chunks
    cai4::SkinnyArgs sk{};
    sk.partials = part;
    sk.chunks = chunks2;
    sk.expert_stride = L->expert_stride;
    sk.M = (int)n;
    sk.G = G;
    sk.sdt = (int)L->scale_dtype;
    sk.glog2 = glog2_of(G);
    sk.tiled = (int)L->tiling;
    uint16_t *xg = reinterpret_cast<uint16_t *>(W + m.ws.xg);
    float *sx = reinterpret_cast<float *>(W + m.ws.seeds_x);
    float *si = reinterpret_cast<float *>(W + m.ws.seeds_i);
    // the token rows as bf16 with their seeds, once per token: the hot
    // gate/up reads its rows through the row map (no copy per assignment)
    const int Tp = cai4::gg_rows_pad((int)T);
    if (e == hipSuccess)
      e = cai4::gg_prep(2, x, nullptr, nullptr, xg, nullptr, sx, (int)T, Tp, H, G, nullptr, st);
    cai4::GgArgs a{};
    a.estride = L->expert_stride;
    a.tiles = chunks;
    a.M = (int)n;
    a.G = G;
    a.sdt = (int)L->scale_dtype;
    a.rows_pad = m.rows_pad;
    if (e == hipSuccess) {
      cai4::GgArgs g = a;
      g.w0 = L->experts + off[0];
      g.s0 = L->experts + off[1];
      g.w1 = L->experts + off[2];
      g.s1 = L->experts + off[3];
      g.x = xg;
      g.seeds = sx;
      g.rows_pad = Tp;
      g.row_map = row_map;
      g.x_rows = (int)T;
      g.y = hi;
      g.y2 = lo;
      g.N = I;
      g.K = H;
      g.ldy = I;
      g.epi = cai4::GG_SWIGLU_HILO;
      g.seeds_out = si;  // the hot rows' down seeds, from the planes as they are written
      g.seeds_gw = cai4::gg_group_width(G);
      g.seeds_rp = m.rows_pad;
      e = cai4::gg_grouped(g, m.ws.max_chunks, st);
    }
    if (e == hipSuccess) {
      cai4::SkinnyArgs a2 = sk;
      a2.w0 = L->experts + off[0];
      a2.s0 = L->experts + off[1];
      a2.w1 = L->experts + off[2];
      a2.s1 = L->experts + off[3];
      a2.x = x;
      a2.row_map = row_map;
      a2.x_rows = (int)T;
      a2.out = hi;
      a2.out2 = lo;
      a2.N = I;
      a2.K = H;
      a2.ldx = H;
      a2.ldo = I;
      e = cai4::skinny_launch(a2, m.gu, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO, st);
    }
    if (e == hipSuccess) {
      cai4::GgArgs dn = a;
      dn.w0 = L->experts + off[4];
      dn.s0 = L->experts + off[5];
      dn.x = hi;
      dn.x2 = lo;
      dn.hilo = 1;
      dn.seeds = si;
      dn.y = y;
      dn.N = H;
      dn.K = I;
      dn.ldy = H;
      dn.epi = cai4::GG_BF16;
      e = cai4::gg_grouped(dn, m.ws.max_chunks, st);
    }
    if (e == hipSuccess) {
      cai4::SkinnyArgs a2 = sk;
      a2.w0 = L->experts + off[4];
      a2.s0 = L->experts + off[5];
      a2.x = hi;
      a2.x2 = lo;
      a2.out = y;
      a2.N = H;
      a2.K = I;
      a2.ldx = I;
      a2.ldo = H;
      e = cai4::skinny_launch(a2, m.dn, cai4::A_HILO, cai4::EPI_BF16, st);
    }
    if (e != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
    if (join_guard.wait() != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
    return hip_status(cai4::moe_combine(residual, sh, y, pos, wts, (int)T, H, k, out, st));
  }
  if (T <= (uint32_t)cai4::kMoePrepMaxTokens) {
    // small decode batches: routing and grouping in one launch
    e = cai4::moe_prep(r, (int)T, E, k, m.ws.chunk_rows, m.ws.max_chunks, ids, wts, pos, row_map,
                       chunks, counts, st);
  } else {
    if (R->mode == CASCADIA_INT4_ROUTE_IDS) {
      e = hipMemcpyAsync(ids, R->ids, n * 4, hipMemcpyDeviceToDevice, st);
      if (e == hipSuccess) e = hipMemcpyAsync(wts, R->weights, n * 4, hipMemcpyDeviceToDevice, st);
    } else {
      e = cai4::moe_route(r, (int)T, E, ids, wts, st);
    }
    if (e == hipSuccess)
      e = cai4::moe_group(ids, wts, R->threshold, (int)T, E, k, m.ws.chunk_rows,
                          m.ws.max_chunks, pos, row_map, chunks, counts, st);
  }
  if (e == hipSuccess) {
    cai4::SkinnyArgs a{};
    a.w0 = L->experts + off[0];
    a.s0 = L->experts + off[1];
    a.w1 = L->experts + off[2];
    a.s1 = L->experts + off[3];
    a.x = x;  // f32 token rows, read through the row map and rounded to bf16 while staged
    a.row_map = row_map;
    a.x_rows = (int)T;
    a.out = hi;
    a.out2 = lo;
    a.partials = part;
    a.chunks = chunks;
    a.expert_stride = L->expert_stride;
    a.N = I;
    a.K = H;
    a.G = G;
    a.M = (int)n;
    a.ldx = H;
    a.ldo = I;
    a.sdt = (int)L->scale_dtype;
    a.glog2 = glog2_of(G);
    a.tiled = (int)L->tiling;
    // one row per chunk (a decode token over distinct experts): the one-token GEMV
    if (cai4::gemv_supported(a, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO, d.num_cus,
                             m.ws.chunk_rows, m.ws.max_chunks))
      e = cai4::gemv_launch(a, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO, d.num_cus, m.ws.max_chunks,
                            st);
    else
      e = cai4::skinny_launch(a, m.gu, cai4::A_GATHER, cai4::EPI_SWIGLU_HILO, st);
  }
  if (e == hipSuccess) {
    cai4::SkinnyArgs a{};
    a.w0 = L->experts + off[4];
    a.s0 = L->experts + off[5];
    a.x = hi;
    a.x2 = lo;
    a.out = y;
    a.partials = part;
    a.chunks = chunks;
    a.expert_stride = L->expert_stride;
    a.N = H;
    a.K = I;
    a.G = G;
    a.M = (int)n;
    a.ldx = I;
    a.ldo = H;
    a.sdt = (int)L->scale_dtype;
    a.glog2 = glog2_of(G);
    a.tiled = (int)L->tiling;
    if (cai4::gemv_supported(a, cai4::A_HILO, cai4::EPI_BF16, d.num_cus, m.ws.chunk_rows,
                             m.ws.max_chunks))
      e = cai4::gemv_launch(a, cai4::A_HILO, cai4::EPI_BF16, d.num_cus, m.ws.max_chunks, st);
    else
      e = cai4::skinny_launch(a, m.dn, cai4::A_HILO, cai4::EPI_BF16, st);
  }
  if (e != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
  if (join_guard.wait() != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
  return hip_status(cai4::moe_combine(residual, sh, y, pos, wts, (int)T, H, k, out, st));
}

}  // namespace

extern "C" {

const char *cascadia_int4_version(void) { return "cascadia-int4-hip 0.1.0 (gfx950)"; }

int cascadia_int4_synchronize(void *stream) {
  return hip_status(hipStreamSynchronize((hipStream_t)stream));
}

int cascadia_int4_dequant_gemv(const cascadia_int4_layout *L, const uint8_t *packed,
                               const uint8_t *scale_bits, const float *x, float *y,
                               void *stream) {
  return cascadia_int4_dequant_gemm_multi(L, packed, scale_bits, x, 1, y, stream);
}

int cascadia_int4_dequant_gemv_rows_subset(const cascadia_int4_layout *L, const uint8_t *packed,
                                           const uint8_t *scale_bits, const float *x, float *y,
                                           const uint32_t *active_rows, uint32_t n_active,
                                           void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (int rc = check_weights(packed, scale_bits)) return rc;
  if (n_active == 0) return CASCADIA_INT4_OK;
  if (!x || !y || !active_rows) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x, 16) || !aligned(y, 4) || !aligned(active_rows, 4) || n_active > (1u << 30))
    return CASCADIA_INT4_ERR_ARG;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const cai4::SkinnyDevice d = device_props(dev);
  cai4::RowsMatrix w{};
  w.packed = packed;
  w.scales = scale_bits;
  w.N = (int)L->n_rows;
  w.K = (int)L->k_cols;
  w.G = (int)L->group_size;
  w.sdt = (int)L->scale_dtype;
  w.tiled = (int)L->tiling;
  return hip_status(cai4::rows_subset(w, x, false, active_rows, (int)n_active, y, d.max_lds,
                                      d.num_cus, static_cast<hipStream_t>(stream)));
}

int cascadia_int4_build_active_mask(const float *gate_out, uint32_t n, float threshold,
                                    const float *thresholds, float *silu_out,
                                    uint32_t *active_out, uint32_t *n_active_out,
                                    void *stream) {
  if (n == 0) return CASCADIA_INT4_OK;
  if (!gate_out || !silu_out || !active_out || !n_active_out) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(gate_out, 4) || !aligned(silu_out, 4) || !aligned(active_out, 4) ||
      !aligned(n_active_out, 4) || (thresholds && !aligned(thresholds, 4)) || n > (1u << 24))
    return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::build_active_mask(gate_out, (int)n, threshold, thresholds, silu_out,
                                            active_out, n_active_out,
                                            static_cast<hipStream_t>(stream)));
}

int cascadia_int4_f32_to_bf16(const float *x, size_t n, uint16_t *out_bf16, void *stream) {
  if (n == 0) return CASCADIA_INT4_OK;
  if (!x || !out_bf16) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x, 4) || !aligned(out_bf16, 2)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::f32_to_bf16_n(x, out_bf16, n, static_cast<hipStream_t>(stream)));
}

int cascadia_int4_bf16_to_f32(const uint16_t *x_bf16, size_t n, float *out, void *stream) {
  if (n == 0) return CASCADIA_INT4_OK;
  if (!x_bf16 || !out) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x_bf16, 2) || !aligned(out, 4)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::bf16_to_f32_n(x_bf16, out, n, static_cast<hipStream_t>(stream)));
}

int cascadia_int4_dequant_gemm_multi(const cascadia_int4_layout *L, const uint8_t *packed,
                                     const uint8_t *scale_bits, const float *xs, uint32_t seq,
                                     float *ys, void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (int rc = check_weights(packed, scale_bits)) return rc;
  if (!xs || !ys) return CASCADIA_INT4_ERR_NULL;
  if (seq == 0) return CASCADIA_INT4_ERR_ARG;  // the crate asserts seq >= 1
  if (!aligned(xs, 16) || !aligned(ys, 4)) return CASCADIA_INT4_ERR_ARG;
  return run_gemm(packed, scale_bits, nullptr, nullptr, (int)L->n_rows, (int)L->k_cols,
                  (int)L->group_size, (int)L->scale_dtype, (int)L->tiling, xs, nullptr, cai4::A_XF32, (int)seq,
                  ys, nullptr, cai4::EPI_F32, (hipStream_t)stream);
}

int cascadia_int4_dequant_gemm_bf16in(const cascadia_int4_layout *L, const uint8_t *packed,
                                      const uint8_t *scale_bits, const uint16_t *xs_bf16,
                                      uint32_t seq, float *ys, void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (int rc = check_weights(packed, scale_bits)) return rc;
  if (!xs_bf16 || !ys) return CASCADIA_INT4_ERR_NULL;
  if (seq == 0) return CASCADIA_INT4_ERR_ARG;
  if (!aligned(xs_bf16, 16) || !aligned(ys, 4)) return CASCADIA_INT4_ERR_ARG;
  if (prefill_shape(L, seq))
    return run_prefill(L, packed, scale_bits, xs_bf16, seq, ys, true, (hipStream_t)stream);
  return run_gemm(packed, scale_bits, nullptr, nullptr, (int)L->n_rows, (int)L->k_cols,
                  (int)L->group_size, (int)L->scale_dtype, (int)L->tiling, xs_bf16, nullptr,
                  cai4::A_BF16,
                  (int)seq, ys, nullptr, cai4::EPI_F32, (hipStream_t)stream);
}

int cascadia_int4_gemm_bf16(const cascadia_int4_layout *L, const uint8_t *packed,
                            const uint8_t *scale_bits, const uint16_t *xs_bf16, uint32_t seq,
                            uint16_t *ys_bf16, void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (int rc = check_weights(packed, scale_bits)) return rc;
  if (!xs_bf16 || !ys_bf16) return CASCADIA_INT4_ERR_NULL;
  if (seq == 0) return CASCADIA_INT4_ERR_ARG;
  if (!aligned(xs_bf16, 16) || !aligned(ys_bf16, 2)) return CASCADIA_INT4_ERR_ARG;
  if (prefill_shape(L, seq))
    return run_prefill(L, packed, scale_bits, xs_bf16, seq, ys_bf16, false, (hipStream_t)stream);
  return run_gemm(packed, scale_bits, nullptr, nullptr, (int)L->n_rows, (int)L->k_cols,
                  (int)L->group_size, (int)L->scale_dtype, (int)L->tiling, xs_bf16, nullptr,
                  cai4::A_BF16,
                  (int)seq, ys_bf16, nullptr, cai4::EPI_BF16, (hipStream_t)stream);
}

size_t cascadia_int4_expert_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size) {
  if (group_size == 0) return 0;
  size_t off[6];
  expert_sections(hidden, inter, group_size, off);
  return off[5] + (size_t)hidden * (inter / group_size) * 2;
}

int cascadia_int4_expert_from_flat(const uint8_t *flat, uint32_t hidden, uint32_t inter,
                                   uint32_t group_size, cascadia_int4_expert *out) {
  if (!flat || !out) return CASCADIA_INT4_ERR_NULL;
  if (group_size == 0 || group_size % 32 || hidden % group_size || inter % group_size)
    return CASCADIA_INT4_ERR_ARG;
  size_t off[6];
  expert_sections(hidden, inter, group_size, off);
  out->gate_packed = flat + off[0];
  out->gate_scale = flat + off[1];
  out->up_packed = flat + off[2];
  out->up_scale = flat + off[3];
  out->down_packed = flat + off[4];
  out->down_scale = flat + off[5];
  out->tiling = CASCADIA_INT4_TILING_CRATE;
  return CASCADIA_INT4_OK;
}

int cascadia_int4_tiled_sizes(const cascadia_int4_layout *L, size_t *packed_bytes,
                              size_t *scale_bytes) {
  if (int rc = check_layout(L)) return rc;
  if (!packed_bytes || !scale_bytes) return CASCADIA_INT4_ERR_NULL;
  cai4::tiled_sizes((int)L->n_rows, (int)L->k_cols, (int)L->group_size, packed_bytes,
                    scale_bytes);
  return CASCADIA_INT4_OK;
}

int cascadia_int4_tile_weights(const cascadia_int4_layout *L, const uint8_t *packed,
                               const uint8_t *scale_bits, uint8_t *packed_tiled,
                               uint8_t *scale_tiled, void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (int rc = check_weights(packed, scale_bits)) return rc;
  if (!packed_tiled || !scale_tiled) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(packed_tiled, 16) || !aligned(scale_tiled, 2)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::tile_weights(packed, scale_bits, (int)L->n_rows, (int)L->k_cols,
                                       (int)L->group_size, packed_tiled, scale_tiled,
                                       (hipStream_t)stream));
}


size_t cascadia_int4_expert_tiled_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size) {
  if (group_size == 0 || group_size % 32 || hidden % group_size || inter % group_size) return 0;
  size_t off[7];
  tiled_expert_sections(hidden, inter, group_size, off);
  return off[6];
}

int cascadia_int4_tile_expert(uint32_t hidden, uint32_t inter, uint32_t group_size,
                              const cascadia_int4_expert *src, uint8_t *dst,
                              cascadia_int4_expert *out, void *stream) {
  if (!dst || !out) return CASCADIA_INT4_ERR_NULL;
  if (int rc = check_expert(hidden, inter, group_size, 0, src)) return rc;
  if (src->tiling != CASCADIA_INT4_TILING_CRATE) return CASCADIA_INT4_ERR_ARG;
  if (!aligned(dst, 256)) return CASCADIA_INT4_ERR_ARG;
  size_t off[7];
  tiled_expert_sections(hidden, inter, group_size, off);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = cai4::tile_weights(src->gate_packed, src->gate_scale, (int)inter, (int)hidden,
                                    (int)group_size, dst + off[0], dst + off[1], st);
  if (e == hipSuccess)
    e = cai4::tile_weights(src->up_packed, src->up_scale, (int)inter, (int)hidden,
                           (int)group_size, dst + off[2], dst + off[3], st);
  if (e == hipSuccess)
    e = cai4::tile_weights(src->down_packed, src->down_scale, (int)hidden, (int)inter,
                           (int)group_size, dst + off[4], dst + off[5], st);
  if (e != hipSuccess) return CASCADIA_INT4_ERR_DEVICE;
  out->gate_packed = dst + off[0];
  out->gate_scale = dst + off[1];
  out->up_packed = dst + off[2];
  out->up_scale = dst + off[3];
  out->down_packed = dst + off[4];
  out->down_scale = dst + off[5];
  out->tiling = CASCADIA_INT4_TILING_MFMA;
  return CASCADIA_INT4_OK;
}

size_t cascadia_int4_ffn_workspace_bytes(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t n_tokens) {
  int dev;
  if (current_device(&dev)) return 0;
  if (group_size == 0 || group_size % 32) return 0;
  const FfnWorkspace f = ffn_workspace(dev, hidden, inter, group_size, n_tokens, true);
  const FfnWorkspace b = ffn_workspace(dev, hidden, inter, group_size, n_tokens, false);
  return f.total() > b.total() ? f.total() : b.total();
}

int cascadia_int4_expert_forward_device(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                        uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                        const uint16_t *x_bf16, uint32_t n_tokens,
                                        uint16_t *out_bf16, void *workspace, void *stream) {
  return ffn_common(hidden, inter, group_size, scale_dtype, expert, x_bf16, false,
                    n_tokens, out_bf16, true, workspace, (hipStream_t)stream);
}

int cascadia_int4_expert_forward_noalloc(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t scale_dtype,
                                         const cascadia_int4_expert *expert,
                                         const uint16_t *x_bf16, uint32_t n_tokens,
                                         uint16_t *out_bf16, void *stream) {
  if (int rc = check_expert(hidden, inter, group_size, scale_dtype, expert)) return rc;
  if (n_tokens == 0) return CASCADIA_INT4_OK;
  if (!x_bf16 || !out_bf16) return CASCADIA_INT4_ERR_NULL;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  const FfnWorkspace need = ffn_workspace(dev, hidden, inter, group_size, n_tokens, false);
  if (need.total() > kNoAllocScratchBytes) return CASCADIA_INT4_ERR_ARG;
  void *ws = nullptr;
  if (int rc = noalloc_scratch(dev, &ws)) return rc;
  return ffn_common(hidden, inter, group_size, scale_dtype, expert, x_bf16, false, n_tokens,
                    out_bf16, true, ws, (hipStream_t)stream);
}

int cascadia_int4_ffn_forward_f32(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                  uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                  const float *x, uint32_t n_tokens, float *out,
                                  void *workspace, void *stream) {
  return ffn_common(hidden, inter, group_size, scale_dtype, expert, x, true, n_tokens, out,
                    false, workspace, (hipStream_t)stream);
}

int cascadia_int4_transpose_requantize_down(uint32_t hidden, uint32_t inter,
                                            uint32_t group_size, uint32_t scale_dtype,
                                            const uint8_t *packed, const uint8_t *scale_bits,
                                            uint8_t *packed_t, uint8_t *scale_t_bits,
                                            void *stream) {
  if (!packed || !scale_bits || !packed_t || !scale_t_bits) return CASCADIA_INT4_ERR_NULL;
  if (hidden == 0 || inter == 0 || group_size == 0 || group_size % 32 || inter % group_size ||
      hidden % 32 || scale_dtype > 1 || hidden > (1u << 30) || inter > (1u << 30) ||
      (size_t)hidden * inter > ((size_t)1 << 34))
    return CASCADIA_INT4_ERR_ARG;
  if (!aligned(packed_t, 16) || !aligned(scale_bits, 2) || !aligned(scale_t_bits, 2))
    return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::transpose_requantize(packed, scale_bits, (int)hidden, (int)inter,
                                               (int)group_size, (int)scale_dtype, packed_t,
                                               scale_t_bits, (hipStream_t)stream));
}

size_t cascadia_int4_axpy_workspace_bytes(uint32_t hidden, uint32_t n_active) {
  return align256(cai4::axpy_plan((int)hidden, (int)n_active).partial_bytes);
}

int cascadia_int4_dequant_axpy_active(const uint8_t *packed_t, const uint8_t *scale_t_bits,
                                      const float *scalars, const uint32_t *active,
                                      uint32_t n_active, uint32_t inter, uint32_t hidden,
                                      float *y, void *workspace, void *stream) {
  if (!packed_t || !scale_t_bits || !scalars || !y || (n_active && !active))
    return CASCADIA_INT4_ERR_NULL;
  if (hidden == 0 || inter == 0 || hidden % 32 || hidden > (1u << 30) || inter > (1u << 30) ||
      n_active > (1u << 30))
    return CASCADIA_INT4_ERR_ARG;
  if (!aligned(packed_t, 16) || !aligned(scale_t_bits, 2) || !aligned(scalars, 4) ||
      !aligned(y, 4) || (active && !aligned(active, 4)) || (workspace && !aligned(workspace, 16)))
    return CASCADIA_INT4_ERR_ARG;
  if (n_active == 0) return CASCADIA_INT4_OK;
  const cai4::AxpyPlan p = cai4::axpy_plan((int)hidden, (int)n_active);
  void *ws = workspace;
  if (!ws) {
    int dev;
    if (int rc = current_device(&dev)) return rc;
    if (int rc = lib_workspace(dev, p.partial_bytes, &ws, (hipStream_t)stream)) return rc;
  }
  return hip_status(cai4::axpy_active(packed_t, scale_t_bits, scalars, active, (int)n_active,
                                      (int)hidden, (int)inter, static_cast<float *>(ws), y,
                                      (hipStream_t)stream));
}

size_t cascadia_int4_ffn_sparse_workspace_bytes(uint32_t hidden, uint32_t inter,
                                                uint32_t group_size, uint32_t n_tokens) {
  int dev;
  if (current_device(&dev)) return 0;
  if (group_size == 0 || group_size % 32) return 0;
  return sparse_workspace(dev, hidden, inter, group_size, n_tokens).total;
}

int cascadia_int4_ffn_forward_sparse_f32(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                         uint32_t scale_dtype,
                                         const cascadia_int4_expert *expert, const float *x,
                                         uint32_t n_tokens, float threshold,
                                         const float *thresholds, float *out,
                                         uint32_t *active_counts, void *workspace,
                                         void *stream) {
  return sparse_common(hidden, inter, group_size, scale_dtype, expert, x, true, n_tokens,
                       threshold, thresholds, out, false, active_counts, workspace,
                       (hipStream_t)stream);
}

int cascadia_int4_expert_forward_sparse(uint32_t hidden, uint32_t inter, uint32_t group_size,
                                        uint32_t scale_dtype, const cascadia_int4_expert *expert,
                                        const uint16_t *x_bf16, uint32_t n_tokens,
                                        float threshold, const float *thresholds,
                                        uint16_t *out_bf16, uint32_t *active_counts,
                                        void *workspace, void *stream) {
  return sparse_common(hidden, inter, group_size, scale_dtype, expert, x_bf16, false, n_tokens,
                       threshold, thresholds, out_bf16, true, active_counts, workspace,
                       (hipStream_t)stream);
}

int cascadia_int4_ov_to_crate(const uint8_t *packed_ov, size_t n_bytes, uint8_t *packed_crate,
                              void *stream) {
  if (n_bytes == 0) return CASCADIA_INT4_OK;
  if (!packed_ov || !packed_crate) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(packed_ov, 4) || !aligned(packed_crate, 4)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::ov_to_crate(packed_ov, n_bytes, packed_crate, (hipStream_t)stream));
}

size_t cascadia_int4_ov_gemv_workspace_bytes(const cascadia_int4_ov_segment *segs,
                                             uint32_t n_segs, uint32_t k_cols,
                                             uint32_t group_size, uint32_t rows) {
  int dev;
  if (!segs || current_device(&dev) || group_size == 0 || group_size % 32) return 0;
  const cai4::SkinnyDevice d = device_props(dev);
  size_t n_total = 0, part = 0;
  for (uint32_t i = 0; i < n_segs; ++i) {
    n_total += segs[i].n_rows;
    const size_t pb = cai4::skinny_plan((int)segs[i].n_rows, (int)k_cols, (int)group_size,
                                        (int)rows, cai4::A_XF32, cai4::EPI_F32, d)
                          .partial_bytes;
    part = pb > part ? pb : part;
  }
  return align256((size_t)rows * k_cols * 4) + align256((size_t)rows * n_total * 4) + part;
}

int cascadia_int4_ov_gemv(const cascadia_int4_ov_segment *segs, uint32_t n_segs,
                          uint32_t k_cols, uint32_t group_size, const void *act,
                          uint32_t act_f16, uint32_t rows, void *out, uint32_t out_f16,
                          void *workspace, void *stream) {
  if (!segs || !act || !out) return CASCADIA_INT4_ERR_NULL;
  if (n_segs == 0 || rows == 0 || k_cols == 0 || group_size == 0 || group_size % 32 ||
      k_cols % group_size || act_f16 > 1 || out_f16 > 1 || k_cols > (1u << 30))
    return CASCADIA_INT4_ERR_ARG;
  size_t n_total = 0;
  for (uint32_t i = 0; i < n_segs; ++i) {
    if (int rc = check_weights(segs[i].packed, segs[i].scale_f16)) return rc;
    if (segs[i].n_rows == 0 || segs[i].tiling > CASCADIA_INT4_TILING_MFMA)
      return CASCADIA_INT4_ERR_ARG;
    n_total += segs[i].n_rows;
  }
  if (n_total > (1u << 30) || !aligned(act, act_f16 ? 2 : 16) || !aligned(out, out_f16 ? 2 : 4) ||
      (workspace && !aligned(workspace, 256)))
    return CASCADIA_INT4_ERR_ARG;
  if (!act_fits((int)rows, (int)k_cols, cai4::A_XF32)) return CASCADIA_INT4_ERR_ARG;
  int dev;
  if (int rc = current_device(&dev)) return rc;
  hipStream_t st = (hipStream_t)stream;
  const size_t need =
      cascadia_int4_ov_gemv_workspace_bytes(segs, n_segs, k_cols, group_size, rows);
  void *ws = workspace;
  if (!ws) {
    if (int rc = lib_workspace(dev, need, &ws, st)) return rc;
  }
  uint8_t *b = static_cast<uint8_t *>(ws);
  const size_t act_b = align256((size_t)rows * k_cols * 4);
  const size_t out_b = align256((size_t)rows * n_total * 4);
  const float *x = static_cast<const float *>(act);
  if (act_f16) {  // the op's f16 activations (gemv_offload.cpp:485-488), exactly in f32
    float *xf = reinterpret_cast<float *>(b);
    if (hipError_t e = cai4::f16_to_f32(static_cast<const uint16_t *>(act),
                                        (size_t)rows * k_cols, xf, st))
      return hip_status(e);
    x = xf;
  }
  float *y = out_f16 ? reinterpret_cast<float *>(b + act_b) : static_cast<float *>(out);
  void *part = b + act_b + out_b;
  size_t start = 0;
  for (uint32_t i = 0; i < n_segs; ++i) {  // the segments' rows concatenated (:434-452)
    if (int rc = run_gemm(segs[i].packed, segs[i].scale_f16, nullptr, nullptr,
                          (int)segs[i].n_rows, (int)k_cols, (int)group_size,
                          CASCADIA_INT4_SCALE_F16, (int)segs[i].tiling, x, nullptr, cai4::A_XF32,
                          (int)rows, y + start, nullptr, cai4::EPI_F32, st, part, false,
                          (int)n_total))
      return rc;
    start += segs[i].n_rows;
  }
  if (out_f16)  // ov::float16(acc): round to nearest even
    return hip_status(cai4::f32_to_f16(y, (size_t)rows * n_total, static_cast<uint16_t *>(out),
                                       st));
  return CASCADIA_INT4_OK;
}

size_t cascadia_int4_ffn_sparse_axpy_workspace_bytes(uint32_t hidden, uint32_t inter,
                                                     uint32_t group_size, uint32_t n_tokens) {
  int dev;
  if (current_device(&dev)) return 0;
  if (group_size == 0 || group_size % 32) return 0;
  return axpy_ffn_workspace(dev, hidden, inter, group_size, n_tokens).total;
}

int cascadia_int4_ffn_forward_sparse_axpy_f32(uint32_t hidden, uint32_t inter,
                                              uint32_t group_size, uint32_t scale_dtype,
                                              const cascadia_int4_expert *expert, const float *x,
                                              uint32_t n_tokens, float threshold,
                                              const float *thresholds, float *out,
                                              uint32_t *active_counts, void *workspace,
                                              void *stream) {
  return axpy_ffn(hidden, inter, group_size, scale_dtype, expert, x, n_tokens, threshold,
                  thresholds, out, active_counts, workspace, (hipStream_t)stream);
}

int cascadia_int4_gate_up_silu(uint32_t hidden, uint32_t inter, uint32_t group_size,
                               uint32_t scale_dtype, const cascadia_int4_expert *expert,
                               const void *x, uint32_t x_is_f32, uint32_t n_tokens,
                               float *inter_out, void *stream) {
  if (int rc = check_expert(hidden, inter, group_size, scale_dtype, expert)) return rc;
  if (n_tokens == 0) return CASCADIA_INT4_OK;
  if (!x || !inter_out) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(x, 16) || !aligned(inter_out, 4)) return CASCADIA_INT4_ERR_ARG;
  return run_gemm(expert->gate_packed, expert->gate_scale, expert->up_packed, expert->up_scale,
                  (int)inter, (int)hidden, (int)group_size, (int)scale_dtype,
                  (int)expert->tiling, x, nullptr,
                  x_is_f32 ? cai4::A_XF32 : cai4::A_BF16, (int)n_tokens, inter_out, nullptr,
                  cai4::EPI_SWIGLU, (hipStream_t)stream);
}

int cascadia_int4_debug_dequant(const cascadia_int4_layout *L, const uint8_t *packed,
                                const uint8_t *scale_bits, float *w_out, void *stream) {
  if (int rc = check_layout(L)) return rc;
  if (L->tiling != CASCADIA_INT4_TILING_CRATE) return CASCADIA_INT4_ERR_ARG;
  if (!packed || !scale_bits || !w_out) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(packed, 4) || !aligned(scale_bits, 2) || !aligned(w_out, 4))
    return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::debug_dequant(packed, scale_bits, (int)L->n_rows, (int)L->k_cols,
                                        (int)L->group_size, (int)L->scale_dtype, w_out,
                                        (hipStream_t)stream));
}

int cascadia_int4_quantize_bf16(const uint16_t *w_bf16, uint32_t n_rows, uint32_t k_cols,
                                uint32_t group_size, uint8_t *packed, uint16_t *scale_bits,
                                void *stream) {
  if (!w_bf16 || !packed || !scale_bits) return CASCADIA_INT4_ERR_NULL;
  if (n_rows == 0 || k_cols == 0 || group_size == 0 || group_size % 32 ||
      k_cols % group_size || n_rows > (1u << 30) || k_cols > (1u << 30))
    return CASCADIA_INT4_ERR_ARG;
  if (!aligned(w_bf16, 16) || !aligned(packed, 4) || !aligned(scale_bits, 2))
    return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::quantize_group(w_bf16, (int)n_rows, (int)k_cols, (int)group_size,
                                         packed, scale_bits, (hipStream_t)stream));
}

int cascadia_int4_stream_read(const void *buf, size_t bytes, uint32_t *sink, void *stream) {
  if (bytes == 0) return CASCADIA_INT4_OK;
  if (!buf || !sink) return CASCADIA_INT4_ERR_NULL;
  if (!aligned(buf, 16) || bytes % 16 || !aligned(sink, 4)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::stream_read(buf, bytes, sink, static_cast<hipStream_t>(stream)));
}

int cascadia_int4_fill_synthetic(uint32_t kind, uint64_t seed, uint64_t stream_id, size_t n,
                                 double p0, double p1, uint32_t dtype, void *out,
                                 void *stream) {
  if (!out) return CASCADIA_INT4_ERR_NULL;
  if (kind > 3 || dtype > 1) return CASCADIA_INT4_ERR_ARG;
  if (kind == 0 && !aligned(out, 8)) return CASCADIA_INT4_ERR_ARG;
  if (kind == 2 && !aligned(out, 4)) return CASCADIA_INT4_ERR_ARG;
  if ((kind == 1 || kind == 3) && !aligned(out, 2)) return CASCADIA_INT4_ERR_ARG;
  return hip_status(cai4::fill_synthetic((int)kind, seed, stream_id, n, p0, p1, (int)dtype, out,
                                         (hipStream_t)stream));
}

size_t cascadia_int4_moe_workspace_bytes(const cascadia_int4_moe_layer *layer, uint32_t top_k,
                                         uint32_t n_tokens) {
  if (moe_check(layer, top_k, n_tokens)) return 0;
  int dev;
  if (current_device(&dev)) return 0;
  const MoePlan a = moe_plan(dev, layer, top_k, n_tokens, false);
  const MoePlan b = moe_plan(dev, layer, top_k, n_tokens, true);
  return a.ws.total > b.ws.total ? a.ws.total : b.ws.total;
}

int cascadia_int4_moe_forward(const cascadia_int4_moe_layer *layer,
                              const cascadia_int4_routing *routing, const float *x,
                              const float *residual, uint32_t n_tokens, float *out,
                              int32_t *ids_out, float *weights_out, void *workspace,
                              void *stream) {
  return moe_forward(layer, routing, x, residual, n_tokens, out, ids_out, weights_out, workspace,
                     (hipStream_t)stream);
}

}  // extern "C"
