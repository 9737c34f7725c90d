/* cascadia_int4.hpp -- C++17 host API over libcascadia_int4_hip.so, mirroring
 * the public API of the crate crates/cascadia-int4-gemm (src/lib.rs:29-78):
 * the same function names, argument order and meaning, and error behaviour
 * (the crate's assert_eq! panics become std::invalid_argument; its GemmError
 * is cascadia_int4::GemmError; a HIP failure is cascadia_int4::DeviceError).
 *
 * What differs from the crate, by design:
 *  - Slices are device memory (HBM).  DeviceSlice<T> is a pointer and an
 *    element count; DeviceBuffer<T> owns one.  Weights are uploaded once.
 *  - Every call is synchronous by default, as the crate's are; with
 *    Options::synchronize = false it is only enqueued on Options::stream.
 *  - Options carry what the crate fixes at compile time: the group size (any
 *    multiple of 32; the crate: 32), the scale dtype (bf16 as the crate, or
 *    fp16) and the weight layout (the crate's bytes, or the MFMA-tiled copy of
 *    ExpertWeights::tiled() / tile_weights()).
 *
 * Header-only; link with -lcascadia_int4_hip -lamdhip64.
 */
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "cascadia_int4.h"

namespace cascadia_int4 {

// Architecture constants of K2.6 (lib.rs:71-78).
constexpr size_t HIDDEN = 7168;
constexpr size_t INTERMEDIATE = 2048;
constexpr size_t GROUP_SIZE = 32;
constexpr size_t NIBBLES_PER_INT32 = 8;
constexpr size_t GROUPS_IN = HIDDEN / GROUP_SIZE;
constexpr size_t GROUPS_MID = INTERMEDIATE / GROUP_SIZE;
constexpr size_t PACKED_COLS_IN = HIDDEN / NIBBLES_PER_INT32;
constexpr size_t PACKED_COLS_MID = INTERMEDIATE / NIBBLES_PER_INT32;

enum class ScaleDtype : uint32_t { Bf16 = CASCADIA_INT4_SCALE_BF16, F16 = CASCADIA_INT4_SCALE_F16 };
enum class Tiling : uint32_t {
  Crate = CASCADIA_INT4_TILING_CRATE,
  Mfma = CASCADIA_INT4_TILING_MFMA,
  MfmaUpRows = CASCADIA_INT4_TILING_MFMA_UP_ROWS,  // sparse entry points only
};

struct Options {
  size_t group_size = GROUP_SIZE;
  ScaleDtype scale_dtype = ScaleDtype::Bf16;
  Tiling tiling = Tiling::Crate;
  hipStream_t stream = nullptr;
  bool synchronize = true;     // the crate's calls return with the result written
  void *workspace = nullptr;   // null: the library's per-device buffer
};

// A HIP or device-memory failure (the C ABI's -3 / -4).
class DeviceError : public std::runtime_error {
 public:
  DeviceError(const std::string &fn, int code)
      : std::runtime_error(fn + " failed with " + std::to_string(code)), code(code) {}
  int code;
};

// format.rs:28-33: an I/O error, or a file too small for the expert.
class GemmError : public std::runtime_error {
 public:
  enum class Kind { Io, Truncated };
  GemmError(Kind kind, const std::string &what, size_t expected = 0, size_t actual = 0)
      : std::runtime_error(what), kind(kind), expected(expected), actual(actual) {}
  Kind kind;
  size_t expected, actual;
};

template <class T>
struct DeviceSlice {
  T *data = nullptr;
  size_t len = 0;
  DeviceSlice() = default;
  DeviceSlice(T *data, size_t len) : data(data), len(len) {}
  template <class U>  // DeviceSlice<const T> from DeviceSlice<T>
  DeviceSlice(const DeviceSlice<U> &o) : data(o.data), len(o.len) {}
  size_t size() const { return len; }
};

// An owned device array (hipMalloc / hipFree); move-only.
template <class T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t len) : len_(len) {
    if (len && hipMalloc(reinterpret_cast<void **>(&p_), len * sizeof(T)) != hipSuccess)
      throw DeviceError("hipMalloc", CASCADIA_INT4_ERR_NOMEM);
  }
  ~DeviceBuffer() {
    if (p_) (void)hipFree(p_);
  }
  DeviceBuffer(DeviceBuffer &&o) noexcept : p_(o.p_), len_(o.len_) { o.p_ = nullptr, o.len_ = 0; }
  DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
    std::swap(p_, o.p_);
    std::swap(len_, o.len_);
    return *this;
  }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
  T *data() const { return p_; }
  size_t size() const { return len_; }
  DeviceSlice<T> slice() const { return {p_, len_}; }
  operator DeviceSlice<T>() const { return slice(); }
  operator DeviceSlice<const T>() const { return {p_, len_}; }
  // host -> device / device -> host copies of the whole buffer
  void upload(const T *host) { upload(host, 0, len_); }
  // host[0 .. count) -> elements [offset, offset + count)
  void upload(const T *host, size_t offset, size_t count) {
    if (offset > len_ || count > len_ - offset)
      throw std::out_of_range("DeviceBuffer::upload past the end");
    if (count && hipMemcpy(p_ + offset, host, count * sizeof(T), hipMemcpyHostToDevice) !=
                     hipSuccess)
      throw DeviceError("hipMemcpy", CASCADIA_INT4_ERR_DEVICE);
  }
  std::vector<T> download() const {
    std::vector<T> h(len_);
    if (len_ && hipMemcpy(h.data(), p_, len_ * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
      throw DeviceError("hipMemcpy", CASCADIA_INT4_ERR_DEVICE);
    return h;
  }

 private:
  T *p_ = nullptr;
  size_t len_ = 0;
};

namespace detail {

inline void require(bool ok, const char *what) {
  if (!ok) throw std::invalid_argument(what);
}

// The C ABI's status codes: -1 / -2 are the crate's panics, the rest device errors.
inline void check(int rc, const char *fn) {
  if (rc == CASCADIA_INT4_OK) return;
  if (rc == CASCADIA_INT4_ERR_NULL || rc == CASCADIA_INT4_ERR_ARG)
    throw std::invalid_argument(std::string(fn) + ": invalid argument (" + std::to_string(rc) + ")");
  throw DeviceError(fn, rc);
}

inline void finish(const Options &o) {
  if (o.synchronize) check(cascadia_int4_synchronize(o.stream), "cascadia_int4_synchronize");
}

inline cascadia_int4_layout layout(size_t n_rows, size_t k_cols, const Options &o) {
  require(n_rows <= UINT32_MAX && k_cols <= UINT32_MAX && o.group_size <= UINT32_MAX,
          "dimensions exceed 32 bits");
  return cascadia_int4_layout{(uint32_t)n_rows, (uint32_t)k_cols, (uint32_t)o.group_size,
                              (uint32_t)o.scale_dtype, (uint32_t)o.tiling};
}

// The byte sizes of one matrix's codes and scales in the options' layout.
inline std::pair<size_t, size_t> matrix_bytes(size_t n_rows, size_t k_cols, const Options &o) {
  require(o.group_size > 0 && o.group_size % 32 == 0 && k_cols % o.group_size == 0,
          "k_cols must be a multiple of the group size, itself a multiple of 32");
  if (o.tiling == Tiling::Crate)
    return {n_rows * k_cols / 2, n_rows * (k_cols / o.group_size) * 2};
  cascadia_int4_layout l = layout(n_rows, k_cols, o);
  l.tiling = CASCADIA_INT4_TILING_MFMA;
  size_t p = 0, s = 0;
  check(cascadia_int4_tiled_sizes(&l, &p, &s), "cascadia_int4_tiled_sizes");
  return {p, s};
}

inline void matrix_args(DeviceSlice<const uint8_t> packed, DeviceSlice<const uint8_t> scale_bits,
                        size_t n_rows, size_t k_cols, const Options &o) {
  const auto sz = matrix_bytes(n_rows, k_cols, o);
  require(packed.len == sz.first, "packed length does not match n_rows x k_cols");
  require(scale_bits.len == sz.second, "scale length does not match n_rows x k_cols / group");
}

struct Expert {
  cascadia_int4_expert e;
  size_t hidden, inter;
};

// The six slices of one expert and its dims: hidden from the caller (the
// crate: x's length), inter from the gate scales' length (kernel.rs:86).
inline Expert expert(size_t hidden, DeviceSlice<const uint8_t> gp, DeviceSlice<const uint8_t> gs,
                     DeviceSlice<const uint8_t> up, DeviceSlice<const uint8_t> us,
                     DeviceSlice<const uint8_t> dp, DeviceSlice<const uint8_t> ds,
                     const Options &o, size_t inter = 0) {
  require(hidden > 0 && hidden % o.group_size == 0, "hidden must be a multiple of the group size");
  if (!inter) {
    require(o.tiling == Tiling::Crate, "inter must be given for tiled weights");
    inter = gs.len / 2 / (hidden / o.group_size);
  }
  Options up_o = o;
  if (o.tiling == Tiling::MfmaUpRows) up_o.tiling = Tiling::Crate;
  Options gd_o = o;
  if (o.tiling == Tiling::MfmaUpRows) gd_o.tiling = Tiling::Mfma;
  matrix_args(gp, gs, inter, hidden, gd_o);
  matrix_args(up, us, inter, hidden, up_o);
  return Expert{{gp.data, gs.data, up.data, us.data, dp.data, ds.data, (uint32_t)o.tiling}, hidden,
                inter};
}

inline void down_args(const Expert &x, DeviceSlice<const uint8_t> dp,
                      DeviceSlice<const uint8_t> ds, const Options &o) {
  Options gd_o = o;
  if (o.tiling == Tiling::MfmaUpRows) gd_o.tiling = Tiling::Mfma;
  matrix_args(dp, ds, x.hidden, x.inter, gd_o);
}

// Per-thread device scratch for the active counts the sparse calls return,
// one word on each device the thread calls on (the sparse calls read it back
// before they return, so a thread's calls never overlap on it).
inline uint32_t *count_scratch() {
  constexpr int kMaxDevices = 64;
  thread_local DeviceBuffer<uint32_t> bufs[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    throw DeviceError("hipGetDevice", CASCADIA_INT4_ERR_DEVICE);
  if (!bufs[dev].data()) bufs[dev] = DeviceBuffer<uint32_t>(1);
  return bufs[dev].data();
}

// The count a sparse call left in count_scratch() (waits for the call).
inline uint32_t read_count(const Options &o) {
  uint32_t n = 0;
  if (hipMemcpyAsync(&n, count_scratch(), 4, hipMemcpyDeviceToHost, o.stream) != hipSuccess ||
      hipStreamSynchronize(o.stream) != hipSuccess)
    throw DeviceError("hipMemcpyAsync", CASCADIA_INT4_ERR_DEVICE);
  return n;
}

// The crate's return value of the sparse calls: active lanes / inter.
inline float active_fraction(size_t inter, const Options &o) {
  const uint32_t n = read_count(o);
  return inter ? (float)n / (float)inter : 0.f;
}

}  // namespace detail

// ---- scalar conversions (format.rs:130-160) ----

inline float bf16_bits_to_f32(uint16_t bits) {
  const uint32_t u = (uint32_t)bits << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Round to nearest even; a NaN stays a quiet NaN.
inline uint16_t f32_to_bf16_bits(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x0040u);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// ---- GEMV / GEMM (kernel.rs:31-71, kernel_avx512.rs:92, kernel_avx512_multi.rs:207,
// kernel_avx512_multi_blocked.rs:295) ----

inline void dequant_gemv_int4(DeviceSlice<const uint8_t> packed,
                              DeviceSlice<const uint8_t> scale_bits, DeviceSlice<const float> x,
                              size_t n_rows, size_t k_cols, DeviceSlice<float> y,
                              const Options &o = {}) {
  detail::matrix_args(packed, scale_bits, n_rows, k_cols, o);
  detail::require(x.len == k_cols, "x length must be k_cols");
  detail::require(y.len == n_rows, "y length must be n_rows");
  const cascadia_int4_layout l = detail::layout(n_rows, k_cols, o);
  detail::check(cascadia_int4_dequant_gemv(&l, packed.data, scale_bits.data, x.data, y.data,
                                           o.stream),
                "cascadia_int4_dequant_gemv");
  detail::finish(o);
}

inline void dequant_gemv_int4_auto(DeviceSlice<const uint8_t> packed,
                                   DeviceSlice<const uint8_t> scale_bits,
                                   DeviceSlice<const float> x, size_t n_rows, size_t k_cols,
                                   DeviceSlice<float> y, const Options &o = {}) {
  dequant_gemv_int4(packed, scale_bits, x, n_rows, k_cols, y, o);
}

inline void dequant_gemm_int4_multi_auto(DeviceSlice<const uint8_t> packed,
                                         DeviceSlice<const uint8_t> scale_bits,
                                         DeviceSlice<const float> xs, size_t n_rows,
                                         size_t k_cols, size_t seq, DeviceSlice<float> ys,
                                         const Options &o = {}) {
  detail::matrix_args(packed, scale_bits, n_rows, k_cols, o);
  detail::require(xs.len == seq * k_cols, "xs length must be seq x k_cols");
  detail::require(ys.len == seq * n_rows, "ys length must be seq x n_rows");
  detail::require(seq <= UINT32_MAX, "seq exceeds 32 bits");
  const cascadia_int4_layout l = detail::layout(n_rows, k_cols, o);
  detail::check(cascadia_int4_dequant_gemm_multi(&l, packed.data, scale_bits.data, xs.data,
                                                 (uint32_t)seq, ys.data, o.stream),
                "cascadia_int4_dequant_gemm_multi");
  detail::finish(o);
}

inline void dequant_gemm_int4_multi_blocked_auto(DeviceSlice<const uint8_t> packed,
                                                 DeviceSlice<const uint8_t> scale_bits,
                                                 DeviceSlice<const float> xs, size_t n_rows,
                                                 size_t k_cols, size_t seq,
                                                 DeviceSlice<float> ys, const Options &o = {}) {
  dequant_gemm_int4_multi_auto(packed, scale_bits, xs, n_rows, k_cols, seq, ys, o);
}

// ffn_sparsity.rs:187-348: y[r] for the listed rows only (others untouched).
inline void dequant_gemv_int4_rows_subset(DeviceSlice<const uint8_t> packed,
                                          DeviceSlice<const uint8_t> scale_bits,
                                          DeviceSlice<const float> x, size_t n_rows,
                                          size_t k_cols, DeviceSlice<float> y,
                                          DeviceSlice<const uint32_t> active_rows,
                                          const Options &o = {}) {
  detail::matrix_args(packed, scale_bits, n_rows, k_cols, o);
  detail::require(x.len == k_cols, "x length must be k_cols");
  detail::require(y.len == n_rows, "y length must be n_rows");
  detail::require(active_rows.len <= UINT32_MAX, "too many active rows");
  const cascadia_int4_layout l = detail::layout(n_rows, k_cols, o);
  detail::check(cascadia_int4_dequant_gemv_rows_subset(&l, packed.data, scale_bits.data, x.data,
                                                       y.data, active_rows.data,
                                                       (uint32_t)active_rows.len, o.stream),
                "cascadia_int4_dequant_gemv_rows_subset");
  detail::finish(o);
}

inline void dequant_gemv_int4_rows_subset_auto(DeviceSlice<const uint8_t> packed,
                                               DeviceSlice<const uint8_t> scale_bits,
                                               DeviceSlice<const float> x, size_t n_rows,
                                               size_t k_cols, DeviceSlice<float> y,
                                               DeviceSlice<const uint32_t> active_rows,
                                               const Options &o = {}) {
  dequant_gemv_int4_rows_subset(packed, scale_bits, x, n_rows, k_cols, y, active_rows, o);
}

// ---- the expert FFN (kernel.rs:75-136) ----

// x_bf16, out_bf16: one token of hidden bf16 values (hidden = x's length).
inline void expert_forward(DeviceSlice<const uint16_t> x_bf16, DeviceSlice<const uint8_t> gate_p,
                           DeviceSlice<const uint8_t> gate_s, DeviceSlice<const uint8_t> up_p,
                           DeviceSlice<const uint8_t> up_s, DeviceSlice<const uint8_t> down_p,
                           DeviceSlice<const uint8_t> down_s, DeviceSlice<uint16_t> out_bf16,
                           const Options &o = {}, size_t inter = 0) {
  const detail::Expert e =
      detail::expert(x_bf16.len, gate_p, gate_s, up_p, up_s, down_p, down_s, o, inter);
  detail::down_args(e, down_p, down_s, o);
  detail::require(out_bf16.len == e.hidden, "out length must be hidden");
  detail::require(o.tiling != Tiling::MfmaUpRows, "the up-rows layout is for the sparse calls");
  detail::check(cascadia_int4_expert_forward_device((uint32_t)e.hidden, (uint32_t)e.inter,
                                                    (uint32_t)o.group_size,
                                                    (uint32_t)o.scale_dtype, &e.e, x_bf16.data,
                                                    1, out_bf16.data, o.workspace, o.stream),
                "cascadia_int4_expert_forward_device");
  detail::finish(o);
}

// ffn_sparsity.rs:71-91.  Global: one cutoff for every lane (<= 0: dense);
// PerChannel: a device array of inter cutoffs (dense when none is > 0).
class SparsityMode {
 public:
  static SparsityMode Global(float threshold) { return SparsityMode(threshold, {}); }
  static SparsityMode PerChannel(DeviceSlice<const float> thresholds) {
    return SparsityMode(0.f, thresholds);
  }
  bool per_channel() const { return per_channel_; }
  float threshold() const { return threshold_; }
  DeviceSlice<const float> thresholds() const { return thresholds_; }
  // Global: the crate's `t <= 0` (a NaN is sparse).  PerChannel needs the
  // device values: the library decides on the device.
  bool is_dense_global() const { return !per_channel_ && threshold_ <= 0.f; }

 private:
  SparsityMode(float t, DeviceSlice<const float> th)
      : threshold_(t), thresholds_(th), per_channel_(th.data != nullptr) {}
  float threshold_;
  DeviceSlice<const float> thresholds_;
  bool per_channel_;
};

// expert_forward_sparse_mode (ffn_sparsity.rs:812-867): returns the active fraction.
inline float expert_forward_sparse_mode(DeviceSlice<const uint16_t> x_bf16,
                                        DeviceSlice<const uint8_t> gate_p,
                                        DeviceSlice<const uint8_t> gate_s,
                                        DeviceSlice<const uint8_t> up_p,
                                        DeviceSlice<const uint8_t> up_s,
                                        DeviceSlice<const uint8_t> down_p,
                                        DeviceSlice<const uint8_t> down_s,
                                        DeviceSlice<uint16_t> out_bf16, SparsityMode mode,
                                        const Options &o = {}, size_t inter = 0) {
  const detail::Expert e =
      detail::expert(x_bf16.len, gate_p, gate_s, up_p, up_s, down_p, down_s, o, inter);
  detail::down_args(e, down_p, down_s, o);
  detail::require(out_bf16.len == e.hidden, "out length must be hidden");
  if (mode.per_channel())
    detail::require(mode.thresholds().len == e.inter, "one threshold per intermediate lane");
  detail::check(cascadia_int4_expert_forward_sparse(
                    (uint32_t)e.hidden, (uint32_t)e.inter, (uint32_t)o.group_size,
                    (uint32_t)o.scale_dtype, &e.e, x_bf16.data, 1, mode.threshold(),
                    mode.thresholds().data, out_bf16.data, detail::count_scratch(), o.workspace,
                    o.stream),
                "cascadia_int4_expert_forward_sparse");
  return detail::active_fraction(e.inter, o);
}

inline float expert_forward_sparse(DeviceSlice<const uint16_t> x_bf16,
                                   DeviceSlice<const uint8_t> gate_p,
                                   DeviceSlice<const uint8_t> gate_s,
                                   DeviceSlice<const uint8_t> up_p,
                                   DeviceSlice<const uint8_t> up_s,
                                   DeviceSlice<const uint8_t> down_p,
                                   DeviceSlice<const uint8_t> down_s,
                                   DeviceSlice<uint16_t> out_bf16, float threshold,
                                   const Options &o = {}, size_t inter = 0) {
  return expert_forward_sparse_mode(x_bf16, gate_p, gate_s, up_p, up_s, down_p, down_s, out_bf16,
                                    SparsityMode::Global(threshold), o, inter);
}

inline float expert_forward_sparse_per_channel(
    DeviceSlice<const uint16_t> x_bf16, DeviceSlice<const uint8_t> gate_p,
    DeviceSlice<const uint8_t> gate_s, DeviceSlice<const uint8_t> up_p,
    DeviceSlice<const uint8_t> up_s, DeviceSlice<const uint8_t> down_p,
    DeviceSlice<const uint8_t> down_s, DeviceSlice<uint16_t> out_bf16,
    DeviceSlice<const float> thresholds, const Options &o = {}, size_t inter = 0) {
  return expert_forward_sparse_mode(x_bf16, gate_p, gate_s, up_p, up_s, down_p, down_s, out_bf16,
                                    SparsityMode::PerChannel(thresholds), o, inter);
}

// ffn_forward_sparse_f32_mode (ffn_sparsity.rs:438-538): f32 in / out (the
// shared expert's form); returns the active fraction.
inline float ffn_forward_sparse_f32_mode(DeviceSlice<const float> x_f32, size_t hidden,
                                         size_t intermediate, DeviceSlice<const uint8_t> gate_p,
                                         DeviceSlice<const uint8_t> gate_s,
                                         DeviceSlice<const uint8_t> up_p,
                                         DeviceSlice<const uint8_t> up_s,
                                         DeviceSlice<const uint8_t> down_p,
                                         DeviceSlice<const uint8_t> down_s,
                                         DeviceSlice<float> out_f32, SparsityMode mode,
                                         const Options &o = {}) {
  const detail::Expert e =
      detail::expert(hidden, gate_p, gate_s, up_p, up_s, down_p, down_s, o, intermediate);
  detail::down_args(e, down_p, down_s, o);
  detail::require(x_f32.len == hidden && out_f32.len == hidden, "x and out must be hidden long");
  if (mode.per_channel())
    detail::require(mode.thresholds().len == intermediate, "one threshold per intermediate lane");
  detail::check(cascadia_int4_ffn_forward_sparse_f32(
                    (uint32_t)hidden, (uint32_t)intermediate, (uint32_t)o.group_size,
                    (uint32_t)o.scale_dtype, &e.e, x_f32.data, 1, mode.threshold(),
                    mode.thresholds().data, out_f32.data, detail::count_scratch(), o.workspace,
                    o.stream),
                "cascadia_int4_ffn_forward_sparse_f32");
  return detail::active_fraction(intermediate, o);
}

inline float ffn_forward_sparse_f32(DeviceSlice<const float> x_f32, size_t hidden,
                                    size_t intermediate, DeviceSlice<const uint8_t> gate_p,
                                    DeviceSlice<const uint8_t> gate_s,
                                    DeviceSlice<const uint8_t> up_p,
                                    DeviceSlice<const uint8_t> up_s,
                                    DeviceSlice<const uint8_t> down_p,
                                    DeviceSlice<const uint8_t> down_s, DeviceSlice<float> out_f32,
                                    float threshold, const Options &o = {}) {
  return ffn_forward_sparse_f32_mode(x_f32, hidden, intermediate, gate_p, gate_s, up_p, up_s,
                                     down_p, down_s, out_f32, SparsityMode::Global(threshold), o);
}

inline float ffn_forward_sparse_f32_per_channel(
    DeviceSlice<const float> x_f32, size_t hidden, size_t intermediate,
    DeviceSlice<const uint8_t> gate_p, DeviceSlice<const uint8_t> gate_s,
    DeviceSlice<const uint8_t> up_p, DeviceSlice<const uint8_t> up_s,
    DeviceSlice<const uint8_t> down_p, DeviceSlice<const uint8_t> down_s,
    DeviceSlice<float> out_f32, DeviceSlice<const float> thresholds, const Options &o = {}) {
  return ffn_forward_sparse_f32_mode(x_f32, hidden, intermediate, gate_p, gate_s, up_p, up_s,
                                     down_p, down_s, out_f32,
                                     SparsityMode::PerChannel(thresholds), o);
}

// build_active_mask_mode (ffn_sparsity.rs:131-179) on one row of gate values.
struct ActiveMask {
  DeviceBuffer<float> silu;       // the stable SiLU of every lane
  DeviceBuffer<uint32_t> active;  // the active lanes, ascending (active.size() of them)
};

inline ActiveMask build_active_mask_mode(DeviceSlice<const float> gate_out, SparsityMode mode,
                                         const Options &o = {}) {
  detail::require(gate_out.len > 0 && gate_out.len <= UINT32_MAX, "gate_out length");
  if (mode.per_channel())
    detail::require(mode.thresholds().len == gate_out.len, "one threshold per lane");
  DeviceBuffer<float> silu(gate_out.len);
  DeviceBuffer<uint32_t> active(gate_out.len);
  detail::check(cascadia_int4_build_active_mask(gate_out.data, (uint32_t)gate_out.len,
                                                mode.threshold(), mode.thresholds().data,
                                                silu.data(), active.data(),
                                                detail::count_scratch(), o.stream),
                "cascadia_int4_build_active_mask");
  const size_t n = detail::read_count(o);
  DeviceBuffer<uint32_t> list(n);
  if (n && hipMemcpyAsync(list.data(), active.data(), n * 4, hipMemcpyDeviceToDevice, o.stream) !=
               hipSuccess)
    throw DeviceError("hipMemcpyAsync", CASCADIA_INT4_ERR_DEVICE);
  detail::check(cascadia_int4_synchronize(o.stream), "cascadia_int4_synchronize");
  return ActiveMask{std::move(silu), std::move(list)};
}

inline ActiveMask build_active_mask(DeviceSlice<const float> gate_out, float threshold,
                                    const Options &o = {}) {
  return build_active_mask_mode(gate_out, SparsityMode::Global(threshold), o);
}

inline ActiveMask build_active_mask_per_channel(DeviceSlice<const float> gate_out,
                                                DeviceSlice<const float> thresholds,
                                                const Options &o = {}) {
  return build_active_mask_mode(gate_out, SparsityMode::PerChannel(thresholds), o);
}

// ---- the AXPY form (ffn_axpy.rs:82-440, ffn_sparsity.rs:569-740) ----

// transpose_requantize_down (ffn_axpy.rs:342-440): the down matrix [hidden,
// inter] (crate layout) -> (packed_t [inter, hidden / 2], bf16 scale_t
// [inter, hidden / 32]).
inline std::pair<DeviceBuffer<uint8_t>, DeviceBuffer<uint8_t>> transpose_requantize_down(
    DeviceSlice<const uint8_t> src_packed, DeviceSlice<const uint8_t> src_scale_bits,
    size_t n_hidden, size_t n_intermediate, const Options &o = {}) {
  Options c = o;
  c.tiling = Tiling::Crate;
  detail::matrix_args(src_packed, src_scale_bits, n_hidden, n_intermediate, c);
  detail::require(n_hidden % 32 == 0, "hidden must be a multiple of 32");
  DeviceBuffer<uint8_t> pt(n_intermediate * n_hidden / 2), st(n_intermediate * (n_hidden / 32) * 2);
  detail::check(cascadia_int4_transpose_requantize_down(
                    (uint32_t)n_hidden, (uint32_t)n_intermediate, (uint32_t)o.group_size,
                    (uint32_t)o.scale_dtype, src_packed.data, src_scale_bits.data, pt.data(),
                    st.data(), o.stream),
                "cascadia_int4_transpose_requantize_down");
  detail::finish(o);
  return {std::move(pt), std::move(st)};
}

// dequant_axpy_int4_active (ffn_axpy.rs:82-160): y[hidden] += sum over the
// active lanes a of scalars[a] * dequant(packed_t[a, :]).
inline void dequant_axpy_int4_active(DeviceSlice<const uint8_t> packed_t,
                                     DeviceSlice<const uint8_t> scale_t_bits,
                                     DeviceSlice<const float> scalars,
                                     DeviceSlice<const uint32_t> active, size_t n_intermediate,
                                     size_t n_hidden, DeviceSlice<float> y,
                                     const Options &o = {}) {
  detail::require(packed_t.len == n_intermediate * n_hidden / 2, "packed_t length");
  detail::require(scale_t_bits.len == n_intermediate * (n_hidden / 32) * 2, "scale_t length");
  detail::require(scalars.len == n_intermediate && y.len == n_hidden, "scalars / y length");
  detail::require(active.len <= UINT32_MAX, "too many active lanes");
  detail::check(cascadia_int4_dequant_axpy_active(packed_t.data, scale_t_bits.data, scalars.data,
                                                  active.data, (uint32_t)active.len,
                                                  (uint32_t)n_intermediate, (uint32_t)n_hidden,
                                                  y.data, o.workspace, o.stream),
                "cascadia_int4_dequant_axpy_active");
  detail::finish(o);
}

inline void dequant_axpy_int4_active_auto(DeviceSlice<const uint8_t> packed_t,
                                          DeviceSlice<const uint8_t> scale_t_bits,
                                          DeviceSlice<const float> scalars,
                                          DeviceSlice<const uint32_t> active,
                                          size_t n_intermediate, size_t n_hidden,
                                          DeviceSlice<float> y, const Options &o = {}) {
  dequant_axpy_int4_active(packed_t, scale_t_bits, scalars, active, n_intermediate, n_hidden, y,
                           o);
}

// The crate's FfnScratch (ffn_axpy.rs:452-500): here the device workspace of
// the AXPY-form FFN, grown on demand.
class FfnScratch {
 public:
  FfnScratch() = default;
  FfnScratch(size_t hidden, size_t intermediate, size_t group = GROUP_SIZE) {
    resize_for(hidden, intermediate, group);
  }
  void resize_for(size_t hidden, size_t intermediate, size_t group = GROUP_SIZE) {
    const size_t b = cascadia_int4_ffn_sparse_axpy_workspace_bytes(
        (uint32_t)hidden, (uint32_t)intermediate, (uint32_t)group, 1);
    if (b > ws_.size()) ws_ = DeviceBuffer<uint8_t>(b);
  }
  void *data() const { return ws_.data(); }

 private:
  DeviceBuffer<uint8_t> ws_;
};

// ffn_forward_sparse_axpy_f32_mode (ffn_sparsity.rs:638-740): the down slots
// hold transpose_requantize_down's output; returns the active fraction.
inline float ffn_forward_sparse_axpy_f32_mode(
    FfnScratch &scratch, DeviceSlice<const float> x_f32, size_t hidden, size_t intermediate,
    DeviceSlice<const uint8_t> gate_p, DeviceSlice<const uint8_t> gate_s,
    DeviceSlice<const uint8_t> up_p, DeviceSlice<const uint8_t> up_s,
    DeviceSlice<const uint8_t> down_packed_t, DeviceSlice<const uint8_t> down_scale_t_bits,
    DeviceSlice<float> out_f32, SparsityMode mode, const Options &o = {}) {
  const detail::Expert e = detail::expert(hidden, gate_p, gate_s, up_p, up_s, down_packed_t,
                                          down_scale_t_bits, o, intermediate);
  detail::require(down_packed_t.len == intermediate * hidden / 2, "down_packed_t length");
  detail::require(down_scale_t_bits.len == intermediate * (hidden / 32) * 2,
                  "down_scale_t length");
  detail::require(x_f32.len == hidden && out_f32.len == hidden, "x and out must be hidden long");
  if (mode.per_channel())
    detail::require(mode.thresholds().len == intermediate, "one threshold per intermediate lane");
  scratch.resize_for(hidden, intermediate, o.group_size);
  detail::check(cascadia_int4_ffn_forward_sparse_axpy_f32(
                    (uint32_t)hidden, (uint32_t)intermediate, (uint32_t)o.group_size,
                    (uint32_t)o.scale_dtype, &e.e, x_f32.data, 1, mode.threshold(),
                    mode.thresholds().data, out_f32.data, detail::count_scratch(),
                    scratch.data(), o.stream),
                "cascadia_int4_ffn_forward_sparse_axpy_f32");
  return detail::active_fraction(intermediate, o);
}

inline float ffn_forward_sparse_axpy_f32(
    FfnScratch &scratch, DeviceSlice<const float> x_f32, size_t hidden, size_t intermediate,
    DeviceSlice<const uint8_t> gate_p, DeviceSlice<const uint8_t> gate_s,
    DeviceSlice<const uint8_t> up_p, DeviceSlice<const uint8_t> up_s,
    DeviceSlice<const uint8_t> down_packed_t, DeviceSlice<const uint8_t> down_scale_t_bits,
    DeviceSlice<float> out_f32, float threshold, const Options &o = {}) {
  return ffn_forward_sparse_axpy_f32_mode(scratch, x_f32, hidden, intermediate, gate_p, gate_s,
                                          up_p, up_s, down_packed_t, down_scale_t_bits, out_f32,
                                          SparsityMode::Global(threshold), o);
}

inline float ffn_forward_sparse_axpy_f32_per_channel(
    FfnScratch &scratch, DeviceSlice<const float> x_f32, size_t hidden, size_t intermediate,
    DeviceSlice<const uint8_t> gate_p, DeviceSlice<const uint8_t> gate_s,
    DeviceSlice<const uint8_t> up_p, DeviceSlice<const uint8_t> up_s,
    DeviceSlice<const uint8_t> down_packed_t, DeviceSlice<const uint8_t> down_scale_t_bits,
    DeviceSlice<float> out_f32, DeviceSlice<const float> thresholds, const Options &o = {}) {
  return ffn_forward_sparse_axpy_f32_mode(scratch, x_f32, hidden, intermediate, gate_p, gate_s,
                                          up_p, up_s, down_packed_t, down_scale_t_bits, out_f32,
                                          SparsityMode::PerChannel(thresholds), o);
}

// ---- load time (shell_int4.rs:148-212) ----

// bf16 weights [n_rows, k_cols] -> (packed codes, bf16 scales) in the crate
// layout, groups of Options::group_size.
inline std::pair<DeviceBuffer<uint8_t>, DeviceBuffer<uint8_t>> quantize_int4_group(
    DeviceSlice<const uint16_t> weight_bf16, size_t n_rows, size_t k_cols, const Options &o = {}) {
  detail::require(weight_bf16.len == n_rows * k_cols, "weight length must be n_rows x k_cols");
  detail::require(k_cols % o.group_size == 0, "k_cols must be a multiple of the group size");
  DeviceBuffer<uint8_t> packed(n_rows * k_cols / 2), scales(n_rows * (k_cols / o.group_size) * 2);
  detail::check(cascadia_int4_quantize_bf16(weight_bf16.data, (uint32_t)n_rows, (uint32_t)k_cols,
                                            (uint32_t)o.group_size, packed.data(),
                                            reinterpret_cast<uint16_t *>(scales.data()),
                                            o.stream),
                "cascadia_int4_quantize_bf16");
  detail::finish(o);
  return {std::move(packed), std::move(scales)};
}

// ---- one expert's weights (format.rs:51-125) ----

// The six sections of one expert in HBM, in the crate's flat order
// (gate | gate_s | up | up_s | down | down_s) or, after tiled(), in the
// MFMA-tiled layout.  Owns its device memory.
class ExpertWeights {
 public:
  // format.rs:63-96: read a flat expert file (K2.6 dims by default) into HBM.
  static ExpertWeights open(const std::string &path, size_t hidden = HIDDEN,
                            size_t intermediate = INTERMEDIATE, size_t group = GROUP_SIZE,
                            ScaleDtype sdt = ScaleDtype::Bf16) {
    const size_t need = cascadia_int4_expert_bytes((uint32_t)hidden, (uint32_t)intermediate,
                                                   (uint32_t)group);
    detail::require(need > 0, "unsupported expert dims");
    std::FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) throw GemmError(GemmError::Kind::Io, "io: cannot open " + path);
    std::vector<uint8_t> host(need);
    const size_t got = std::fread(host.data(), 1, need, f);
    const bool err = std::ferror(f) != 0;
    std::fclose(f);
    if (err) throw GemmError(GemmError::Kind::Io, "io: read error on " + path);
    if (got < need)
      throw GemmError(GemmError::Kind::Truncated,
                      "file too small: expected at least " + std::to_string(need) + ", got " +
                          std::to_string(got),
                      need, got);
    return from_host(host.data(), need, hidden, intermediate, group, sdt);
  }

  // One flat expert already in host memory (no crate counterpart: open's
  // upload without the file), exactly cascadia_int4_expert_bytes long.
  static ExpertWeights from_host(const uint8_t *flat, size_t len, size_t hidden,
                                 size_t intermediate, size_t group = GROUP_SIZE,
                                 ScaleDtype sdt = ScaleDtype::Bf16) {
    const size_t need = cascadia_int4_expert_bytes((uint32_t)hidden, (uint32_t)intermediate,
                                                   (uint32_t)group);
    detail::require(need > 0, "unsupported expert dims");
    detail::require(flat && len == need, "flat expert length does not match its dims");
    ExpertWeights w(hidden, intermediate, group, sdt, Tiling::Crate, DeviceBuffer<uint8_t>(need));
    w.blob_.upload(flat);
    w.slice();
    return w;
  }

  // The MFMA-tiled copy (faster kernels; the same results bit for bit).
  ExpertWeights tiled() const {
    detail::require(tiling_ == Tiling::Crate, "already tiled");
    DeviceBuffer<uint8_t> t(cascadia_int4_expert_tiled_bytes((uint32_t)hidden_, (uint32_t)inter_,
                                                             (uint32_t)group_));
    cascadia_int4_expert out{};
    detail::check(cascadia_int4_tile_expert((uint32_t)hidden_, (uint32_t)inter_, (uint32_t)group_,
                                            &e_, t.data(), &out, nullptr),
                  "cascadia_int4_tile_expert");
    detail::check(cascadia_int4_synchronize(nullptr), "cascadia_int4_synchronize");
    ExpertWeights w(hidden_, inter_, group_, sdt_, Tiling::Mfma, std::move(t));
    w.e_ = out;
    return w;
  }

  DeviceSlice<const uint8_t> gate_packed_bytes() const { return part(0); }
  DeviceSlice<const uint8_t> gate_scale_bits() const { return part(1); }
  DeviceSlice<const uint8_t> up_packed_bytes() const { return part(2); }
  DeviceSlice<const uint8_t> up_scale_bits() const { return part(3); }
  DeviceSlice<const uint8_t> down_packed_bytes() const { return part(4); }
  DeviceSlice<const uint8_t> down_scale_bits() const { return part(5); }

  // The options the entry points need for these weights.
  Options options() const {
    Options o;
    o.group_size = group_;
    o.scale_dtype = sdt_;
    o.tiling = tiling_;
    return o;
  }
  size_t hidden() const { return hidden_; }
  size_t intermediate() const { return inter_; }
  const cascadia_int4_expert &c_expert() const { return e_; }

 private:
  ExpertWeights(size_t h, size_t i, size_t g, ScaleDtype s, Tiling t, DeviceBuffer<uint8_t> b)
      : hidden_(h), inter_(i), group_(g), sdt_(s), tiling_(t), blob_(std::move(b)) {}
  void slice() {
    detail::check(cascadia_int4_expert_from_flat(blob_.data(), (uint32_t)hidden_, (uint32_t)inter_,
                                                 (uint32_t)group_, &e_),
                  "cascadia_int4_expert_from_flat");
  }
  DeviceSlice<const uint8_t> part(int k) const {
    Options o = options();
    const auto gu = detail::matrix_bytes(inter_, hidden_, o);
    const auto dn = detail::matrix_bytes(hidden_, inter_, o);
    const uint8_t *p[6] = {e_.gate_packed, e_.gate_scale, e_.up_packed,
                           e_.up_scale,    e_.down_packed, e_.down_scale};
    const size_t n[6] = {gu.first, gu.second, gu.first, gu.second, dn.first, dn.second};
    return {p[k], n[k]};
  }
  size_t hidden_, inter_, group_;
  ScaleDtype sdt_;
  Tiling tiling_;
  DeviceBuffer<uint8_t> blob_;
  cascadia_int4_expert e_{};
};

// expert_forward over an ExpertWeights (its dims, layout and dtype).
inline void expert_forward(const ExpertWeights &w, DeviceSlice<const uint16_t> x_bf16,
                           DeviceSlice<uint16_t> out_bf16, const Options &call = {}) {
  Options o = w.options();
  o.stream = call.stream;
  o.synchronize = call.synchronize;
  o.workspace = call.workspace;
  detail::require(x_bf16.len == w.hidden(), "x length must be the expert's hidden size");
  expert_forward(x_bf16, w.gate_packed_bytes(), w.gate_scale_bits(), w.up_packed_bytes(),
                 w.up_scale_bits(), w.down_packed_bytes(), w.down_scale_bits(), out_bf16, o,
                 w.intermediate());
}

// ---- the sparse-MoE layer (runner.rs:1806-1832, batched over tokens) ----

// The routed experts of one layer in one device blob: expert e at e * stride()
// (a multiple of 256), in the crate's flat order or MFMA-tiled.
class ExpertStack {
 public:
  // n_experts flat experts (format.rs:35-47) back to back in host memory;
  // o.tiling Crate keeps their bytes, Mfma tiles each on the device.
  static ExpertStack upload(const uint8_t *host_flat, size_t n_experts, size_t hidden,
                            size_t intermediate, const Options &o = {}) {
    detail::require(host_flat && n_experts > 0, "no experts");
    detail::require(o.tiling == Tiling::Crate || o.tiling == Tiling::Mfma,
                    "experts are crate-layout or MFMA-tiled");
    const uint32_t h = (uint32_t)hidden, i = (uint32_t)intermediate, g = (uint32_t)o.group_size;
    const size_t flat = cascadia_int4_expert_bytes(h, i, g);
    detail::require(flat > 0, "unsupported expert dims");
    const size_t per = o.tiling == Tiling::Crate ? flat : cascadia_int4_expert_tiled_bytes(h, i, g);
    ExpertStack s(hidden, intermediate, n_experts, (per + 255) / 256 * 256, o);
    s.blob_ = DeviceBuffer<uint8_t>(n_experts * s.stride_);
    if (o.tiling == Tiling::Crate) {  // each expert at its stride; the padding is never read
      for (size_t e = 0; e < n_experts; ++e) s.blob_.upload(host_flat + e * flat, e * s.stride_, flat);
      return s;
    }
    DeviceBuffer<uint8_t> one(flat);
    for (size_t e = 0; e < n_experts; ++e) {
      one.upload(host_flat + e * flat);
      cascadia_int4_expert src{}, dst{};
      detail::check(cascadia_int4_expert_from_flat(one.data(), h, i, g, &src),
                    "cascadia_int4_expert_from_flat");
      detail::check(cascadia_int4_tile_expert(h, i, g, &src, s.blob_.data() + e * s.stride_, &dst,
                                              nullptr),
                    "cascadia_int4_tile_expert");
      // `one` is refilled by the next upload: the tiling must have read it
      detail::check(cascadia_int4_synchronize(nullptr), "cascadia_int4_synchronize");
    }
    return s;
  }
  const uint8_t *data() const { return blob_.data(); }
  size_t stride() const { return stride_; }
  size_t n_experts() const { return n_; }
  size_t hidden() const { return hidden_; }
  size_t intermediate() const { return inter_; }
  Options options() const { return o_; }

 private:
  ExpertStack(size_t h, size_t i, size_t n, size_t stride, const Options &o)
      : hidden_(h), inter_(i), n_(n), stride_(stride), o_(o) {}
  size_t hidden_, inter_, n_, stride_;
  Options o_;
  DeviceBuffer<uint8_t> blob_;
};

// One layer's experts: the routed stack and an optional shared expert
// (shell_int4.rs:629) of the same hidden size, group, scale dtype and layout.
// Refers to, does not own, the weights.
class MoeLayer {
 public:
  explicit MoeLayer(const ExpertStack &routed) {
    const Options o = routed.options();
    detail::require(routed.n_experts() <= 1024, "at most 1024 experts");
    l_.hidden = (uint32_t)routed.hidden();
    l_.inter = (uint32_t)routed.intermediate();
    l_.group_size = (uint32_t)o.group_size;
    l_.scale_dtype = (uint32_t)o.scale_dtype;
    l_.tiling = (uint32_t)o.tiling;
    l_.n_experts = (uint32_t)routed.n_experts();
    l_.experts = routed.data();
    l_.expert_stride = routed.stride();
  }
  MoeLayer &with_shared(const ExpertWeights &shared) {
    const Options s = shared.options();
    detail::require(shared.hidden() == l_.hidden && s.group_size == l_.group_size &&
                        (uint32_t)s.scale_dtype == l_.scale_dtype &&
                        (uint32_t)s.tiling == l_.tiling,
                    "the shared expert must match the routed experts' hidden size, group, "
                    "scale dtype and layout");
    l_.shared = shared.c_expert();
    l_.shared_inter = (uint32_t)shared.intermediate();
    return *this;
  }
  size_t hidden() const { return l_.hidden; }
  size_t n_experts() const { return l_.n_experts; }
  bool has_shared() const { return l_.shared.gate_packed != nullptr; }
  const cascadia_int4_moe_layer &c_layer() const { return l_; }
  // device workspace bytes of moe_forward (Options::workspace)
  size_t workspace_bytes(size_t top_k, size_t n_tokens) const {
    return cascadia_int4_moe_workspace_bytes(&l_, (uint32_t)top_k, (uint32_t)n_tokens);
  }

 private:
  cascadia_int4_moe_layer l_{};
};

// How tokens pick their top_k experts (shell_int4.rs:588-620, glm/gate.rs:24-62,
// or given ids / weights); slots with a weight below threshold are skipped
// (runner.rs:1811).
class Routing {
 public:
  // s = sigmoid(logit); top_k by s + bias (ties to the lower id);
  // w = s / (sum s + 1e-20) * scale when normalize, else s * scale.
  static Routing sigmoid_bias(DeviceSlice<const float> logits, size_t top_k, float scale,
                              bool normalize, DeviceSlice<const float> bias = {}) {
    Routing r(CASCADIA_INT4_ROUTE_SIGMOID_BIAS, top_k);
    r.r_.logits = logits.data;
    r.r_.bias = bias.data;
    r.r_.scale = scale;
    r.r_.normalize = normalize ? 1u : 0u;
    r.logits_len_ = logits.len;
    r.bias_len_ = bias.len;
    return r;
  }
  // the top_k logits (ties to the lower id), w = softmax over them
  static Routing softmax_topk(DeviceSlice<const float> logits, size_t top_k) {
    Routing r(CASCADIA_INT4_ROUTE_SOFTMAX_TOPK, top_k);
    r.r_.logits = logits.data;
    r.logits_len_ = logits.len;
    return r;
  }
  // [n_tokens, top_k] expert ids and weights
  static Routing given(DeviceSlice<const int32_t> ids, DeviceSlice<const float> weights,
                       size_t top_k) {
    Routing r(CASCADIA_INT4_ROUTE_IDS, top_k);
    detail::require(ids.len == weights.len, "ids and weights differ in length");
    r.r_.ids = ids.data;
    r.r_.weights = weights.data;
    r.ids_len_ = ids.len;
    return r;
  }
  Routing &threshold(float t) {
    r_.threshold = t;
    return *this;
  }
  size_t top_k() const { return r_.top_k; }
  const cascadia_int4_routing &c_routing() const { return r_; }

  // the argument lengths for n_tokens tokens over n_experts
  void check(size_t n_tokens, size_t n_experts) const {
    detail::require(r_.top_k >= 1 && r_.top_k <= 16 && r_.top_k <= n_experts,
                    "top_k must be 1..16 and at most the expert count");
    if (r_.mode == CASCADIA_INT4_ROUTE_IDS) {
      detail::require(ids_len_ == n_tokens * r_.top_k, "ids must be n_tokens x top_k");
      return;
    }
    detail::require(logits_len_ == n_tokens * n_experts, "logits must be n_tokens x n_experts");
    detail::require(bias_len_ == 0 || bias_len_ == n_experts, "bias must be n_experts long");
  }

 private:
  Routing(uint32_t mode, size_t top_k) {
    detail::require(top_k <= 16, "top_k must be at most 16");
    r_.mode = mode;
    r_.top_k = (uint32_t)top_k;
    r_.scale = 1.f;
  }
  cascadia_int4_routing r_{};
  size_t logits_len_ = 0, bias_len_ = 0, ids_len_ = 0;
};

// One MoE layer for n_tokens tokens: out_t = residual_t + shared(x_t) +
// sum over the routed slots, in slot order, of w * bf16->f32(expert(bf16(x_t)))
// (runner.rs:1806-1832).  x, out, residual (empty: zero): f32 [n_tokens,
// hidden]; ids_out / weights_out (may be empty) receive the routing.  call
// supplies the stream, synchronisation and workspace.
inline void moe_forward(const MoeLayer &layer, const Routing &routing,
                        DeviceSlice<const float> x, size_t n_tokens, DeviceSlice<float> out,
                        DeviceSlice<const float> residual = {},
                        DeviceSlice<int32_t> ids_out = {}, DeviceSlice<float> weights_out = {},
                        const Options &call = {}) {
  const size_t h = layer.hidden(), k = routing.top_k();
  detail::require(n_tokens > 0 && n_tokens <= UINT32_MAX, "n_tokens must be 1..2^32-1");
  routing.check(n_tokens, layer.n_experts());
  detail::require(x.len == n_tokens * h && out.len == n_tokens * h,
                  "x and out must be n_tokens x hidden");
  detail::require(residual.data == nullptr || residual.len == n_tokens * h,
                  "residual must be n_tokens x hidden");
  detail::require(ids_out.data == nullptr || ids_out.len == n_tokens * k,
                  "ids_out must be n_tokens x top_k");
  detail::require(weights_out.data == nullptr || weights_out.len == n_tokens * k,
                  "weights_out must be n_tokens x top_k");
  detail::check(cascadia_int4_moe_forward(&layer.c_layer(), &routing.c_routing(), x.data,
                                          residual.data, (uint32_t)n_tokens, out.data,
                                          ids_out.data, weights_out.data, call.workspace,
                                          call.stream),
                "cascadia_int4_moe_forward");
  detail::finish(call);
}

// ---- the crate's C handle API (c_ffi.rs:35-341) as an owning object ----

// A model directory (safetensors, or an int4_bin manifest with flat expert
// files) whose experts are read once and kept in HBM.  Calls are
// synchronous; the handle serialises them.
class Source {
 public:
  struct CacheStats {
    uint64_t cached, evictions, resident_bytes;
  };
  struct PrefetchStats {
    uint64_t submits, drops, processed, loaded;
  };

  // c_ffi.rs open_source: -2 (invalid UTF-8) -> invalid_argument, -3 (not a
  // model directory) -> GemmError::Io.
  static Source open(const std::string &model_dir) {
    CascadiaInt4Source *h = nullptr;
    const int rc = cascadia_int4_open_source(model_dir.c_str(), &h);
    if (rc == -3) throw GemmError(GemmError::Kind::Io, "io: cannot open model dir " + model_dir);
    if (rc != 0)
      throw std::invalid_argument("cascadia_int4_open_source: " + std::to_string(rc));
    return Source(h);
  }
  ~Source() { cascadia_int4_destroy_source(h_); }
  Source(Source &&o) noexcept : h_(o.h_) { o.h_ = nullptr; }
  Source &operator=(Source &&o) noexcept {
    std::swap(h_, o.h_);
    return *this;
  }
  Source(const Source &) = delete;
  Source &operator=(const Source &) = delete;

  // Read (layer, expert) into HBM now.
  void prewarm(uint32_t layer, uint32_t expert) {
    expert_call(cascadia_int4_prewarm(h_, layer, expert), layer, expert);
  }
  // x, out: host arrays of the model's hidden size; f32 -> bf16 at entry,
  // bf16 -> f32 at exit (c_ffi.rs:323-339).
  void expert_forward(uint32_t layer, uint32_t expert, const float *x, float *out) {
    detail::require(x && out, "null x or out");
    expert_call(cascadia_int4_expert_forward(h_, layer, expert, x, out), layer, expert);
  }
  std::vector<float> expert_forward(uint32_t layer, uint32_t expert, const std::vector<float> &x) {
    std::vector<float> out(x.size());
    expert_forward(layer, expert, x.data(), out.data());
    return out;
  }

  // The expert cache (runner.rs:148-170): at most max_experts resident and
  // max_bytes of HBM (0 = unbounded); lowering a limit evicts at once.
  void set_cache_limits(uint64_t max_experts, uint64_t max_bytes) {
    device_call(cascadia_int4_source_set_cache_limits(h_, max_experts, max_bytes),
                "cascadia_int4_source_set_cache_limits");
  }
  CacheStats cache_stats() const {
    CacheStats s{};
    device_call(cascadia_int4_source_cache_stats(h_, &s.cached, &s.evictions, &s.resident_bytes),
                "cascadia_int4_source_cache_stats");
    return s;
  }

  // The runner's Prefetcher (runner.rs:282-360): queue (layer, expert) for the
  // handle's loader thread; never blocks (a full queue drops the request).
  void prefetch(uint32_t layer, uint32_t expert) {
    device_call(cascadia_int4_prefetch(h_, layer, expert), "cascadia_int4_prefetch");
  }
  void prefetch_wait() { device_call(cascadia_int4_prefetch_wait(h_), "cascadia_int4_prefetch_wait"); }
  PrefetchStats prefetch_stats() const {
    PrefetchStats s{};
    device_call(cascadia_int4_prefetch_stats(h_, &s.submits, &s.drops, &s.processed, &s.loaded),
                "cascadia_int4_prefetch_stats");
    return s;
  }

  CascadiaInt4Source *handle() const { return h_; }

 private:
  explicit Source(CascadiaInt4Source *h) : h_(h) {}
  // -2: the expert cannot be read (missing, short, or not in the index)
  static void expert_call(int rc, uint32_t layer, uint32_t expert) {
    if (rc == -2)
      throw GemmError(GemmError::Kind::Io, "io: cannot read expert " + std::to_string(expert) +
                                               " of layer " + std::to_string(layer));
    device_call(rc, "cascadia_int4 source call");
  }
  static void device_call(int rc, const char *fn) {
    if (rc == 0) return;
    if (rc == -1) throw std::invalid_argument(std::string(fn) + ": null handle");
    throw DeviceError(fn, rc);
  }
  CascadiaInt4Source *h_ = nullptr;
};

}  // namespace cascadia_int4
