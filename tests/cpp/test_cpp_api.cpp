// The C++ host API (include/cascadia_int4.hpp) on the GPU against the CPU
// oracle (oracle/int4_oracle.h, test infrastructure): every call through the
// header, on seeded inputs, at the parity bars (rel-L2 <= 1e-3, max-abs <=
// 2e-2 against the f32-accumulated CPU result; codes, scales and active lists
// exact), plus the crate's error behaviour (length mismatch -> invalid
// argument, a missing or short expert file -> GemmError).
//
// usage: test_cpp_api <fixture expert .bin (hidden 64, inter 32, G32 bf16)>
// Prints one line per check and "cpp api: N checks OK"; exit status 1 on the
// first failure.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include <sys/stat.h>
#include <unistd.h>

#include "cascadia_int4.hpp"
#include "../../oracle/int4_oracle.h"

namespace ci = cascadia_int4;

namespace {

int g_checks = 0;

[[noreturn]] void fail(const std::string &what) {
  std::printf("FAIL %s\n", what.c_str());
  std::fflush(stdout);
  std::exit(1);
}

void pass(const std::string &what) {
  ++g_checks;
  std::printf("ok   %s\n", what.c_str());
}

double rel_l2(const std::vector<float> &got, const std::vector<float> &want) {
  double n = 0, d = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double e = (double)got[i] - (double)want[i];
    n += e * e;
    d += (double)want[i] * want[i];
  }
  return d > 0 ? std::sqrt(n / d) : std::sqrt(n);
}

double max_abs(const std::vector<float> &got, const std::vector<float> &want) {
  double m = 0;
  for (size_t i = 0; i < got.size(); ++i) m = std::fmax(m, std::fabs((double)got[i] - want[i]));
  return m;
}

void check_close(const std::vector<float> &got, const std::vector<float> &want, const std::string &what) {
  if (got.size() != want.size()) fail(what + ": sizes differ");
  const double r = rel_l2(got, want), m = max_abs(got, want);
  if (!(r <= 1e-3 && m <= 2e-2)) fail(what + ": rel_l2 " + std::to_string(r) + " max_abs " + std::to_string(m));
  pass(what + " (rel_l2 " + std::to_string(r) + ")");
}

std::vector<float> bf16_to_f32(const std::vector<uint16_t> &b);

// bf16 outputs: every element within max-abs 2e-2 or one bf16 ulp of the
// reference (two roundings of nearly equal f32 sums may land one ulp apart),
// rel-L2 <= 1e-3 over the whole
void check_close_bf16(const std::vector<uint16_t> &got_b, const std::vector<uint16_t> &want_b,
                      const std::string &what) {
  const std::vector<float> got = bf16_to_f32(got_b), want = bf16_to_f32(want_b);
  if (got.size() != want.size()) fail(what + ": sizes differ");
  const double r = rel_l2(got, want);
  if (!(r <= 1e-3)) fail(what + ": rel_l2 " + std::to_string(r));
  for (size_t i = 0; i < got.size(); ++i) {
    const double w = std::fabs((double)want[i]);
    const double ulp = std::ldexp(1.0, (int)std::floor(std::log2(std::fmax(w, 0x1p-126))) - 7);
    if (std::fabs((double)got[i] - want[i]) > std::fmax(2e-2, ulp))
      fail(what + ": element " + std::to_string(i) + " off by more than one bf16 ulp");
  }
  pass(what + " (rel_l2 " + std::to_string(r) + ")");
}

template <class T>
ci::DeviceBuffer<T> dev(const std::vector<T> &h) {
  ci::DeviceBuffer<T> d(h.size());
  d.upload(h.data());
  return d;
}

std::vector<float> bf16_to_f32(const std::vector<uint16_t> &b) {
  std::vector<float> f(b.size());
  for (size_t i = 0; i < b.size(); ++i) f[i] = or_bf16_to_f32(b[i]);
  return f;
}

std::vector<uint8_t> bytes(uint64_t seed, uint64_t stream, size_t n) {
  std::vector<uint8_t> v(n);
  or_fill_bytes(seed, stream, n, v.data());
  return v;
}

std::vector<uint8_t> scales(uint64_t seed, uint64_t stream, size_t n) {
  std::vector<uint16_t> v(n);
  or_fill_scales(seed, stream, n, OR_SCALE_BF16, 0.02, 1e-3, v.data());
  return std::vector<uint8_t>(reinterpret_cast<uint8_t *>(v.data()),
                              reinterpret_cast<uint8_t *>(v.data()) + 2 * n);
}

std::vector<float> normal(uint64_t seed, uint64_t stream, size_t n) {
  std::vector<float> v(n);
  or_fill_normal_f32(seed, stream, n, v.data());
  return v;
}

template <class F>
void expect_invalid(F f, const std::string &what) {
  try {
    f();
  } catch (const std::invalid_argument &) {
    pass(what + " -> invalid_argument");
    return;
  }
  fail(what + ": no invalid_argument");
}

// One expert in the crate's flat layout, seeded.
struct HostExpert {
  size_t hidden, inter, group;
  std::vector<uint8_t> flat;
  size_t off[6];
  std::vector<uint8_t> part(int k) const {
    const size_t end = k < 5 ? off[k + 1] : flat.size();
    return std::vector<uint8_t>(flat.begin() + off[k], flat.begin() + end);
  }
};

HostExpert make_expert(size_t hidden, size_t inter, size_t group, uint64_t seed) {
  HostExpert e{hidden, inter, group, bytes(seed, 1, or_expert_bytes(hidden, inter, group)), {}};
  or_expert_offsets(hidden, inter, group, e.off);
  for (int k = 1; k < 6; k += 2) {
    const size_t n = (k < 5 ? e.off[k + 1] : e.flat.size()) - e.off[k];
    const std::vector<uint8_t> s = scales(seed, 10 + k, n / 2);
    std::copy(s.begin(), s.end(), e.flat.begin() + e.off[k]);
  }
  return e;
}

double bf16_ulp(double v) {
  return std::ldexp(1.0, (int)std::floor(std::log2(std::fmax(std::fabs(v), 0x1p-126))) - 7);
}

// One MoE layer's output against the oracle's layer on the GPU's own routing
// (a near-tie resolved one libm ulp apart cannot move a token between the
// sides): h and h - residual (the experts' part) within rel-L2 1e-3, every
// element within max-abs 2e-2 or, where routed outputs are large enough that
// one bf16 ulp exceeds that, within sum_k w_k ulp(y_k) plus 1e-5 max |h - x|
// (each expert output is rounded to bf16, kernel.rs:133-135).
void check_moe(const std::vector<float> &got, const std::vector<float> &x, size_t T, size_t h,
               size_t inter, const std::vector<uint8_t> &experts, size_t stride, size_t E,
               const HostExpert *shared, const std::vector<int32_t> &ids,
               const std::vector<float> &w, size_t k, float thr, const std::string &what) {
  std::vector<int64_t> ids64(ids.begin(), ids.end());
  std::vector<float> want(T * h);
  or_moe_layer(x.data(), T, h, inter, 32, OR_SCALE_BF16, OR_ORDER_AVX512, experts.data(), stride,
               E, shared ? shared->flat.data() : nullptr, shared ? shared->inter : 0,
               ids64.data(), w.data(), k, thr, want.data());
  const double r = rel_l2(got, want);
  std::vector<float> dg(T * h), dw(T * h);
  double dmax = 0;
  for (size_t q = 0; q < T * h; ++q) {
    dg[q] = got[q] - x[q];
    dw[q] = want[q] - x[q];
    dmax = std::fmax(dmax, std::fabs((double)dw[q]));
  }
  const double rd = rel_l2(dg, dw);
  if (!(r <= 1e-3 && rd <= 1e-3))
    fail(what + ": rel_l2 " + std::to_string(r) + ", experts' part " + std::to_string(rd));
  for (size_t t = 0; t < T; ++t) {
    std::vector<uint16_t> xb(h), y(h);
    for (size_t c = 0; c < h; ++c) xb[c] = or_f32_to_bf16(x[t * h + c]);
    std::vector<double> allow(h, 0.0);
    for (size_t s = 0; s < k; ++s) {
      if (w[t * k + s] < thr) continue;
      const uint8_t *e = experts.data() + (size_t)ids[t * k + s] * stride;
      or_expert_forward(xb.data(), h, inter, 32, OR_SCALE_BF16, OR_ORDER_AVX512, e, y.data());
      for (size_t c = 0; c < h; ++c)
        allow[c] += std::fabs((double)w[t * k + s]) * bf16_ulp(or_bf16_to_f32(y[c]));
    }
    for (size_t c = 0; c < h; ++c) {
      const double a = std::fmax(2e-2, allow[c] + 1e-5 * dmax);
      if (std::fabs((double)got[t * h + c] - want[t * h + c]) > a)
        fail(what + ": token " + std::to_string(t) + " element " + std::to_string(c));
    }
  }
  pass(what + " (rel_l2 " + std::to_string(r) + ", experts' part " + std::to_string(rd) + ")");
}

void write_file(const std::string &path, const std::string &text) {
  std::FILE *f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(text.data(), 1, text.size(), f) != text.size()) fail("write " + path);
  std::fclose(f);
}

}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    std::printf("usage: %s <fixture expert .bin>\n", argv[0]);
    return 2;
  }
  try {
    // ---- scalar conversions (format.rs:130-160) ----
    {
      const float vals[] = {0.f, -0.f, 1.f, 1.00390625f, 1.01171875f, -3.5e-39f, 65504.f,
                            3.4e38f, INFINITY, -INFINITY, NAN, 1e-45f, 0.333333343f};
      for (float v : vals) {
        if (ci::f32_to_bf16_bits(v) != or_f32_to_bf16(v)) fail("f32_to_bf16_bits");
        const uint16_t b = or_f32_to_bf16(v);
        const float back = ci::bf16_bits_to_f32(b), want = or_bf16_to_f32(b);
        if (std::memcmp(&back, &want, 4) != 0) fail("bf16_bits_to_f32");
      }
      pass("bf16 conversions equal the oracle's (ties, specials, NaN)");
    }

    // ---- GEMV, multi-token GEMM, rows subset (crate layout, G32 bf16) ----
    const size_t n = 256, k = 1024, g = 32;
    const std::vector<uint8_t> hp = bytes(7, 1, n * k / 2), hs = scales(7, 2, n * (k / g));
    const std::vector<float> hx = normal(7, 3, 4 * k);
    auto dp = dev(hp);
    auto ds = dev(hs);
    auto dx = dev(hx);
    {
      ci::DeviceBuffer<float> y(n);
      ci::dequant_gemv_int4(dp, ds, ci::DeviceSlice<const float>(dx.data(), k), n, k, y);
      std::vector<float> want(n);
      or_gemv(hp.data(), hs.data(), hx.data(), n, k, g, OR_SCALE_BF16, OR_ORDER_AVX512, want.data());
      check_close(y.download(), want, "dequant_gemv_int4 256x1024");
      ci::DeviceBuffer<float> y2(n);
      ci::dequant_gemv_int4_auto(dp, ds, ci::DeviceSlice<const float>(dx.data(), k), n, k, y2);
      check_close(y2.download(), want, "dequant_gemv_int4_auto");

      ci::DeviceBuffer<float> ys(4 * n);
      ci::dequant_gemm_int4_multi_auto(dp, ds, dx, n, k, 4, ys);
      std::vector<float> wm(4 * n);
      or_gemm_multi(hp.data(), hs.data(), hx.data(), n, k, 4, g, OR_SCALE_BF16, OR_ORDER_AVX512,
                    wm.data());
      check_close(ys.download(), wm, "dequant_gemm_int4_multi_auto seq 4");
      ci::DeviceBuffer<float> yb(4 * n);
      ci::dequant_gemm_int4_multi_blocked_auto(dp, ds, dx, n, k, 4, yb);
      check_close(yb.download(), wm, "dequant_gemm_int4_multi_blocked_auto seq 4");

      // rows subset: the listed rows (shuffled, one repeated) equal the GEMV,
      // every other row keeps its sentinel
      const std::vector<uint32_t> rows = {200, 3, 77, 3, 255, 0, 128};
      auto drows = dev(rows);
      std::vector<float> sentinel(n, -12345.f);
      auto ysub = dev(sentinel);
      ci::dequant_gemv_int4_rows_subset(dp, ds, ci::DeviceSlice<const float>(dx.data(), k), n, k,
                                        ysub, drows);
      std::vector<float> got = ysub.download(), want_sub = sentinel;
      for (uint32_t r : rows) want_sub[r] = want[r];
      for (size_t r = 0; r < n; ++r) {
        bool listed = false;
        for (uint32_t q : rows) listed |= q == r;
        if (!listed && got[r] != -12345.f) fail("rows_subset touched an unlisted row");
      }
      check_close(got, want_sub, "dequant_gemv_int4_rows_subset (unlisted rows untouched)");

      expect_invalid([&] {
        ci::DeviceBuffer<float> yy(n - 1);
        ci::dequant_gemv_int4(dp, ds, ci::DeviceSlice<const float>(dx.data(), k), n, k, yy);
      }, "dequant_gemv_int4 with y one short");
      expect_invalid([&] {
        ci::dequant_gemv_int4(ci::DeviceSlice<const uint8_t>(dp.data(), hp.size() - 1), ds,
                              ci::DeviceSlice<const float>(dx.data(), k), n, k,
                              ci::DeviceSlice<float>(nullptr, n));
      }, "dequant_gemv_int4 with packed one short");
    }

    // ---- ExpertWeights::open and expert_forward (a reference fixture expert) ----
    {
      const size_t h = 64, i = 32;
      ci::ExpertWeights w = ci::ExpertWeights::open(argv[1], h, i, 32);
      std::vector<uint8_t> flat(or_expert_bytes(h, i, 32));
      std::FILE *f = std::fopen(argv[1], "rb");
      if (!f || std::fread(flat.data(), 1, flat.size(), f) != flat.size()) fail("read fixture");
      std::fclose(f);
      std::vector<uint16_t> xb(h);
      const std::vector<float> xf = normal(0, 4, h);
      for (size_t c = 0; c < h; ++c) xb[c] = or_f32_to_bf16(xf[c]);
      auto dxb = dev(xb);
      ci::DeviceBuffer<uint16_t> out(h);
      ci::expert_forward(w, dxb, out);
      std::vector<uint16_t> want(h);
      or_expert_forward(xb.data(), h, i, 32, OR_SCALE_BF16, OR_ORDER_AVX512, flat.data(),
                        want.data());
      const std::vector<uint16_t> got = out.download();
      check_close_bf16(got, want, "ExpertWeights::open + expert_forward (fixture)");
      // the crate-shaped call on the six slices (inter from the gate scales)
      ci::DeviceBuffer<uint16_t> out2(h);
      ci::expert_forward(dxb, w.gate_packed_bytes(), w.gate_scale_bits(), w.up_packed_bytes(),
                         w.up_scale_bits(), w.down_packed_bytes(), w.down_scale_bits(), out2);
      if (out2.download() != got) fail("expert_forward on the six slices differs");
      pass("expert_forward on the six slices equals the ExpertWeights call");
      // the tiled copy: bit-identical
      ci::ExpertWeights t = w.tiled();
      ci::DeviceBuffer<uint16_t> out3(h);
      ci::expert_forward(t, dxb, out3);
      if (out3.download() != got) fail("tiled expert differs");
      pass("ExpertWeights::tiled(): expert_forward bit-identical");

      try {
        (void)ci::ExpertWeights::open(std::string(argv[1]) + ".missing", h, i, 32);
        fail("open of a missing file");
      } catch (const ci::GemmError &e) {
        if (e.kind != ci::GemmError::Kind::Io) fail("missing file: not Io");
        pass("ExpertWeights::open on a missing file -> GemmError::Io");
      }
      try {
        (void)ci::ExpertWeights::open(argv[1], h, i * 2, 32);  // wants twice the bytes
        fail("open of a short file");
      } catch (const ci::GemmError &e) {
        if (e.kind != ci::GemmError::Kind::Truncated || e.actual != flat.size())
          fail("short file: not Truncated");
        pass("ExpertWeights::open on a short file -> GemmError::Truncated");
      }
    }

    // ---- activation-sparse forms (hidden 512, inter 256, G32 bf16) ----
    {
      const size_t h = 512, i = 256;
      const HostExpert he = make_expert(h, i, 32, 21);
      std::vector<ci::DeviceBuffer<uint8_t>> parts;
      for (int q = 0; q < 6; ++q) parts.push_back(dev(he.part(q)));
      auto P = [&](int q) { return ci::DeviceSlice<const uint8_t>(parts[q].data(), parts[q].size()); };
      const std::vector<float> xf = normal(21, 5, h);
      std::vector<uint16_t> xb(h);
      for (size_t c = 0; c < h; ++c) xb[c] = or_f32_to_bf16(xf[c]);
      auto dxb = dev(xb);
      auto dxf = dev(xf);

      for (float tau : {0.0f, 0.3f}) {
        ci::DeviceBuffer<uint16_t> out(h);
        const float frac = ci::expert_forward_sparse(dxb, P(0), P(1), P(2), P(3), P(4), P(5), out,
                                                     tau);
        std::vector<uint16_t> want(h);
        const float wf = or_expert_forward_sparse(xb.data(), h, i, 32, OR_SCALE_BF16,
                                                  OR_ORDER_AVX512, he.flat.data(), tau,
                                                  want.data());
        check_close_bf16(out.download(), want, "expert_forward_sparse tau " + std::to_string(tau));
        if (frac != wf) fail("expert_forward_sparse active fraction");
        pass("expert_forward_sparse active fraction " + std::to_string(frac));
      }

      // per-channel thresholds through the f32 form
      std::vector<float> thr(i);
      for (size_t r = 0; r < i; ++r) thr[r] = (r % 3) * 0.2f;
      auto dthr = dev(thr);
      ci::DeviceBuffer<float> outf(h);
      const float frac = ci::ffn_forward_sparse_f32_per_channel(dxf, h, i, P(0), P(1), P(2), P(3),
                                                                P(4), P(5), outf, dthr);
      std::vector<float> wantf(h);
      const float wf = or_ffn_forward_f32_mode(xf.data(), h, i, 32, OR_SCALE_BF16,
                                               OR_ORDER_AVX512, he.flat.data(), 0.f, thr.data(),
                                               wantf.data());
      check_close(outf.download(), wantf, "ffn_forward_sparse_f32_per_channel");
      if (frac != wf) fail("ffn_forward_sparse_f32_per_channel active fraction");
      pass("ffn_forward_sparse_f32_per_channel active fraction");

      // build_active_mask on a gate row: the list exact
      const std::vector<float> gate = normal(21, 6, i);
      auto dgate = dev(gate);
      ci::ActiveMask m = ci::build_active_mask(dgate, 0.3f);
      std::vector<float> silu(i);
      std::vector<uint32_t> act(i);
      const size_t na = or_build_active_mask(gate.data(), i, 0.3f, silu.data(), act.data());
      act.resize(na);
      if (m.active.download() != act) fail("build_active_mask list");
      check_close(m.silu.download(), silu, "build_active_mask SiLU");
      pass("build_active_mask: " + std::to_string(na) + " lanes, the list exact");

      // the AXPY form: transposed down bit-exact, then the FFN
      auto td = ci::transpose_requantize_down(P(4), P(5), h, i);
      std::vector<uint8_t> pt(i * h / 2), st(i * (h / 32) * 2);
      or_transpose_requantize_down(he.part(4).data(), he.part(5).data(), h, i, pt.data(), st.data());
      if (td.first.download() != pt || td.second.download() != st)
        fail("transpose_requantize_down bytes");
      pass("transpose_requantize_down bytes exact");
      ci::FfnScratch scratch(h, i);
      ci::DeviceBuffer<float> outa(h);
      const float fa = ci::ffn_forward_sparse_axpy_f32(scratch, dxf, h, i, P(0), P(1), P(2), P(3),
                                                       td.first, td.second, outa, 0.3f);
      std::vector<float> wanta(h);
      const float wfa = or_ffn_forward_sparse_axpy_f32_mode(
          xf.data(), h, i, 32, OR_SCALE_BF16, OR_ORDER_AVX512, he.part(0).data(),
          he.part(1).data(), he.part(2).data(), he.part(3).data(), pt.data(), st.data(), 0.3f,
          nullptr, wanta.data());
      check_close(outa.download(), wanta, "ffn_forward_sparse_axpy_f32 tau 0.3");
      if (fa != wfa) fail("ffn_forward_sparse_axpy_f32 active fraction");
      pass("ffn_forward_sparse_axpy_f32 active fraction");

      expect_invalid([&] {
        ci::DeviceBuffer<uint16_t> o(h + 1);
        ci::expert_forward(dxb, P(0), P(1), P(2), P(3), P(4), P(5), o);
      }, "expert_forward with out one long");
    }

    // ---- load-time quantiser (shell_int4.rs:148-212) ----
    {
      const size_t qn = 48, qk = 512;
      std::vector<uint16_t> wb(qn * qk);
      const std::vector<float> w = normal(33, 7, qn * qk);
      for (size_t q = 0; q < wb.size(); ++q) wb[q] = or_f32_to_bf16(w[q] * 0.05f);
      auto dwb = dev(wb);
      auto qz = ci::quantize_int4_group(dwb, qn, qk);
      std::vector<uint8_t> wp(qn * qk / 2), ws(qn * (qk / 32) * 2);
      or_quantize_int4_group(wb.data(), qn, qk, 32, wp.data(), ws.data());
      if (qz.first.download() != wp || qz.second.download() != ws) fail("quantize_int4_group bytes");
      pass("quantize_int4_group codes and scales exact");
    }

    // ---- one sparse-MoE layer (runner.rs:1806-1832): both layouts, a shared
    //      expert, the three routing modes, one token and several ----
    {
      const size_t E = 8, h = 256, i = 128, k = 2, si = 64;
      const size_t per = or_expert_bytes(h, i, 32), stride = (per + 255) / 256 * 256;
      std::vector<uint8_t> flat(E * per), strided(E * stride, 0);
      for (size_t e = 0; e < E; ++e) {
        const HostExpert he = make_expert(h, i, 32, 40 + e);
        std::copy(he.flat.begin(), he.flat.end(), flat.begin() + e * per);
        std::copy(he.flat.begin(), he.flat.end(), strided.begin() + e * stride);
      }
      const HostExpert shared = make_expert(h, si, 32, 60);
      for (ci::Tiling tl : {ci::Tiling::Crate, ci::Tiling::Mfma}) {
        const std::string lay = tl == ci::Tiling::Crate ? "crate" : "tiled";
        ci::Options wo;
        wo.tiling = tl;
        const ci::ExpertStack stack = ci::ExpertStack::upload(flat.data(), E, h, i, wo);
        ci::ExpertWeights sh = ci::ExpertWeights::from_host(shared.flat.data(), shared.flat.size(),
                                                            h, si, 32);
        if (tl == ci::Tiling::Mfma) sh = sh.tiled();
        ci::MoeLayer layer(stack);
        layer.with_shared(sh);
        for (size_t T : {size_t(1), size_t(5)}) {
          const std::string tag = lay + " T" + std::to_string(T);
          const std::vector<float> x = normal(70 + T, 1, T * h), logits = normal(70 + T, 2, T * E);
          const std::vector<float> bias = normal(70 + T, 3, E);
          auto dx = dev(x);
          auto dl = dev(logits);
          auto db = dev(bias);
          ci::DeviceBuffer<float> out(T * h), wts(T * k);
          ci::DeviceBuffer<int32_t> ids(T * k);
          // sigmoid + bias, renormalised x 2.5, residual = x
          ci::moe_forward(layer, ci::Routing::sigmoid_bias(dl, k, 2.5f, true, db), dx, T, out, dx,
                          ids, wts);
          const std::vector<int32_t> gi = ids.download();
          const std::vector<float> gw = wts.download();
          for (size_t t = 0; t < T; ++t) {
            int64_t wi[k];
            float ww[k];
            or_route_sigmoid_bias(logits.data() + t * E, bias.data(), E, k, 2.5f, 1, wi, ww);
            for (size_t s = 0; s < k; ++s) {
              if (gi[t * k + s] != wi[s]) fail("moe routing ids " + tag);
              if (std::fabs((double)gw[t * k + s] - ww[s]) >
                  4 * std::ldexp(1.0, (int)std::floor(std::log2(std::fabs(ww[s]))) - 23))
                fail("moe routing weights " + tag);
            }
          }
          pass("moe_forward routing (sigmoid + bias) ids exact, weights within 4 ulp, " + tag);
          check_moe(out.download(), x, T, h, i, strided, stride, E, &shared, gi, gw, k, 0.f,
                    "moe_forward sigmoid + bias + shared, " + tag);

          // given ids / weights with a skip threshold, no shared expert, no residual
          ci::MoeLayer plain(stack);
          std::vector<int32_t> gid(T * k);
          std::vector<float> gwt(T * k);
          for (size_t q = 0; q < T * k; ++q) {
            gid[q] = (int32_t)((q * 5 + T) % E);
            gwt[q] = 0.1f + 0.2f * (float)(q % 4);
          }
          auto dgi = dev(gid);
          auto dgw = dev(gwt);
          ci::DeviceBuffer<float> out2(T * h);
          ci::moe_forward(plain, ci::Routing::given(dgi, dgw, k).threshold(0.3f), dx, T, out2);
          // no residual: the layer's output is the routed sum alone; the
          // oracle's layer adds x
          std::vector<float> got2 = out2.download();
          for (size_t q = 0; q < T * h; ++q) got2[q] += x[q];
          check_moe(got2, x, T, h, i, strided, stride, E, nullptr, gid, gwt, k, 0.3f,
                    "moe_forward given ids, threshold 0.3, no residual, " + tag);
        }
      }
      // softmax over the top-k logits, crate layout, 3 tokens
      {
        const size_t T = 3;
        const ci::ExpertStack stack = ci::ExpertStack::upload(flat.data(), E, h, i);
        ci::MoeLayer layer(stack);
        const std::vector<float> x = normal(90, 1, T * h), logits = normal(90, 2, T * E);
        auto dx = dev(x);
        auto dl = dev(logits);
        ci::DeviceBuffer<float> out(T * h), wts(T * k);
        ci::DeviceBuffer<int32_t> ids(T * k);
        ci::moe_forward(layer, ci::Routing::softmax_topk(dl, k), dx, T, out, dx, ids, wts);
        const std::vector<int32_t> gi = ids.download();
        const std::vector<float> gw = wts.download();
        for (size_t t = 0; t < T; ++t) {
          int64_t wi[k];
          float ww[k];
          or_route_softmax_topk(logits.data() + t * E, E, k, wi, ww);
          for (size_t s = 0; s < k; ++s)
            if (gi[t * k + s] != wi[s]) fail("softmax routing ids");
        }
        check_moe(out.download(), x, T, h, i, strided, stride, E, nullptr, gi, gw, k, 0.f,
                  "moe_forward softmax top-k, crate T3");
        expect_invalid([&] {
          ci::DeviceBuffer<float> o(T * h - 1);
          ci::moe_forward(layer, ci::Routing::softmax_topk(dl, k), dx, T, o);
        }, "moe_forward with out one short");
        expect_invalid([&] {
          ci::moe_forward(layer, ci::Routing::softmax_topk(ci::DeviceSlice<const float>(dl.data(), T * E - 1), k),
                          dx, T, ci::DeviceSlice<float>(nullptr, T * h));
        }, "moe_forward with logits one short");
      }
    }

    // ---- the handle API over an int4_bin directory (c_ffi.rs:35-341,
    //      manifest.rs:137-142): forward, prefetch, the cache, errors ----
    {
      const size_t h = 64, i = 32;
      char tmpl[] = "/tmp/cascadia_cpp_api_XXXXXX";
      if (!mkdtemp(tmpl)) fail("mkdtemp");
      const std::string dir = tmpl, edir = dir + "/experts", ldir = edir + "/layer_00";
      if (mkdir(edir.c_str(), 0700) || mkdir(ldir.c_str(), 0700)) fail("mkdir");
      write_file(dir + "/manifest.json",
                 "{\"arch\": \"test\", \"experts_format\": \"int4_bin\", \"hidden_size\": 64, "
                 "\"expert_intermediate\": 32, \"num_experts\": 8, \"top_k\": 2}");
      std::vector<uint8_t> fix(or_expert_bytes(h, i, 32));
      std::FILE *f = std::fopen(argv[1], "rb");
      if (!f || std::fread(fix.data(), 1, fix.size(), f) != fix.size()) fail("read fixture");
      std::fclose(f);
      const HostExpert e1 = make_expert(h, i, 32, 80);
      write_file(ldir + "/expert_000.bin", std::string(fix.begin(), fix.end()));
      write_file(ldir + "/expert_001.bin", std::string(e1.flat.begin(), e1.flat.end()));
      {
        ci::Source src = ci::Source::open(dir);
        src.prefetch(0, 1);
        src.prefetch_wait();
        const ci::Source::PrefetchStats ps = src.prefetch_stats();
        if (ps.submits != 1 || ps.processed != 1 || ps.loaded != 1 || ps.drops != 0)
          fail("prefetch stats");
        pass("Source::prefetch loaded expert 1 ahead of use");
        const std::vector<uint8_t> *flats[2] = {&fix, &e1.flat};
        for (uint32_t e = 0; e < 2; ++e) {
          const std::vector<float> x = normal(81, e, h);
          const std::vector<float> got = src.expert_forward(0, e, x);
          std::vector<uint16_t> xb(h), want(h), gotb(h);
          for (size_t c = 0; c < h; ++c) {
            xb[c] = or_f32_to_bf16(x[c]);
            gotb[c] = ci::f32_to_bf16_bits(got[c]);
            if (ci::bf16_bits_to_f32(gotb[c]) != got[c]) fail("Source output not a bf16 value");
          }
          or_expert_forward(xb.data(), h, i, 32, OR_SCALE_BF16, OR_ORDER_AVX512,
                            flats[e]->data(), want.data());
          check_close_bf16(gotb, want, "Source::expert_forward expert " + std::to_string(e));
        }
        ci::Source::CacheStats cs = src.cache_stats();
        if (cs.cached != 2 || cs.evictions != 0) fail("cache stats after two experts");
        src.set_cache_limits(1, 0);
        cs = src.cache_stats();
        if (cs.cached != 1 || cs.evictions != 1) fail("cache limit of one expert");
        pass("Source cache: two resident, a limit of one evicts one");
        try {
          src.prewarm(0, 7);
          fail("prewarm of a missing expert");
        } catch (const ci::GemmError &e) {
          pass("Source::prewarm of a missing expert file -> GemmError::Io");
        }
      }
      try {
        (void)ci::Source::open(dir + "/no_such_dir");
        fail("open of a missing directory");
      } catch (const ci::GemmError &e) {
        pass("Source::open of a missing directory -> GemmError::Io");
      }
      for (const char *name : {"/expert_000.bin", "/expert_001.bin"}) std::remove((ldir + name).c_str());
      std::remove((dir + "/manifest.json").c_str());
      rmdir(ldir.c_str());
      rmdir(edir.c_str());
      rmdir(dir.c_str());
    }
  } catch (const std::exception &e) {
    fail(std::string("exception: ") + e.what());
  }
  std::printf("cpp api: %d checks OK\n", g_checks);
  return 0;
}
