"""Pins the CPU oracle (oracle/int4_oracle.c) before anything is checked
against it.  Each check is one the reference holds (known answers, invariant
suites, fixture bins) or one the mathematics fixes (f64 brute force over an
independent numpy decode, closed forms) -- chosen so that a dropped term, a
wrong sign/index or a transposed operand in the oracle fails one of them.
"""
import glob
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, rel_l2

BF16, F16 = 0, 1


# ----------------------------------------------------------------------------
# independent numpy decode (not the oracle's code path)
# ----------------------------------------------------------------------------

def np_dequant(packed, scales, n, k, group, sdt):
    p = np.frombuffer(np.ascontiguousarray(packed, np.uint8).tobytes(), np.uint8).reshape(n, k // 2)
    nib = np.empty((n, k), np.int32)
    nib[:, 0::2] = p & 0x0F
    nib[:, 1::2] = p >> 4
    s16 = np.frombuffer(np.ascontiguousarray(scales, np.uint8).tobytes(), "<u2").reshape(n, k // group)
    if sdt == F16:
        s = s16.view(np.float16).astype(np.float64)
    else:
        s = (s16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return (nib - 8).astype(np.float64) * np.repeat(s, group, axis=1)


def rand_layout(rng, n, k, group, sdt):
    packed = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    sc = np.abs(rng.normal(0, 0.02, n * (k // group))) + 1e-3
    if sdt == F16:
        bits = sc.astype(np.float16).view(np.uint16)
    else:
        bits = torch.tensor(sc, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return packed, bits.astype("<u2").view(np.uint8).copy()


# reference generator, kernel_avx512_multi.rs:255-291 (and _blocked.rs)
def ref_make_test_data(n_rows, k_cols, seq):
    r = np.arange(n_rows)[:, None]
    c = np.arange(k_cols // 2)[None, :]
    packed = ((r * 31 + c) & 0xFF).astype(np.uint8).ravel()
    ng = k_cols // 32
    g = np.arange(ng)[None, :]
    s = (0.5 + ((r * 7 + g * 3) % 11).astype(np.float32) * np.float32(0.1)).astype(np.float32)
    u = s.view(np.uint32).astype(np.uint64)
    bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype("<u2")
    t = np.arange(seq)[:, None]
    cc = np.arange(k_cols)[None, :]
    xs = (np.sin((t * 17 + cc * 5).astype(np.float32)) * np.float32(0.5)).astype(np.float32)
    return packed, bits.view(np.uint8).ravel().copy(), xs.ravel()


# ----------------------------------------------------------------------------
# a2: conversions
# ----------------------------------------------------------------------------

def test_bf16_rne_matches_half_cases(orc):
    """format.rs:173-201 case list; expected bits from torch's RNE bf16."""
    cases = [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.0, 0.125, 1.0e-30, np.pi, -42.5]
    for x in cases:
        want = int(torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).item()) & 0xFFFF
        assert orc.lib().or_f32_to_bf16(x) == want, x
    nan = orc.lib().or_f32_to_bf16(float("nan"))
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_rne_random_sweep(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    x = x[finite]
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = orc.f32_to_bf16(x)
    assert np.array_equal(got, want)
    # the C scalar agrees with the vectorised helper
    for v in x[:2000]:
        assert orc.lib().or_f32_to_bf16(float(v)) == orc.f32_to_bf16(np.float32(v))[()]


def test_f16_conversions_match_numpy(orc):
    rng = np.random.default_rng(2)
    # every fp16 bit pattern decodes exactly
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = allh.view(np.float16).astype(np.float32)
    L = orc.lib()
    got = np.array([L.or_f16_to_f32(int(h)) for h in allh], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    # f32 -> f16 RNE incl. subnormals, ties and overflow
    xs = np.concatenate([
        rng.normal(0, 1, 20000), rng.normal(0, 1e-5, 20000), rng.normal(0, 3e4, 5000),
        [65504.0, 65520.0, 65519.99, 2.0**-24, 2.0**-25, 1.5 * 2.0**-25, 2.0**-26, 0.0, -0.0],
    ]).astype(np.float32)
    w = xs.astype(np.float16).view(np.uint16)
    g = np.array([L.or_f32_to_f16(float(v)) for v in xs], np.uint16)
    assert np.array_equal(g, w)


# ----------------------------------------------------------------------------
# a3/a4: GEMV known answers (kernel.rs:144-181)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("order", [0, 1])
def test_zero_weight_zero_output(orc, order):
    n, k = 4, 32
    packed = np.full(n * k // 2, 0x88, np.uint8)
    scales = np.tile(np.array([0x80, 0x3F], np.uint8), n * (k // 32))
    x = np.arange(k, dtype=np.float32) * np.float32(0.1)
    y = orc.gemv(packed, scales, x, n, k, 32, BF16, order)
    assert np.all(np.abs(y) < 1e-6)


@pytest.mark.parametrize("order", [0, 1])
def test_unit_weight_picks_first_column(orc, order):
    n, k = 1, 32
    packed = np.full(n * k // 2, 0x88, np.uint8)
    packed[0] = 0x89  # low nibble 9 -> +1 at column 0
    scales = np.array([0x80, 0x3F], np.uint8)
    x = np.arange(k, dtype=np.float32) + 1
    y = orc.gemv(packed, scales, x, n, k, 32, BF16, order)
    assert abs(y[0] - 1.0) < 1e-5
    packed[0] = 0x98  # high nibble -> column 1
    assert abs(orc.gemv(packed, scales, x, n, k, 32, BF16, order)[0] - 2.0) < 1e-5


@pytest.mark.parametrize("order", [0, 1])
def test_one_hot_every_position(orc, order):
    """A +1 code at (row r, col c) with unit scale must return exactly x[c]
    in row r and 0 elsewhere: pins nibble order, row stride and group index."""
    n, k, G = 3, 128, 64
    x = (np.arange(k, dtype=np.float32) * np.float32(0.37) - 3).astype(np.float32)
    rng = np.random.default_rng(3)
    for _ in range(40):
        r, c = int(rng.integers(n)), int(rng.integers(k))
        sc = rng.choice([0.5, 1.0, 2.0, 0.25])
        packed = np.full(n * k // 2, 0x88, np.uint8)
        b = r * (k // 2) + c // 2
        packed[b] = (0x89 if c % 2 == 0 else 0x98)
        scales = np.full(n * (k // G), np.float16(sc).view(np.uint16), np.uint16).view(np.uint8)
        y = orc.gemv(packed, scales, x, n, k, G, F16, order)
        want = np.zeros(n, np.float32)
        want[r] = x[c] * np.float32(sc)
        assert np.array_equal(y, want), (r, c)


@pytest.mark.parametrize("group,sdt", [(32, BF16), (32, F16), (64, F16), (128, F16), (128, BF16)])
def test_dequant_bit_exact_vs_numpy(orc, group, sdt):
    rng = np.random.default_rng(group + sdt)
    n, k = 24, 512
    packed, scales = rand_layout(rng, n, k, group, sdt)
    got = orc.dequant(packed, scales, n, k, group, sdt)
    want = np_dequant(packed, scales, n, k, group, sdt).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("group,sdt", [(32, BF16), (64, F16), (128, F16)])
def test_gemv_vs_f64_brute_force(orc, order, group, sdt):
    rng = np.random.default_rng(7 * group + sdt + order)
    n, k = 64, 1024
    packed, scales = rand_layout(rng, n, k, group, sdt)
    x = rng.normal(0, 1, k).astype(np.float32)
    y = orc.gemv(packed, scales, x, n, k, group, sdt, order)
    want = np_dequant(packed, scales, n, k, group, sdt) @ x.astype(np.float64)
    assert rel_l2(y, want) < 2e-6
    # a transposed read or a dropped group would be O(1) wrong
    assert np.max(np.abs(y - want)) < 1e-4 * np.max(np.abs(want))


def test_scalar_and_avx512_orders_differ_only_by_rounding(orc):
    packed, scales, xs = ref_make_test_data(96, 1536, 1)
    a = orc.gemv(packed, scales, xs, 96, 1536, 32, BF16, 0)
    b = orc.gemv(packed, scales, xs, 96, 1536, 32, BF16, 1)
    assert rel_l2(a, b) < 1e-6


# ----------------------------------------------------------------------------
# a5/a6: multi / blocked tiles bit-identical per token
# (kernel_avx512_multi.rs:293-396, kernel_avx512_multi_blocked.rs:392-595)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,seq", [(64, 128, 1), (64, 128, 4), (96, 1536, 8), (65, 256, 5),
                                     (63, 8192, 16), (128, 256, 2), (32, 256, 64), (16, 256, 65)])
def test_cpu_tiles_bit_identical_to_per_token(orc, n, k, seq):
    """The timed AVX-512 tiles (cpu_baseline.c) == per-token restatement,
    bitwise, on the crate's own generator; odd rows hit the RB=2 tail."""
    if orc.cpu_isa() != 2:
        pytest.skip("host has no AVX-512; the tiles then use another order")
    packed, scales, xs = ref_make_test_data(n, k, seq)
    want = orc.gemm_multi(packed, scales, xs, n, k, seq, 32, BF16, 1)
    got = orc.cpu_gemm(packed, scales, xs, n, k, seq, 32, BF16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("group,sdt", [(128, F16), (32, F16)])
def test_cpu_tiles_generalised_group(orc, group, sdt):
    if orc.cpu_isa() != 2:
        pytest.skip("host has no AVX-512")
    rng = np.random.default_rng(11)
    n, k = 48, 1024
    packed, scales = rand_layout(rng, n, k, group, sdt)
    for seq in (1, 3, 8, 20):
        xs = rng.normal(0, 1, seq * k).astype(np.float32)
        want = orc.gemm_multi(packed, scales, xs, n, k, seq, group, sdt, 1)
        got = orc.cpu_gemm(packed, scales, xs, n, k, seq, group, sdt)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), seq


# ----------------------------------------------------------------------------
# a7/a8: expert FFN, sparse variants (ffn_sparsity.rs:981-1194)
# ----------------------------------------------------------------------------

def fake_expert(hidden, inter, gate_b=0x9A, up_b=0x8B, down_b=0x7C):
    """ffn_sparsity.rs:985-1002: constant bytes, unit bf16 scales, G=32."""
    one = np.array([0x80, 0x3F], np.uint8)
    parts = [np.full(inter * hidden // 2, gate_b, np.uint8), np.tile(one, inter * (hidden // 32)),
             np.full(inter * hidden // 2, up_b, np.uint8), np.tile(one, inter * (hidden // 32)),
             np.full(hidden * inter // 2, down_b, np.uint8), np.tile(one, hidden * (inter // 32))]
    return np.concatenate(parts)


def test_sparse_tau_zero_matches_dense(orc):
    h = i = 32
    flat = fake_expert(h, i)
    x = orc.f32_to_bf16(np.arange(h, dtype=np.float32) * np.float32(0.05) - np.float32(0.5))
    dense = orc.expert_forward(x, flat, h, i, 32, BF16)
    sparse, frac = orc.expert_forward_sparse(x, flat, h, i, 32, BF16, 0.0)
    assert frac == 1.0 and np.array_equal(dense, sparse)


@pytest.mark.parametrize("tau", [0.1, 0.3])
def test_sparse_tau_matches_masked_dense(orc, tau):
    """ffn_sparsity.rs:499-537, 756-867: at tau > 0 the output is the dense FFN
    with the intermediate lanes whose |silu(gate)| is under tau * max zeroed
    (numpy f64 over the pinned GEMVs), and the active fraction counts those
    kept.  Random codes and scales, so the mask splits the lanes."""
    h, i, g = 64, 96, 32
    offs, sizes = orc.expert_offsets(h, i, g)
    flat = orc.fill_bytes(5, 1, offs[5] + sizes[5])
    for j in (1, 3, 5):  # the three scale sections
        flat[offs[j]:offs[j] + sizes[j]] = orc.fill_scales(5, 10 + j, sizes[j] // 2, BF16).view(np.uint8)
    x = orc.f32_to_bf16(orc.fill_normal_f32(5, 20, h))
    xf = orc.bf16_to_f32(x)
    gate = orc.gemv(flat[offs[0]:offs[1]], flat[offs[1]:offs[2]], xf, i, h, g, BF16)
    up = orc.gemv(flat[offs[2]:offs[3]], flat[offs[3]:offs[4]], xf, i, h, g, BF16)
    silu = gate.astype(np.float64) / (1.0 + np.exp(-gate.astype(np.float64)))
    keep = np.abs(silu) >= tau * np.max(np.abs(silu))
    assert 0 < keep.sum() < i  # the mask splits the lanes
    m = np.where(keep, silu * up, 0.0)
    dq = orc.dequant(flat[offs[4]:offs[5]], flat[offs[5]:], h, i, g, BF16).astype(np.float64)
    want = dq @ m
    got, frac = orc.expert_forward_sparse(x, flat, h, i, g, BF16, tau)
    assert frac == pytest.approx(keep.sum() / i)
    got = orc.bf16_to_f32(got).astype(np.float64)
    # bf16 output: within a few bf16 ulps of the f64 reference
    assert np.max(np.abs(got - want)) <= 2.0 ** -6 * np.max(np.abs(want))
    # and the lanes masked out matter: the dense output differs
    dense = orc.bf16_to_f32(orc.expert_forward(x, flat, h, i, g, BF16)).astype(np.float64)
    assert np.max(np.abs(dense - want)) > 2.0 ** -6 * np.max(np.abs(want))


def test_ffn_f32_tau_zero_matches_inline_dense(orc):
    """ffn_sparsity.rs:1110-1194: tau 0 == gemv, gemv, swiglu_mul, gemv (bitwise)."""
    h = i = 32
    flat = fake_expert(h, i)
    o, _ = orc.expert_offsets(h, i, 32)
    x = (np.arange(h, dtype=np.float32) * np.float32(0.05) - np.float32(0.5)).astype(np.float32)
    g = orc.gemv(flat[o[0]:o[1]], flat[o[1]:o[2]], x, i, h, 32, BF16)
    u = orc.gemv(flat[o[2]:o[3]], flat[o[3]:o[4]], x, i, h, 32, BF16)
    m = (g / (np.float32(1) + np.exp(-g))).astype(np.float32) * u
    ref = orc.gemv(flat[o[4]:o[5]], flat[o[5]:], m.astype(np.float32), h, i, 32, BF16)
    got, frac = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.0)
    assert frac == 1.0
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_mask_threshold_cases(orc):
    _, act = orc.build_active_mask(np.array([1.0, -2.0, 0.5, -0.1], np.float32), 0.0)
    assert act.tolist() == [0, 1, 2, 3]
    g = np.array([10.0, 0.001, 5.0, -0.001], np.float32)
    silu, act = orc.build_active_mask(g, 0.5)
    assert silu[0] > 5.0 and act.tolist() == [0]
    _, act2 = orc.build_active_mask(g, 0.1)
    assert act2.tolist() == [0, 2]


def test_rows_subset(orc):
    n, k = 4, 32
    packed = (np.arange(n * k // 2) % 256).astype(np.uint8)
    scales = np.tile(np.array([0x80, 0x3F], np.uint8), n)
    x = np.arange(k, dtype=np.float32) * np.float32(0.01)
    dense = orc.gemv(packed, scales, x, n, k, 32, BF16)
    y = np.zeros(n, np.float32)
    orc.gemv_rows_subset(packed, scales, x, n, k, 32, BF16, np.arange(n), y)
    assert np.array_equal(dense, y)
    y = np.full(n, 123.0, np.float32)
    orc.gemv_rows_subset(np.full(n * k // 2, 0xAA, np.uint8), scales, np.ones(k, np.float32),
                         n, k, 32, BF16, [1], y)
    assert y[0] == 123.0 and y[2] == 123.0 and y[3] == 123.0 and abs(y[1] - 123.0) > 1e-3


def ref_pack(w, out, inn, G=32):
    """ov_moe.rs:837-862 test packer (test-data preparation)."""
    ng = inn // G
    wg = w.reshape(out, ng, G)
    mx = np.abs(wg).max(axis=2)
    s = np.where(mx > 0, mx / np.float32(7), np.float32(1)).astype(np.float32)
    q = np.clip(np.round(wg / s[:, :, None]), -8, 7).astype(np.int32)
    nib = (q + 8).astype(np.uint8).reshape(out, inn)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    u = s.view(np.uint32).astype(np.uint64)
    bf = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype("<u2")
    return packed.ravel(), bf.view(np.uint8).ravel()


def test_int4_expert_vs_fp32_swiglu(orc):
    """ov_moe.rs:888-920: int4 expert within rel-L2 0.1 of the fp32 SwiGLU."""
    h, m = 64, 32

    def mk(n, seed):
        i = np.arange(n, dtype=np.uint64)
        v = ((i * 2654435761 + seed) & 0xFFFFFFFF) % 1000
        return ((v.astype(np.float32) / np.float32(1000) - np.float32(0.5)) * np.float32(0.2)).astype(np.float32)

    gate, up, down, x = mk(m * h, 1), mk(m * h, 2), mk(h * m, 3), mk(h, 4)
    flat = np.concatenate([*ref_pack(gate, m, h), *ref_pack(up, m, h), *ref_pack(down, h, m)])
    xb = orc.f32_to_bf16(x)
    got = orc.bf16_to_f32(orc.expert_forward(xb, flat, h, m, 32, BF16))
    G, U, D = gate.reshape(m, h), up.reshape(m, h), down.reshape(h, m)
    g = G @ x
    u = U @ x
    want = D @ ((g / (1 + np.exp(-g))) * u)
    assert rel_l2(got, want) < 0.1


# ----------------------------------------------------------------------------
# reference fixture bins (real exporter output in the crate layout)
# ----------------------------------------------------------------------------

FIXTURES = [("dsv4_layer_00", 64, 32), ("dsv4_layer_01", 64, 32), ("glm5_layer_01", 32, 32)]


def fixture_files():
    for d, h, i in FIXTURES:
        for f in sorted(glob.glob(os.path.join(GOLDEN, "fixture_experts", d, "*.bin"))):
            yield f, h, i


def test_fixture_bins_layout_invariants(orc):
    """Every (row, group) of every section holds a |q| = 7 code and no -8
    code, or is an all-zero group with scale 1.0 -- the exporter's quantiser
    (tools/export_deepseek_v4.py:85-94).  A wrong row stride, group width,
    zero point or section order breaks it."""
    n_files = 0
    for f, h, i in fixture_files():
        flat = np.fromfile(f, np.uint8)
        assert flat.size == orc.expert_bytes(h, i, 32)
        o, sz = orc.expert_offsets(h, i, 32)
        for (rows, cols), (po, so) in zip([(i, h), (i, h), (h, i)], [(0, 1), (2, 3), (4, 5)]):
            p = flat[o[po]:o[po] + sz[po]].reshape(rows, cols // 2)
            nib = np.empty((rows, cols), np.int32)
            nib[:, 0::2] = p & 15
            nib[:, 1::2] = p >> 4
            q = (nib - 8).reshape(rows, cols // 32, 32)
            s = np.frombuffer(flat[o[so]:o[so] + sz[so]].tobytes(), "<u2").reshape(rows, cols // 32)
            zero = np.all(q == 0, axis=2)
            assert np.all(s[zero] == 0x3F80)
            assert np.all(np.abs(q).max(axis=2)[~zero] == 7)
            assert not np.any(q == -8)
            sf = (s.astype(np.uint32) << 16).view(np.float32)
            assert np.all(sf > 0) and np.all(np.isfinite(sf))
        n_files += 1
    assert n_files == 23


def test_fixture_expert_forward_vs_f64(orc):
    """expert_forward on every fixture expert vs an f64 numpy SwiGLU over an
    independent decode, both rounded at the crate's points."""
    rng = np.random.default_rng(5)
    for f, h, i in fixture_files():
        flat = np.fromfile(f, np.uint8)
        o, sz = orc.expert_offsets(h, i, 32)
        Wg = np_dequant(flat[o[0]:o[1]], flat[o[1]:o[2]], i, h, 32, BF16)
        Wu = np_dequant(flat[o[2]:o[3]], flat[o[3]:o[4]], i, h, 32, BF16)
        Wd = np_dequant(flat[o[4]:o[5]], flat[o[5]:], h, i, 32, BF16)
        xb = orc.f32_to_bf16(rng.normal(0, 1, h).astype(np.float32))
        x = orc.bf16_to_f32(xb).astype(np.float64)
        g, u = Wg @ x, Wu @ x
        want = Wd @ ((g / (1 + np.exp(-g))) * u)
        got = orc.bf16_to_f32(orc.expert_forward(xb, flat, h, i, 32, BF16))
        assert rel_l2(got, want) < 4e-3, f  # bf16 output rounding dominates
        sh, _ = orc.ffn_forward_f32(x.astype(np.float32), flat, h, i, 32, BF16, 0.0)
        assert rel_l2(sh, want) < 1e-5, f


# ----------------------------------------------------------------------------
# a9: routing
# ----------------------------------------------------------------------------

def test_glm_gate_tie_breaks_to_lower_id(orc):
    """glm/gate.rs:67-80."""
    ids, w = orc.route_sigmoid_bias([0, 0, 0, 0], [0.1, 0.1, 0, 0], 2, 2.5, True)
    assert ids.tolist() == [0, 1]
    assert abs(w[0] - 1.25) < 1e-6 and abs(w[1] - 1.25) < 1e-6


def test_glm_gate_no_norm_at_top1(orc):
    """glm/gate.rs:82-89."""
    ids, w = orc.route_sigmoid_bias([10.0, -10.0], [0, 0], 1, 2.0, True)
    assert ids.tolist() == [0]
    assert abs(w[0] - 2.0 * (1 / (1 + np.exp(-10.0)))) < 1e-6


def test_k26_router_vs_numpy(orc):
    """shell_int4.rs:588-620: stable descending sort of sigmoid+bias."""
    rng = np.random.default_rng(9)
    for _ in range(50):
        l = rng.normal(0, 1, 384).astype(np.float32)
        l[rng.integers(384, size=20)] = l[0]  # plant ties
        b = (rng.normal(0, 0.01, 384) * rng.integers(0, 2)).astype(np.float32)
        ids, w = orc.route_sigmoid_bias(l, b, 8, 2.827, True)
        sc = (1 / (1 + np.exp(-l.astype(np.float64))))
        ch = sc.astype(np.float32) + b
        order = np.argsort(-ch, kind="stable")[:8]
        assert ids.tolist() == order.tolist()
        ww = sc[order] / (sc[order].sum() + 1e-20) * 2.827
        assert np.allclose(w, ww, rtol=1e-5)


def test_softmax_topk_vs_numpy(orc):
    rng = np.random.default_rng(10)
    for _ in range(50):
        l = rng.normal(0, 1, 256).astype(np.float32)
        l[5] = l[200] = l.max() + 1  # tie at the top -> lower id first
        ids, w = orc.route_softmax_topk(l, 8)
        order = np.argsort(-l, kind="stable")[:8]
        assert ids.tolist() == order.tolist() and ids[0] == 5 and ids[1] == 200
        e = np.exp(l[order].astype(np.float64) - l[order].max())
        assert np.allclose(w, e / e.sum(), rtol=1e-6)
        assert abs(float(w.sum()) - 1.0) < 1e-6


# ----------------------------------------------------------------------------
# a10: per-token dispatch + combine (runner.rs:1806-1832)
# ----------------------------------------------------------------------------

def test_moe_combine_slot_order_and_threshold(orc):
    h, i, E, k, T = 64, 32, 8, 2, 3
    files = sorted(glob.glob(os.path.join(GOLDEN, "fixture_experts", "dsv4_layer_00", "expert_0*.bin")))
    experts = np.concatenate([np.fromfile(f, np.uint8) for f in files])
    shared = np.fromfile(os.path.join(GOLDEN, "fixture_experts", "dsv4_layer_00", "expert_shared.bin"), np.uint8)
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (T, h)).astype(np.float32)
    ids = np.array([[3, 1], [0, 7], [5, 5]], np.int64)
    w = np.array([[0.7, 0.3], [0.05, 0.95], [0.5, 0.25]], np.float32)
    got = orc.moe_routed(x, experts, E, h, i, 32, BF16, ids, w, threshold=0.1)
    stride = experts.size // E
    for t in range(T):
        acc = np.zeros(h, np.float32)
        xb = orc.f32_to_bf16(x[t])
        for s in range(k):
            if w[t, s] < 0.1:
                continue
            y = orc.bf16_to_f32(orc.expert_forward(xb, experts[ids[t, s] * stride:(ids[t, s] + 1) * stride], h, i, 32, BF16))
            acc = (acc + w[t, s] * y).astype(np.float32)
        assert np.array_equal(got[t], acc)
    layer = orc.moe_layer(x, experts, E, shared, i, h, i, 32, BF16, ids, w, threshold=0.1)
    for t in range(T):
        sh, _ = orc.ffn_forward_f32(x[t], shared, h, i, 32, BF16, 0.0)
        assert np.array_equal(layer[t], ((x[t] + sh).astype(np.float32) + got[t]).astype(np.float32))


@pytest.mark.parametrize("group,sdt,thr", [(32, BF16, 0.1), (128, F16, 0.0)])
def test_cpu_moe_layer_bit_identical_to_oracle(orc, group, sdt, thr):
    """The timed per-(token, slot) MoE loop on the AVX-512 kernels (the MoE
    CPU baseline, and the checker of full-size GPU MoE layers) equals the
    restatement's layer at the AVX-512 order, bitwise, shared expert included."""
    if orc.cpu_isa() != 2:
        pytest.skip("host has no AVX-512; the port then uses another order")
    h, i, E, k, T, si = 256, 128, 6, 3, 4, 64
    per = orc.expert_bytes(h, i, group)
    offs, sizes = orc.expert_offsets(h, i, group)
    experts = np.concatenate([orc.fill_bytes(3, 10 + e, per) for e in range(E)])
    for e in range(E):
        for s_ in (1, 3, 5):
            o = e * per + offs[s_]
            experts[o:o + sizes[s_]] = orc.fill_scales(3, 20 + 10 * e + s_, sizes[s_] // 2, sdt).view(np.uint8)
    shared = orc.fill_bytes(3, 90, orc.expert_bytes(h, si, group))
    so, ss = orc.expert_offsets(h, si, group)
    for s_ in (1, 3, 5):
        shared[so[s_]:so[s_] + ss[s_]] = orc.fill_scales(3, 91 + s_, ss[s_] // 2, sdt).view(np.uint8)
    x = orc.fill_normal_f32(3, 7, T * h).reshape(T, h)
    rng = np.random.default_rng(4)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int64)
    w = rng.random((T, k)).astype(np.float32)
    want = orc.moe_layer(x, experts, E, shared, si, h, i, group, sdt, ids, w, thr)
    got = orc.cpu_moe_layer(x, experts, E, shared, si, h, i, group, sdt, ids, w, thr)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    want0 = orc.moe_layer(x, experts, E, None, 0, h, i, group, sdt, ids, w, thr)
    got0 = orc.cpu_moe_layer(x, experts, E, None, 0, h, i, group, sdt, ids, w, thr)
    assert np.array_equal(got0.view(np.uint32), want0.view(np.uint32))


# ----------------------------------------------------------------------------
# a11: load-time quantiser (shell_int4.rs:148-212)
# ----------------------------------------------------------------------------

def test_quantize_roundtrip(orc):
    rng = np.random.default_rng(13)
    n, k = 16, 256
    w = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    w[3, :32] = 0.0  # all-zero group -> scale 1e-10, codes 8
    wb = orc.f32_to_bf16(w)
    packed, scales = orc.quantize_int4_group(wb, n, k, 32)
    deq = np_dequant(packed, scales, n, k, 32, BF16)
    wf = orc.bf16_to_f32(wb).reshape(n, k).astype(np.float64)
    s = np.repeat((np.frombuffer(scales.tobytes(), "<u2").astype(np.uint32) << 16).view(np.float32).reshape(n, k // 32), 32, axis=1)
    assert np.all(np.abs(deq - wf) <= 0.5 * s + 1e-12)
    assert np.all(packed[3 * (k // 2):3 * (k // 2) + 16] == 0x88)


def test_quantize_known_answers(orc):
    """Closed-form codes: a group whose max is 0.875 has scale 0.875 / 7 =
    0.125 exactly (bf16 0x3E00) and 1 / scale = 8, so w = (2m + 1) / 16 lands
    on m + 0.5 and rounds away from zero (Rust f32::round) to m + 1 (m < 7: every
    |w| below the max)."""
    g = 32
    j = np.arange(g)
    w = ((j % 7) * 2 + 1) * 0.0625 * np.where(j % 2, -1.0, 1.0)
    w[0] = 0.875
    packed, scales = orc.quantize_int4_group(orc.f32_to_bf16(w.astype(np.float32)), 1, g, g)
    assert scales.view("<u2")[0] == 0x3E00
    q = np.stack([packed & 15, packed >> 4], 1).reshape(-1).astype(np.int32) - 8
    want = (j % 7 + 1) * np.where(j % 2, -1, 1)
    want[0] = 7
    assert np.array_equal(q, want)


# ----------------------------------------------------------------------------
# generators
# ----------------------------------------------------------------------------

def test_generators_deterministic_and_distributed(orc):
    a = orc.fill_bytes(0, 1, 1 << 16)
    assert np.array_equal(a, orc.fill_bytes(0, 1, 1 << 16))
    assert not np.array_equal(a, orc.fill_bytes(0, 2, 1 << 16))
    nib = np.concatenate([a & 15, a >> 4])
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * nib.size / 16 and counts.max() < 1.1 * nib.size / 16
    z = orc.fill_normal_f32(0, 3, 100000)
    assert abs(z.mean()) < 0.02 and abs(z.std() - 1) < 0.02
    s = orc.fill_scales(0, 4, 100000, F16).view(np.float16).astype(np.float64)
    assert s.min() >= 1e-3 * 0.999 and abs((s - 1e-3).mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4


def test_mask_per_channel_known_answers(orc):
    """PerChannel (ffn_sparsity.rs:162-175): cutoff_i = t_i * max|silu|.
    silu(10) = 9.9995, silu(5) = 4.9665, silu(+-0.001) = +-0.0005."""
    g = np.array([10.0, 0.001, 5.0, -0.001], np.float32)
    _, act = orc.build_active_mask(g, 0.0, thresholds=np.array([0.9, 0.0, 0.6, 2.0], np.float32))
    assert act.tolist() == [0, 1]
    _, act = orc.build_active_mask(g, 0.0, thresholds=np.array([0.9, 0.0, 0.4, 2.0], np.float32))
    assert act.tolist() == [0, 1, 2]
    # every threshold <= 0 is dense (:88): all lanes, whatever the values
    _, act = orc.build_active_mask(g, 0.0, thresholds=np.array([0, -1, 0, -3], np.float32))
    assert act.tolist() == [0, 1, 2, 3]
    # stable SiLU against float64
    s, _ = orc.build_active_mask(np.array([-30, -3, -0.5, 0, 0.5, 3, 30], np.float32), 0.5)
    x = np.array([-30, -3, -0.5, 0, 0.5, 3, 30], np.float64)
    assert np.allclose(s, x / (1 + np.exp(-x)), rtol=1e-6, atol=1e-30)


def _random_expert(orc, h, i, seed):
    flat = orc.fill_bytes(seed, 60, orc.expert_bytes(h, i, 32))
    offs, sizes = orc.expert_offsets(h, i, 32)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 61 + s_, sizes[s_] // 2, BF16).view(np.uint8)
    return flat


def test_sparse_per_channel_uniform_is_global(orc):
    """A per-channel vector equal to tau everywhere is the global mode, bitwise;
    one with every entry <= 0 is the dense FFN, bitwise."""
    h, i = 256, 128
    flat = _random_expert(orc, h, i, 5)
    x = orc.fill_normal_f32(5, 9, h)
    xb = orc.f32_to_bf16(x)
    for tau in (0.05, 0.3, 1.0):
        a, fa = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, tau)
        b, fb = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.0, thresholds=np.full(i, tau, np.float32))
        assert fa == fb < 1.0 and np.array_equal(a.view(np.uint32), b.view(np.uint32))
        c, fc = orc.expert_forward_sparse(xb, flat, h, i, 32, BF16, tau)
        d, fd = orc.expert_forward_sparse(xb, flat, h, i, 32, BF16, 0.0, thresholds=np.full(i, tau, np.float32))
        assert fc == fd and np.array_equal(c, d)
    dense, _ = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.0)
    pc, f = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.0, thresholds=-np.arange(i, dtype=np.float32))
    assert f == 1.0 and np.array_equal(dense.view(np.uint32), pc.view(np.uint32))


def test_sparse_branch_composition(orc):
    """ffn_sparsity.rs:499-537: the sparse branch is gate in full, the mask,
    up on the active rows, inter = silu * up there and 0 elsewhere, down in
    full -- restated from the oracle's GEMV and mask (pinned above)."""
    h, i = 256, 128
    flat = _random_expert(orc, h, i, 8)
    o, _ = orc.expert_offsets(h, i, 32)
    x = orc.fill_normal_f32(8, 9, h)
    for tau in (0.1, 0.5):
        g = orc.gemv(flat[o[0]:o[1]], flat[o[1]:o[2]], x, i, h, 32, BF16)
        silu, act = orc.build_active_mask(g, tau)
        u = orc.gemv(flat[o[2]:o[3]], flat[o[3]:o[4]], x, i, h, 32, BF16)
        m = np.zeros(i, np.float32)
        m[act] = silu[act] * u[act]
        want = orc.gemv(flat[o[4]:o[5]], flat[o[5]:], m, h, i, 32, BF16)
        got, frac = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, tau)
        assert frac == len(act) / i and 0 < len(act) < i
        assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def _crate_down(orc, h, i, codes, scale_bits):
    """Crate bytes of a down matrix [h, i]: codes int [-8, 7], one scale per
    row-group of 32 (uint16 bits, shape [h, i / 32])."""
    nib = (codes + 8).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    return packed, np.ascontiguousarray(scale_bits, np.uint16).view(np.uint8).reshape(-1)


def test_transpose_requantize_closed_forms(orc):
    """ffn_axpy.rs:342-440.  Codes in [-7, 7] with every destination group
    holding a +-7, all source scales s (a power of two): each destination
    group's max is 7 s, so its scale is s exactly and the codes are the
    transposed source codes; an all-zero group gets scale 1.0 and code 0."""
    h, i = 96, 64
    rng = np.random.default_rng(4)
    codes = rng.integers(-7, 8, (h, i))
    codes[0::32, :] = 7 * np.where(rng.integers(0, 2, i), 1, -1)  # a +-7 in every (r, g)
    codes[64:96, 5] = 0  # destination row 5, group 2: all zero
    for s_bits, s_val in ((0x3F80, 1.0), (0x4000, 2.0), (0x3E00, 0.125)):
        packed, scales = _crate_down(orc, h, i, codes, np.full((h, i // 32), s_bits))
        pt, st = orc.transpose_requantize_down(packed, scales, h, i)
        st = st.view(np.uint16).reshape(i, h // 32)
        got = np.stack([pt & 15, pt >> 4], -1).reshape(i, h).astype(np.int64) - 8
        want = codes.T.copy()
        assert np.array_equal(got, want), s_val
        exp_s = np.full((i, h // 32), s_bits, np.uint16)
        exp_s[5, 2] = 0x3F80
        assert np.array_equal(st, exp_s), s_val


def test_axpy_is_transposed_gemv(orc):
    """ffn_axpy.rs:82-160: with W_t the exact transpose of W (the closed form
    above), y = sum_{r active} s_r W_t[r, :] is W . m with m = s on the
    active rows and 0 elsewhere -- the oracle GEMV, pinned independently."""
    h, i = 96, 64
    rng = np.random.default_rng(5)
    codes = rng.integers(-7, 8, (h, i))
    codes[0::32, :] = 7
    packed, scales = _crate_down(orc, h, i, codes, np.full((h, i // 32), 0x3F00))  # 0.5
    pt, st = orc.transpose_requantize_down(packed, scales, h, i)
    s = rng.normal(0, 1, i).astype(np.float32)
    active = np.sort(rng.choice(i, 20, replace=False)).astype(np.uint32)
    y = orc.dequant_axpy_active(pt, st, s, active, i, h)
    m = np.zeros(i, np.float32)
    m[active] = s[active]
    want = orc.gemv(packed, scales, m, h, i, 32, BF16)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5)
    # accumulates onto y
    y2 = orc.dequant_axpy_active(pt, st, s, active, i, h, y=np.ones(h, np.float32))
    assert np.allclose(y2, y + 1, rtol=1e-6, atol=1e-6)


# ----------------------------------------------------------------------------
# f3: the AXPY-form sparse FFN (ffn_sparsity.rs:569-740)
# ----------------------------------------------------------------------------

def _axpy_fixture():
    """ffn_sparsity.rs:1196-1217: constant gate/up/down bytes, unit bf16
    scales, x = 0.05 i - 0.5, hidden = intermediate = 64."""
    h = i = 64
    flat = fake_expert(h, i)
    offs, _ = _offsets(h, i, 32)
    down = flat[offs[4]:offs[5]]
    down_s = flat[offs[5]:]
    x = (np.arange(h, dtype=np.float32) * np.float32(0.05) - np.float32(0.5)).astype(np.float32)
    return h, i, flat, down, down_s, x


def _offsets(h, i, g):
    gp, gs, dp = i * h // 2, i * (h // g) * 2, h * i // 2
    return [0, gp, gp + gs, 2 * gp + gs, 2 * (gp + gs), 2 * (gp + gs) + dp], None


def test_axpy_ffn_close_to_dense_at_zero(orc):
    """ffn_sparsity.rs:1196-1267: at tau 0 the AXPY form (re-quantised
    transposed down) stays within 20 % of the dense FFN's max."""
    h, i, flat, down, down_s, x = _axpy_fixture()
    dense, _ = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.0)
    pt, st = orc.transpose_requantize_down(down, down_s, h, i)
    axpy, frac = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, 32, BF16, 0.0)
    assert frac == 1.0
    assert np.max(np.abs(dense - axpy)) <= max(float(np.max(np.abs(dense))), 1.0) * 0.20


def test_axpy_ffn_matches_sparse_at_small_tau(orc):
    """ffn_sparsity.rs:1273-1345: at tau 0.1 the two sparse formulations agree
    within 2x the dense max, with a fraction in (0, 1]."""
    h, i, flat, down, down_s, x = _axpy_fixture()
    sparse, _ = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, 0.10)
    pt, st = orc.transpose_requantize_down(down, down_s, h, i)
    axpy, frac = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, 32, BF16, 0.10)
    assert 0.0 < frac <= 1.0
    assert np.max(np.abs(sparse - axpy)) <= max(float(np.max(np.abs(sparse))), 1.0) * 2.0


def test_axpy_per_channel_uniform_matches_global(orc):
    """ffn_sparsity.rs:1497-1560: a per-channel vector of one value tau0 is
    bit-identical to the global tau0 (output and fraction)."""
    h, i, flat, down, down_s, x = _axpy_fixture()
    pt, st = orc.transpose_requantize_down(down, down_s, h, i)
    for tau in (0.0, 0.05, 0.10, 0.30):
        a, fa = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, 32, BF16, tau)
        b, fb = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, 32, BF16, 0.0,
                                                thresholds=np.full(i, tau, np.float32))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)) and fa == fb, tau


@pytest.mark.parametrize("tau", [0.0, 0.2, 0.5])
def test_axpy_ffn_closed_form_exact_transpose(orc, tau):
    """With a down matrix the transpose-requantisation keeps exactly (codes in
    [-7, 7], a +-7 in every group, power-of-two scales), the AXPY FFN is the
    f32 FFN whose intermediate is silu * up on the lanes |silu| >= tau * max
    and 0 elsewhere -- computed here with numpy from the pinned GEMVs; the
    active fraction is that lane count."""
    h, i, g = 96, 64, 32
    rng = np.random.default_rng(9)
    gate_p, gate_s = rand_layout(rng, i, h, g, BF16)
    up_p, up_s = rand_layout(rng, i, h, g, BF16)
    codes = rng.integers(-7, 8, (h, i))
    codes[0::32, :] = 7
    down_p, down_s = _crate_down(orc, h, i, codes, np.full((h, i // 32), 0x3E80))  # 0.25
    flat = np.concatenate([gate_p, gate_s, up_p, up_s, down_p, down_s])
    pt, st = orc.transpose_requantize_down(down_p, down_s, h, i)
    x = rng.normal(0, 1, h).astype(np.float32)
    got, frac = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, g, BF16, tau)
    gate = orc.gemv(gate_p, gate_s, x, i, h, g, BF16).astype(np.float64)
    up = orc.gemv(up_p, up_s, x, i, h, g, BF16).astype(np.float64)
    silu = gate / (1.0 + np.exp(-gate))
    mask = np.abs(silu) >= tau * np.max(np.abs(silu)) if tau > 0 else np.ones(i, bool)
    m = np.where(mask, silu * up, 0.0)
    w_down = codes.astype(np.float64) * 0.25
    want = w_down @ m
    assert frac == mask.sum() / i
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4 * np.max(np.abs(want)))


def test_nan_tau_is_sparse_everywhere(orc):
    """SparsityMode::is_dense is `t <= 0.0` (ffn_sparsity.rs:85-90), so a NaN
    tau is NOT dense: its cutoff NaN * max passes no lane (while max|silu| > 0).
    Every oracle form must agree -- the mask, the GEMV-form sparse FFN and the
    AXPY form -- with zero active lanes and an all-zero output."""
    h, i, flat, down, down_s, x = _axpy_fixture()
    nan = np.float32("nan")
    _, act = orc.build_active_mask(np.array([1.0, -2.0, 0.5, -0.1], np.float32), nan)
    assert act.size == 0
    out, frac = orc.ffn_forward_f32(x, flat, h, i, 32, BF16, nan)
    assert frac == 0.0 and np.all(out == 0.0)
    pt, st = orc.transpose_requantize_down(down, down_s, h, i)
    out, frac = orc.ffn_forward_sparse_axpy_f32(x, flat, pt, st, h, i, 32, BF16, nan)
    assert frac == 0.0 and np.all(out == 0.0)
    # all-zero gate: max|silu| == 0 makes every lane active whatever tau is
    _, act = orc.build_active_mask(np.zeros(5, np.float32), nan)
    assert act.size == 5


def test_transpose_requantize_uses_f32_inverse(orc):
    """ffn_axpy.rs:406-419: codes are round(v * (1 / scale)) with the f32
    scale max|v| / 7, and the bf16 rounding of the scale is only what is
    stored.  Source scale 0.125 with a -8 and a 4 in the destination group:
    scale = 1/7 in f32, v = 0.5 -> 0.5 * 6.9999995 = 3.4999998 -> code 3;
    with 1 / bf16(scale) = 1 / 0.142578125 it would be 3.507 -> code 4."""
    h, i = 64, 32
    codes = np.zeros((h, i), np.int64)
    codes[0, :] = -8   # the group max: |-8 * 0.125| = 1.0
    codes[1, :] = 4    # v = 0.5
    codes[2, :] = 3    # v = 0.375 -> 2.6249998 -> 3 either way
    packed, scales = _crate_down(orc, h, i, codes, np.full((h, i // 32), 0x3E00))  # 0.125
    pt, st = orc.transpose_requantize_down(packed, scales, h, i)
    got = (np.stack([pt & 15, pt >> 4], -1).reshape(i, h).astype(np.int64) - 8)
    assert np.all(got[:, 0] == -7) and np.all(got[:, 1] == 3) and np.all(got[:, 2] == 3)
    st16 = st.view(np.uint16).reshape(i, h // 32)
    assert np.all(st16[:, 0] == 0x3E12)  # bf16(1/7) = 0.142578125


def np_requantize(w):
    """ffn_axpy.rs:393-432 on an exactly dequantised source w [h, i] (f32):
    groups of 32 along h of w^T, scale = max|v| / 7 (f32; 1.0 when 0), codes
    round-half-away(v * f32(1 / scale)) clamped to [-8, 7], stored scale bf16
    (RNE)."""
    h, i = w.shape
    g = np.ascontiguousarray(w.T).reshape(i, h // 32, 32).astype(np.float32)
    m = np.max(np.abs(g), axis=2)
    scale = np.where(m == 0, np.float32(1.0), m / np.float32(7.0)).astype(np.float32)
    inv = np.where(m == 0, np.float32(0.0), np.float32(1.0) / scale).astype(np.float32)
    q = (g * inv[..., None]).astype(np.float32).astype(np.float64)
    q = np.clip(np.sign(q) * np.floor(np.abs(q) + 0.5), -8, 7).astype(np.int64)
    b = scale.view(np.uint32).astype(np.uint64)
    sbits = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return q.reshape(i, h), sbits


def test_np_requantize_matches_oracle(orc):
    """The numpy restatement above (used for the GPU's generalised formats)
    equals the oracle's transpose_requantize_down on the crate's format."""
    h, i = 256, 128
    rng = np.random.default_rng(21)
    packed, scales = rand_layout(rng, h, i, 32, BF16)
    pt, st = orc.transpose_requantize_down(packed, scales, h, i)
    q, sb = np_requantize(orc.dequant(packed, scales, h, i, 32, BF16))
    got = np.stack([pt & 15, pt >> 4], -1).reshape(i, h).astype(np.int64) - 8
    assert np.array_equal(got, q)
    assert np.array_equal(st.view(np.uint16).reshape(i, h // 32), sb)


# ----------------------------------------------------------------------------
# f4: the OpenVINO CascadiaInt4Gemv format (gemv_offload.cpp:150-340, 623-638)
# ----------------------------------------------------------------------------

def test_ov_gemv_sign_extension_closed_form(orc):
    """Two's-complement nibbles: byte 0x8F holds lo = 0xF -> -1 and hi = 0x8
    -> -8 (the crate's offset form would read 7 and 0); with unit scales and a
    one-hot activation the output is that code exactly."""
    n, k, g = 2, 64, 32
    packed = np.full((n, k // 2), 0x8F, np.uint8)
    packed[1] = 0x70  # lo 0, hi 7
    sc = np.full(n * (k // g), 0x3C00, np.uint16)  # f16 1.0
    for col, want in ((0, (-1.0, 0.0)), (1, (-8.0, 7.0)), (34, (-1.0, 0.0)), (63, (-8.0, 7.0))):
        a = np.zeros(k, np.float32)
        a[col] = 1.0
        assert tuple(orc.ov_gemv(packed, sc, a, n, k, g)) == want, col


@pytest.mark.parametrize("g", [32, 64, 128, 48])
def test_ov_gemv_is_crate_gemv_of_xored_bytes(orc, g):
    """(x ^ 8) - 8 == (x ^ 8) - 8 with x ^ 8 the crate's offset nibble: the
    OV bytes XOR 0x88 in the crate layout give the same products, so the
    crate's GEMV over them (f16 scales) matches to f32 summation rounding;
    and an f64 brute force of the two's-complement decode pins both."""
    n, k = 24, 384
    rng = np.random.default_rng(g)
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sc = orc.fill_scales(g, 3, n * (k // g), F16)
    a = rng.normal(0, 1, k).astype(np.float32)
    got = orc.ov_gemv(packed, sc, a, n, k, g)
    lo = ((packed & 15).astype(np.int64) ^ 8) - 8
    hi = ((packed >> 4).astype(np.int64) ^ 8) - 8
    q = np.stack([lo, hi], -1).reshape(n, k)
    s = np.repeat(np.frombuffer(sc.tobytes(), np.float16).astype(np.float64).reshape(n, k // g), g, 1)
    want64 = (q * s) @ a.astype(np.float64)
    assert np.allclose(got, want64, rtol=1e-5, atol=1e-5 * np.max(np.abs(want64)))
    if g % 32 == 0:
        crate = orc.gemv((packed ^ 0x88).reshape(-1), sc.view(np.uint8), a, n, k, g, F16)
        assert np.allclose(got, crate, rtol=1e-5, atol=1e-5 * np.max(np.abs(want64)))
