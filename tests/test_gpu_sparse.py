"""GPU parity of the activation-sparse expert FFN (tau > 0: ffn_sparsity.rs:
131-179 mask, 187-348 rows-subset up, 438-538 and 756-867 the two forms,
global and per-channel thresholds) against the oracle, in both weight
layouts, one and several token rows.

The mask compares |silu(gate)| with a cutoff, so a lane whose value lies
within the GEMV's rounding of the cutoff may land on either side.  Each case
checks from the oracle that no lane is that close (relative margin 1e-5 of
max|silu|; the GPU's gate agrees to ~1e-6), so the active counts must agree
exactly and the outputs to the usual tolerance."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import assert_bf16_close, assert_f32_close

pytestmark = pytest.mark.gpu
BF16, F16 = 0, 1
MARGIN = 1e-5


@pytest.fixture(scope="module")
def cl():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd

    return cascadia_amd


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_expert(orc, h, i, g, sdt, seed):
    flat = orc.fill_bytes(seed, 60, orc.expert_bytes(h, i, g))
    offs, sizes = orc.expert_offsets(h, i, g)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 61 + s_, sizes[s_] // 2, sdt).view(np.uint8)
    return flat


def margin(orc, flat, x_f32, h, i, g, sdt, tau, thr):
    """Smallest | |silu_i| - cutoff_i | / max|silu| over lanes (oracle), the
    max lane aside: it meets tau * itself exactly on both sides."""
    o, _ = orc.expert_offsets(h, i, g)
    gate = orc.gemv(flat[o[0]:o[1]], flat[o[1]:o[2]], x_f32, i, h, g, sdt)
    silu, _ = orc.build_active_mask(gate, tau, thresholds=thr)
    a = np.abs(silu.astype(np.float64))
    mx = a.max()
    cut = (thr.astype(np.float64) if thr is not None else tau) * mx
    d = np.abs(a - cut) / mx
    return float(np.min(np.where(a == mx, np.inf, d)))


def pick_x(orc, flat, h, i, g, sdt, tau, thr, seed):
    """The first seeded bf16 row from `seed` on with no lane near its cutoff."""
    for s in range(seed, seed + 50):
        xb = orc.fill_normal_bf16(s, 90, h)
        if margin(orc, flat, orc.bf16_to_f32(xb), h, i, g, sdt, tau, thr) > MARGIN:
            return xb
    raise AssertionError("no seed keeps every lane away from the cutoff")


CASES = [  # h, i, G, sdt, layout: False crate, True tiled, "rows" gate/down tiled + crate up
    (512, 256, 32, BF16, False),
    (7168, 2048, 32, BF16, True),   # the crate's HIDDEN / INTERMEDIATE
    (7168, 2048, 32, BF16, False),
    (7168, 2048, 32, BF16, "rows"),
    (4096, 1024, 128, F16, True),
    (4096, 1024, 128, F16, "rows"),
    (3072, 1536, 64, F16, False),
]


def _til(cl, tiled):
    return cl.TILING_MFMA_UP_ROWS if tiled == "rows" else cl.TILING_MFMA if tiled else cl.TILING_CRATE


def layout(cl, W, tiled):
    """(expert weights, tiling) for a test layout: False = the crate's, True =
    MFMA-tiled, "rows" = TILING_MFMA_UP_ROWS (up kept in rows)."""
    if tiled == "rows":
        return W.tiled(up_rows=True), cl.TILING_MFMA_UP_ROWS
    if tiled:
        return W.tiled(), cl.TILING_MFMA
    return W, cl.TILING_CRATE


@pytest.mark.parametrize("h,i,g,sdt,tiled", CASES)
@pytest.mark.parametrize("tau", [0.05, 0.3, 1.0])
def test_expert_forward_sparse_global(cl, orc, h, i, g, sdt, tiled, tau):
    flat = make_expert(orc, h, i, g, sdt, h + i + g)
    W, til = layout(cl, cl.ExpertWeights(dev(flat), h, i, g, sdt), tiled)
    T = 3
    xb = np.stack([pick_x(orc, flat, h, i, g, sdt, tau, None, 100 * t + int(tau * 100))
                   for t in range(T)])
    out = torch.empty(T * h, dtype=torch.int16, device="cuda")
    fr = cl.expert_forward_sparse(dev(xb.view(np.int16)), *W.slices(), out, tau, group_size=g,
                                  scale_dtype=sdt, tiling=til)
    got = host(out).view(np.uint16).reshape(T, h)
    for t in range(T):
        want, wf = orc.expert_forward_sparse(xb[t], flat, h, i, g, sdt, tau)
        assert fr[t] == wf, f"token {t}: active {fr[t]} vs {wf}"
        assert_bf16_close(got[t], want, f"{h}x{i} G{g} tau {tau} token {t}")
    if tau == 1.0:
        assert all(f == float(np.float32(1) / np.float32(i)) for f in fr)  # only the max lane
    # f32 form on the same rows
    xf = orc.bf16_to_f32(xb)
    o32 = torch.empty(T * h, dtype=torch.float32, device="cuda")
    fr32 = cl.ffn_forward_sparse_f32(dev(xf), h, i, *W.slices(), o32, tau, group_size=g,
                                     scale_dtype=sdt, tiling=til)
    got32 = host(o32).reshape(T, h)
    for t in range(T):
        want, wf = orc.ffn_forward_f32(xf[t], flat, h, i, g, sdt, tau)
        assert fr32[t] == wf
        assert_f32_close(got32[t], want, f"f32 {h}x{i} tau {tau} token {t}")


@pytest.mark.parametrize("h,i,g,sdt,tiled", [CASES[0], CASES[1], CASES[3], CASES[4]])
def test_sparse_per_channel(cl, orc, h, i, g, sdt, tiled):
    flat = make_expert(orc, h, i, g, sdt, 3 * h + i)
    W, til = layout(cl, cl.ExpertWeights(dev(flat), h, i, g, sdt), tiled)
    rng = np.random.default_rng(h + i)
    thr = rng.uniform(-0.1, 0.6, i).astype(np.float32)  # some lanes always on
    xb = pick_x(orc, flat, h, i, g, sdt, 0.0, thr, 7)
    xf = orc.bf16_to_f32(xb)
    out = torch.empty(h, dtype=torch.int16, device="cuda")
    f = cl.expert_forward_sparse_per_channel(dev(xb.view(np.int16)), *W.slices(), out, dev(thr),
                                             group_size=g, scale_dtype=sdt, tiling=til)
    want, wf = orc.expert_forward_sparse(xb, flat, h, i, g, sdt, 0.0, thresholds=thr)
    assert f == wf and 0 < wf < 1
    assert_bf16_close(host(out).view(np.uint16), want, "per-channel bf16")
    o32 = torch.empty(h, dtype=torch.float32, device="cuda")
    f = cl.ffn_forward_sparse_f32_per_channel(dev(xf), h, i, *W.slices(), o32, dev(thr),
                                              group_size=g, scale_dtype=sdt, tiling=til)
    want32, wf = orc.ffn_forward_f32(xf, flat, h, i, g, sdt, 0.0, thresholds=thr)
    assert f == wf
    assert_f32_close(host(o32), want32, "per-channel f32")
    # every threshold <= 0: the dense FFN (ffn_sparsity.rs:85-90)
    neg = -np.abs(thr)
    f = cl.ffn_forward_sparse_f32_per_channel(dev(xf), h, i, *W.slices(), o32, dev(neg),
                                              group_size=g, scale_dtype=sdt, tiling=til)
    assert f == 1.0
    assert_f32_close(host(o32), orc.ffn_forward_f32(xf, flat, h, i, g, sdt, 0.0)[0], "dense pc")


def test_sparse_edge_cases(cl, orc):
    h, i, g = 512, 256, 32
    flat = make_expert(orc, h, i, g, BF16, 11)
    W = cl.ExpertWeights(dev(flat), h, i, g, BF16)
    # x = 0: gate 0, max|silu| = 0, every lane active (ffn_sparsity.rs:151), out 0
    o32 = torch.full((h,), 7.0, dtype=torch.float32, device="cuda")
    f = cl.ffn_forward_sparse_f32(dev(np.zeros(h, np.float32)), h, i, *W.slices(), o32, 0.5)
    assert f == 1.0 and not np.any(host(o32))
    # tau 0 with a workspace of the sparse size: the dense FFN, fraction 1
    ws = torch.empty(cl.ffn_sparse_workspace_bytes(h, i, 1), dtype=torch.uint8, device="cuda")
    xf = orc.fill_normal_f32(1, 92, h)
    f = cl.ffn_forward_sparse_f32(dev(xf), h, i, *W.slices(), o32, 0.0, workspace=ws)
    assert f == 1.0
    assert_f32_close(host(o32), orc.ffn_forward_f32(xf, flat, h, i, g, BF16, 0.0)[0], "tau 0")
    # a caller workspace on the sparse branch
    assert margin(orc, flat, xf, h, i, g, BF16, 0.2, None) > MARGIN
    f = cl.ffn_forward_sparse_f32(dev(xf), h, i, *W.slices(), o32, 0.2, workspace=ws)
    want, wf = orc.ffn_forward_f32(xf, flat, h, i, g, BF16, 0.2)
    assert f == wf
    assert_f32_close(host(o32), want, "caller workspace")
    # thresholds of the wrong length (ffn_sparsity.rs:117-123 asserts)
    with pytest.raises(ValueError):
        cl.ffn_forward_sparse_f32_per_channel(dev(xf), h, i, *W.slices(), o32,
                                              dev(np.zeros(i - 1, np.float32)))


# ----------------------------------------------------------------------------
# the AXPY form (ffn_sparsity.rs:569-740): f32 in / out, plain SiLU, down as
# an AXPY over the active rows of transpose_requantize_down's matrix
# ----------------------------------------------------------------------------

def _axpy_case(cl, orc, h, i, g, sdt, tiled, seed):
    flat = make_expert(orc, h, i, g, sdt, seed)
    offs, sizes = orc.expert_offsets(h, i, g)
    W = cl.ExpertWeights(dev(flat), h, i, g, sdt)
    pt, st = cl.transpose_requantize_down(W.down_packed_bytes(), W.down_scale_bits(), h, i,
                                          group_size=g, scale_dtype=sdt)
    Wt, til = layout(cl, W, tiled)
    return flat, Wt, pt, st


@pytest.mark.parametrize("tau", [0.0, 0.1, 0.3])
@pytest.mark.parametrize("h,i,g,sdt,tiled", [(512, 256, 32, BF16, False),
                                             (7168, 2048, 32, BF16, True),
                                             (7168, 2048, 32, BF16, "rows"),
                                             (4096, 14336, 128, F16, True),
                                             (4096, 14336, 128, F16, "rows"),
                                             (3072, 1536, 128, F16, "rows"),
                                             (9216, 512, 128, F16, True)])
def test_axpy_ffn_matches_oracle(cl, orc, h, i, g, sdt, tiled, tau):
    """One token: output within rel-L2 1e-3 / max-abs 2e-2 of the oracle fed
    the same transposed down (bit-identical to the crate's for G 32 bf16; for
    config 1's G 128 fp16 source, pinned by test_transpose_requantize_g128_f16),
    the active fraction exact."""
    flat, W, pt, st = _axpy_case(cl, orc, h, i, g, sdt, tiled, h + i + g)
    x = orc.fill_normal_f32(91, h, h)
    if tau > 0:
        assert margin(orc, flat, x, h, i, g, sdt, tau, None) > MARGIN
    out = torch.empty(h, dtype=torch.float32, device="cuda")
    frac = cl.ffn_forward_sparse_axpy_f32(dev(x), h, i, W.gate_packed_bytes(), W.gate_scale_bits(),
                                          W.up_packed_bytes(), W.up_scale_bits(), pt, st, out, tau,
                                          group_size=g, scale_dtype=sdt,
                                          tiling=_til(cl, tiled))
    want, wfrac = orc.ffn_forward_sparse_axpy_f32(x, flat, host(pt), host(st), h, i, g, sdt, tau)
    assert frac == wfrac, f"active fraction {frac} != {wfrac}"
    assert_f32_close(host(out), want, f"axpy ffn {h}x{i} G{g} tau={tau}")


def test_axpy_ffn_rows_and_per_channel(cl, orc):
    """Three token rows, each against the oracle; per-channel thresholds of one
    value equal the global tau bit for bit (ffn_sparsity.rs:1497-1560);
    mixed per-channel thresholds against the oracle."""
    h, i, g, sdt, T = 1024, 768, 64, F16, 3
    flat, W, pt, st = _axpy_case(cl, orc, h, i, g, sdt, True, 5)
    x = orc.fill_normal_f32(92, T, T * h).reshape(T, h)
    args = (W.gate_packed_bytes(), W.gate_scale_bits(), W.up_packed_bytes(), W.up_scale_bits(),
            pt, st)
    kw = dict(group_size=g, scale_dtype=sdt, tiling=cl.TILING_MFMA)
    o1 = torch.empty((T, h), dtype=torch.float32, device="cuda")
    f1 = cl.ffn_forward_sparse_axpy_f32(dev(x), h, i, *args, o1, 0.2, **kw)
    o2 = torch.empty((T, h), dtype=torch.float32, device="cuda")
    f2 = cl.ffn_forward_sparse_axpy_f32_per_channel(dev(x), h, i, *args, o2,
                                                    torch.full((i,), 0.2, device="cuda"), **kw)
    assert np.array_equal(host(o1).view(np.uint32), host(o2).view(np.uint32)) and f1 == f2
    ptn, stn = host(pt), host(st)
    for t in range(T):
        want, wf = orc.ffn_forward_sparse_axpy_f32(x[t], flat, ptn, stn, h, i, g, sdt, 0.2)
        assert f1[t] == wf
        assert_f32_close(host(o1)[t], want, f"row {t}")
    thr = (np.random.default_rng(3).random(i) * 0.4).astype(np.float32)
    o3 = torch.empty((T, h), dtype=torch.float32, device="cuda")
    f3 = cl.ffn_forward_sparse_axpy_f32_per_channel(dev(x), h, i, *args, o3, dev(thr), **kw)
    for t in range(T):
        assert margin(orc, flat, x[t], h, i, g, sdt, 0.0, thr) > MARGIN
        want, wf = orc.ffn_forward_sparse_axpy_f32(x[t], flat, ptn, stn, h, i, g, sdt, 0.0,
                                                   thresholds=thr)
        assert f3[t] == wf
        assert_f32_close(host(o3)[t], want, f"per-channel row {t}")


def test_zero_token_rows(cl, orc):
    """Zero token rows: the crate's forwards loop over no rows and return an
    empty output (kernel.rs:75-136, ffn_sparsity.rs:438-538 iterate over
    x.len() / hidden rows).  Every FFN entry point returns OK without reading
    or writing, even with the NULL buffers of empty tensors, and the sparse
    forms report no fractions."""
    h, i, g = 512, 256, 32
    flat = make_expert(orc, h, i, g, BF16, 12)
    W0 = cl.ExpertWeights(dev(flat), h, i, g, BF16)
    pt, st = cl.transpose_requantize_down(W0.down_packed_bytes(), W0.down_scale_bits(), h, i,
                                          group_size=g, scale_dtype=BF16)
    xb = torch.empty((0, h), dtype=torch.int16, device="cuda")
    xf = torch.empty((0, h), dtype=torch.float32, device="cuda")
    ob = torch.empty((0, h), dtype=torch.int16, device="cuda")
    of = torch.empty((0, h), dtype=torch.float32, device="cuda")
    inter = torch.empty((0, i), dtype=torch.float32, device="cuda")
    for W in (W0, W0.tiled()):
        kw = dict(group_size=g, scale_dtype=BF16,
                  tiling=cl.TILING_MFMA if W is not W0 else cl.TILING_CRATE)
        cl.expert_forward(xb, *W.slices(), ob, **kw)
        cl.gate_up_silu(xf, *W.slices()[:4], inter, **kw)
        assert cl.expert_forward_sparse(xb, *W.slices(), ob, 0.3, **kw) == []
        assert cl.ffn_forward_sparse_f32(xf, h, i, *W.slices(), of, 0.3, **kw) == []
        assert cl.ffn_forward_sparse_f32(xf, h, i, *W.slices(), of, 0.0, **kw) == []
        assert cl.ffn_forward_sparse_axpy_f32(xf, h, i, *W.slices()[:4], pt, st, of, 0.3,
                                              **kw) == []
    torch.cuda.synchronize()


# ----------------------------------------------------------------------------
# the rows-subset GEMV on its own (ffn_sparsity.rs:187-348)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,g,sdt,tiled", [(300, 4096, 128, F16, False), (300, 4096, 128, F16, True),
                                             (130, 7168, 32, BF16, False), (64, 1024, 64, F16, True),
                                             (40, 65536, 128, F16, False)])
def test_rows_subset_gemv(cl, orc, n, k, g, sdt, tiled):
    """Listed rows (ascending, shuffled, repeated, and ids past n_rows, which
    are skipped) equal the oracle's GEMV rows within the GEMV bar; every other
    entry of y keeps the caller's value (the crate touches only active rows,
    ffn_sparsity.rs:184-186).  k = 65536 stages x through global memory (its
    f32 copy exceeds the LDS)."""
    rng = np.random.default_rng(n + k)
    packed = orc.fill_bytes(n, k, n * k // 2)
    scales = orc.fill_scales(n, k + 1, n * (k // g), sdt).view(np.uint8)
    x = orc.fill_normal_f32(n, 7, k)
    want = orc.gemv(packed, scales, x, n, k, g, sdt)
    P, S = dev(packed), dev(scales)
    if tiled:
        P, S = cl.tile_weights(P, S, n, k, g)
    rows = np.sort(rng.choice(n, size=n // 3, replace=False))
    rows = np.concatenate([rows, rows[:5], [n, n + 7, 2 ** 31]]).astype(np.uint32)
    rng.shuffle(rows)
    y = torch.full((n,), 7.0, dtype=torch.float32, device="cuda")
    cl.dequant_gemv_int4_rows_subset(P, S, dev(x), n, k, y, dev(rows.view(np.int32)), group_size=g,
                                     scale_dtype=sdt,
                                     tiling=cl.TILING_MFMA if tiled else cl.TILING_CRATE)
    got = host(y)
    on = np.zeros(n, bool)
    on[rows[rows < n]] = True
    assert np.all(got[~on] == 7.0), "rows outside the list were written"
    assert_f32_close(got[on], want[on], f"rows subset {n}x{k} G{g} tiled={tiled}")
    # an empty list reads nothing and writes nothing
    cl.dequant_gemv_int4_rows_subset(P, S, dev(x), n, k, y, torch.empty(0, dtype=torch.int32,
                                                                           device="cuda"),
                                     group_size=g, scale_dtype=sdt,
                                     tiling=cl.TILING_MFMA if tiled else cl.TILING_CRATE)
    assert np.array_equal(host(y), got)


# ----------------------------------------------------------------------------
# the mask builders and the mode-taking entry points (ffn_sparsity.rs:71-179)
# ----------------------------------------------------------------------------

def test_build_active_mask_modes(cl, orc):
    """silu within 4 ulps of the oracle's (the exp of two libms); the active
    ids exactly those the crate's rule gives on the GPU's own silu values
    (|silu| >= cutoff * max, ascending), and the oracle's ids wherever a lane
    is not within 1e-5 of its cutoff; the dense cases (tau <= 0, every
    per-channel threshold <= 0, an all-zero gate) list every lane, a NaN tau
    none (is_dense is `t <= 0`), tau 1 the max lane alone."""
    n = 3000
    gate = (orc.fill_normal_f32(5, 5, n) * np.float32(3)).astype(np.float32)
    rng = np.random.default_rng(2)
    pc = rng.uniform(-0.2, 0.7, n).astype(np.float32)
    cases = [("global 0.3", 0.3, None), ("global 0", 0.0, None), ("global -1", -1.0, None),
             ("global nan", float("nan"), None), ("global 1", 1.0, None),
             ("per-channel", 0.0, pc), ("per-channel <= 0", 0.0, -np.abs(pc))]
    G = dev(gate)
    for what, tau, thr in cases:
        if thr is None:
            silu, act = cl.build_active_mask(G, tau)
        else:
            silu, act = cl.build_active_mask_per_channel(G, dev(thr))
        s = host(silu)
        a = host(act).astype(np.int64)
        ws, wa = orc.build_active_mask(gate, tau, thresholds=thr)
        assert np.all(np.abs(s.astype(np.float64) - ws) <= 4 * np.spacing(np.abs(ws))), what
        mx = np.max(np.abs(s))
        dense = (thr is None and tau <= 0.0) or (thr is not None and np.all(thr <= 0.0))
        cut = (thr if thr is not None else np.float32(tau)) * np.float32(mx)
        mine = np.arange(n) if dense else np.nonzero(np.abs(s) >= cut)[0]
        assert np.array_equal(a, mine), f"{what}: ids differ from the rule on the GPU's silu"
        near = np.abs(np.abs(ws) - ((thr if thr is not None else tau) * np.max(np.abs(ws)))) \
            <= 1e-5 * np.max(np.abs(ws))
        far = ~near if not dense else np.ones(n, bool)
        assert np.array_equal(np.isin(np.arange(n), a)[far], np.isin(np.arange(n), wa)[far]), what
        if what == "global nan":
            assert a.size == 0
        if what == "global 1":
            assert a.size == 1 and a[0] == int(np.argmax(np.abs(s)))
    silu, act = cl.build_active_mask_mode(dev(np.zeros(17, np.float32)), cl.SparsityMode.Global(0.5))
    assert host(act).size == 17 and not np.any(host(silu))  # max 0: every lane
    with pytest.raises(ValueError):
        cl.build_active_mask_per_channel(G, dev(pc[:-1]))


def test_mode_entry_points_match_named_ones(cl, orc):
    """expert_forward_sparse_mode / ffn_forward_sparse_f32_mode with
    SparsityMode.Global / PerChannel (or a float / tensor) give the named
    entry points' results bit for bit (ffn_sparsity.rs:756-815, 373-436)."""
    h, i, g, sdt = 1024, 512, 64, F16
    flat = make_expert(orc, h, i, g, sdt, 77)
    W, til = layout(cl, cl.ExpertWeights(dev(flat), h, i, g, sdt), "rows")
    kw = dict(group_size=g, scale_dtype=sdt, tiling=til)
    xb = dev(orc.fill_normal_bf16(3, 3, 2 * h).view(np.int16))
    xf = dev(orc.fill_normal_f32(3, 4, 2 * h))
    thr = dev(np.random.default_rng(1).uniform(0.0, 0.5, i).astype(np.float32))
    outs = []
    for mode in (cl.SparsityMode.Global(0.2), 0.2):
        o = torch.empty(2 * h, dtype=torch.int16, device="cuda")
        outs.append((cl.expert_forward_sparse_mode(xb, *W.slices(), o, mode, **kw), host(o)))
    o = torch.empty(2 * h, dtype=torch.int16, device="cuda")
    ref = (cl.expert_forward_sparse(xb, *W.slices(), o, 0.2, **kw), host(o))
    for f, v in outs:
        assert f == ref[0] and np.array_equal(v, ref[1])
    o1 = torch.empty(2 * h, dtype=torch.float32, device="cuda")
    o2 = torch.empty(2 * h, dtype=torch.float32, device="cuda")
    f1 = cl.ffn_forward_sparse_f32_mode(xf, h, i, *W.slices(), o1, cl.SparsityMode.PerChannel(thr),
                                        **kw)
    f2 = cl.ffn_forward_sparse_f32_per_channel(xf, h, i, *W.slices(), o2, thr, **kw)
    assert f1 == f2 and torch.equal(o1, o2)


def test_mixed_layout_only_on_sparse_entry_points(cl, orc):
    """TILING_MFMA_UP_ROWS is an activation-sparse layout: the dense expert
    entry points refuse it (ERR_ARG) rather than misread the up rows."""
    h, i, g = 512, 256, 32
    flat = make_expert(orc, h, i, g, BF16, 13)
    W, til = layout(cl, cl.ExpertWeights(dev(flat), h, i, g, BF16), "rows")
    xb = torch.zeros(h, dtype=torch.int16, device="cuda")
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        cl.expert_forward(xb, *W.slices(), torch.empty_like(xb), group_size=g, tiling=til)
    assert ei.value.rc == -2


def test_bf16_conversions(cl, orc):
    """f32_to_bf16_bits (format.rs:151-160) bit-identical to the oracle's,
    which is pinned to half 2.7.1's from_f32, over random bit patterns and the
    special values; bf16_bits_to_f32 exact on all 65,536 patterns."""
    rng = np.random.default_rng(4)
    bits = rng.integers(0, 2 ** 32, 1 << 16, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001,
                        0xFFFFFFFF, 0x00000001, 0x3F808000, 0x3F818000, 0x7F7FFFFF],
                       np.uint32)
    x = np.concatenate([bits, special]).view(np.float32)
    got = host(cl.f32_to_bf16_bits(dev(x))).view(np.uint16)
    assert np.array_equal(got, orc.f32_to_bf16(x))
    allb = np.arange(1 << 16, dtype=np.uint16)
    back = host(cl.bf16_bits_to_f32(dev(allb.view(np.int16)))).view(np.uint32)
    assert np.array_equal(back, allb.astype(np.uint32) << 16)
    assert cl.f32_to_bf16_bits(1.0) == 0x3F80 and cl.bf16_bits_to_f32(0x4049) == 3.140625


def test_expert_weights_open(cl, orc, tmp_path):
    """ExpertWeights::open (format.rs:63-96): the file's bytes land in HBM
    unchanged (bytes past one expert ignored) and run as that expert."""
    h, i, g = 512, 256, 32
    flat = make_expert(orc, h, i, g, BF16, 21)
    p = tmp_path / "expert_000.bin"
    p.write_bytes(bytes(flat) + b"\x00" * 100)
    W = cl.ExpertWeights.open(str(p), hidden=h, inter=i, group_size=g)
    assert np.array_equal(host(W.flat)[:flat.size], flat)
    xb = orc.fill_normal_bf16(2, 2, h)
    out = torch.empty(h, dtype=torch.int16, device="cuda")
    cl.expert_forward(dev(xb.view(np.int16)), *W.slices(), out, group_size=g)
    assert_bf16_close(host(out).view(np.uint16), orc.expert_forward(xb, flat, h, i, g, BF16), "open")
