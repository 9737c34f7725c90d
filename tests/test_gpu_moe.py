"""GPU parity of the sparse-MoE layer (routing, grouped expert FFNs, shared
expert, slot-ordered combine) against the CPU oracle.

The oracle restates the runner's per-token loop (runner.rs:1806-1832): per
token, per slot in selection order, skip w < threshold, y = bf16 ->
f32(expert_forward(bf16(x))), moe += w * y, h = residual + shared + moe, with
the shared expert f32 in / f32 out (shell_int4.rs:629).  Routing follows
shell_int4.rs:588-620 / glm/gate.rs:24-62 (sigmoid + bias, ties to the lower
id, renormalise + scale) or a softmax over the top-k logits.

Bars: ids identical; routing weights within 4 f32 ulps (sigmoid / exp come
from different libms: parity of those last bits is unpinned); h within rel-L2
1e-3 / max-abs 2e-2, and h - residual (the experts' contribution alone)
within rel-L2 1e-3.  The layer is checked with the GPU's own routing fed to
the oracle, so a near-tie resolved differently by one libm ulp cannot move a
token to another expert between the two sides.
"""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2

pytestmark = pytest.mark.gpu
BF16, F16 = 0, 1


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


def make_experts(orc, E, h, i, g, sdt, seed):
    """E crate-layout expert blobs at a 256-byte stride, seeded scales."""
    per = orc.expert_bytes(h, i, g)
    stride = (per + 255) // 256 * 256
    blob = np.zeros(E * stride, np.uint8)
    offs, sizes = orc.expert_offsets(h, i, g)
    for e in range(E):
        b = orc.fill_bytes(seed, 1000 + e, per)
        for s in (1, 3, 5):
            b[offs[s]:offs[s] + sizes[s]] = orc.fill_scales(seed, 5000 + 10 * e + s, sizes[s] // 2, sdt).view(np.uint8)
        blob[e * stride:e * stride + per] = b
    return blob, stride


def make_shared(orc, h, i, g, sdt, seed, sigma=0.02, offset=1e-3):
    per = orc.expert_bytes(h, i, g)
    b = orc.fill_bytes(seed, 900, per)
    offs, sizes = orc.expert_offsets(h, i, g)
    for s in (1, 3, 5):
        b[offs[s]:offs[s] + sizes[s]] = orc.fill_scales(seed, 910 + s, sizes[s] // 2, sdt, sigma,
                                                        offset).view(np.uint8)
    return b


def build(cl, orc, E, h, i, g, sdt, seed, shared_inter=0, tiled=True):
    blob, stride = make_experts(orc, E, h, i, g, sdt, seed)
    shared = make_shared(orc, h, shared_inter, g, sdt, seed) if shared_inter else None
    sh = cl.ExpertWeights(dev(shared), h, shared_inter, g, sdt) if shared_inter else None
    ex = cl.MoEExperts.from_crate(dev(blob), E, h, i, g, sdt, stride=stride, shared=sh, tiled=tiled)
    return blob, shared, ex


def bf16_ulp(v):
    f = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.maximum(f, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def check_layer(orc, got, x, blob, shared, shared_inter, E, h, i, g, sdt, ids, w, thr, what):
    """h rel-L2 <= 1e-3; the experts' part (h - residual) rel-L2 <= 1e-3; and
    every element within max-abs 2e-2 or, where the routed expert outputs are
    so large that one bf16 ulp exceeds that, within sum_k w_k * ulp(y_k) (the
    crate rounds each expert output to bf16, kernel.rs:133-135, so a
    last-place flip there is the one difference two f32 summation orders may
    leave) plus 1e-5 x max|h - residual|."""
    want = orc.moe_layer(x, blob, E, shared, shared_inter, h, i, g, sdt, ids.astype(np.int64), w, thr)
    r = rel_l2(got, want)
    assert r <= REL_L2_TOL, f"{what}: h rel_l2={r:.3g}"
    xs = x.reshape(got.shape)
    d_got = got.astype(np.float64) - xs
    d_want = want.astype(np.float64) - xs
    rd = rel_l2(d_got, d_want)
    assert rd <= REL_L2_TOL, f"{what}: experts' part rel_l2={rd:.3g}"
    T = got.shape[0]
    stride = blob.size // E
    per = orc.expert_bytes(h, i, g)
    allow = np.full(got.shape, MAX_ABS_TOL, np.float64)
    for t in range(T):
        xb = orc.f32_to_bf16(xs[t].astype(np.float32))
        ulps = np.zeros(h, np.float64)
        for kk in range(ids.shape[1]):
            if w[t, kk] < thr:
                continue
            e = int(ids[t, kk])
            y = orc.expert_forward(xb, blob[e * stride:e * stride + per], h, i, g, sdt)
            ulps += abs(float(w[t, kk])) * bf16_ulp(orc.bf16_to_f32(y))
        allow[t] = np.maximum(allow[t], ulps + 1e-5 * float(np.max(np.abs(d_want))))
    worst = float(np.max(np.abs(d_got - d_want) / allow))
    assert worst <= 1.0, f"{what}: max_abs={max_abs(got, want):.3g}, worst {worst:.2f} of allowance"


def route_oracle(orc, logits, bias, k, mode, scale, norm):
    T = logits.shape[0]
    ids = np.empty((T, k), np.int64)
    w = np.empty((T, k), np.float32)
    for t in range(T):
        if mode == 1:
            ids[t], w[t] = orc.route_sigmoid_bias(logits[t], bias, k, scale, norm)
        else:
            ids[t], w[t] = orc.route_softmax_topk(logits[t], k)
    return ids, w


# T <= 64 takes the one-workgroup prep kernel, larger T the separate
# route / group / gather launches
@pytest.mark.parametrize("T", [33, 100])
@pytest.mark.parametrize("E,k,mode,ties", [(16, 4, 1, False), (256, 8, 2, False), (384, 8, 1, False),
                                           (64, 16, 1, True), (37, 5, 2, True), (1024, 8, 1, False)])
def test_routing_matches_oracle(cl, orc, E, k, mode, ties, T):
    h, i, g = 64, 32, 32
    _, _, ex = build(cl, orc, E, h, i, g, BF16, 3)
    logits = orc.fill_normal_f32(7, E, T * E).reshape(T, E)
    if ties:
        logits = np.round(logits * 2) / 2  # many exact ties
    bias = (orc.fill_normal_f32(8, E, E) * 0.05).astype(np.float32) if mode == 1 else None
    scale = 2.827 if mode == 1 else 1.0
    x = orc.fill_normal_f32(9, h, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    cl.moe_forward(ex, dev(x), out, top_k=k, logits=dev(logits),
                   bias=None if bias is None else dev(bias), mode=mode, scale=scale,
                   normalize=True, ids_out=ids_o, weights_out=w_o)
    want_ids, want_w = route_oracle(orc, logits, bias, k, mode, scale, True)
    got_ids, got_w = host(ids_o), host(w_o)
    assert np.array_equal(got_ids, want_ids), "routing ids differ"
    ulp = np.spacing(np.abs(want_w)).astype(np.float64)
    assert np.all(np.abs(got_w.astype(np.float64) - want_w) <= 4 * ulp), "routing weights differ"


@pytest.mark.parametrize("T", [1, 2, 5, 40, 80])
@pytest.mark.parametrize("mode,shared_inter,tiled,thr", [(1, 64, True, 0.0), (2, 0, True, 0.0),
                                                          (1, 0, False, 0.0), (2, 96, False, 0.2)])
def test_moe_layer_small(cl, orc, T, mode, shared_inter, tiled, thr):
    E, k, h, i, g, sdt = 16, 4, 256, 128, 32, BF16
    blob, shared, ex = build(cl, orc, E, h, i, g, sdt, 11, shared_inter, tiled)
    logits = orc.fill_normal_f32(12, T, T * E).reshape(T, E)
    x = orc.fill_normal_f32(13, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=mode, scale=1.0, threshold=thr,
                   residual=xd, ids_out=ids_o, weights_out=w_o)
    got, ids, w = host(out), host(ids_o), host(w_o)
    check_layer(orc, got, x, blob, shared, shared_inter, E, h, i, g, sdt, ids, w, thr,
                f"T={T} mode={mode} shared={shared_inter} tiled={tiled} thr={thr}")
    if thr > 0 and T > 1:
        assert (w < thr).any(), "threshold case should skip some slots"


@pytest.mark.parametrize("mode,shared_inter,thr", [(1, 128, 0.0), (2, 0, 0.2), (1, 0, 0.3)])
def test_moe_one_token_g128(cl, orc, mode, shared_inter, thr):
    """One routed token over tiled G128 experts: one row per expert chunk, the
    one-token GEMV in grouped mode (gathered f32 row, then hi/lo planes); slots
    under the threshold leave empty chunks (all of them at thr 0.3 with four
    sigmoid weights near 0.25)."""
    E, k, h, i, g, sdt, T = 16, 4, 512, 384, 128, F16, 1
    blob, shared, ex = build(cl, orc, E, h, i, g, sdt, 17, shared_inter, True)
    logits = orc.fill_normal_f32(18, T, T * E).reshape(T, E)
    x = orc.fill_normal_f32(19, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=mode, scale=1.0, threshold=thr,
                   residual=xd, ids_out=ids_o, weights_out=w_o)
    got, ids, w = host(out), host(ids_o), host(w_o)
    check_layer(orc, got, x, blob, shared, shared_inter, E, h, i, g, sdt, ids, w, thr,
                f"one token mode={mode} shared={shared_inter} thr={thr}")
    if thr > 0:
        assert (w < thr).any(), "threshold case should skip some slots"


@pytest.mark.parametrize("k,thr", [(6, 0.0), (6, 0.3), (16, 0.0)])
def test_moe_one_token_given_ids(cl, orc, k, thr):
    """One token, given ids with repeats (one expert in several slots), tiled
    G128 experts: each slot is its own row; slots under the threshold skipped;
    top-k 16 leaves one wave per slot in the down + combine launch."""
    E, h, i, g, T = 20, 384, 256, 128, 1
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 23, 128, True)
    rng = np.random.default_rng(k)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
    ids[0, 1] = ids[0, 0]
    ids[0, 3] = ids[0, 0]
    w = rng.random((T, k)).astype(np.float32)
    x = orc.fill_normal_f32(24, T, T * h).reshape(T, h)
    xd = dev(x)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    cl.moe_forward(ex, xd, out, top_k=k, mode=cl.ROUTE_IDS, ids=dev(ids), weights=dev(w),
                   threshold=thr, residual=xd)
    check_layer(orc, host(out), x, blob, shared, 128, E, h, i, g, F16, ids, w, thr,
                f"one token given ids k={k} thr={thr}")


@pytest.mark.parametrize("h,shared_inter", [(256, 64), (1024, 256), (4096, 512)])
def test_moe_one_token_top1_shared(cl, orc, h, shared_inter):
    """One token, top-1 routing and a tiled shared expert, hidden <= 4096: the
    fused down + combine launch writes the routed sum ([hidden] f32) into the
    expert-output region while the shared expert runs beside it; at top_k 1
    that region must still hold hidden f32 values without reaching the shared
    expert's output."""
    E, k, i, g, T = 8, 1, 128, 32, 1
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 51, shared_inter, True)
    logits = orc.fill_normal_f32(52, T, T * E).reshape(T, E)
    x = orc.fill_normal_f32(53, T, T * h).reshape(T, h)
    xd = dev(x)
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    for rep in range(3):
        out = torch.empty((T, h), dtype=torch.float32, device="cuda")
        cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=cl.ROUTE_SIGMOID_BIAS,
                       scale=1.0, normalize=False, residual=xd, ids_out=ids_o, weights_out=w_o)
        check_layer(orc, host(out), x, blob, shared, shared_inter, E, h, i, g, F16, host(ids_o),
                    host(w_o), 0.0, f"top-1 one token h={h} shared={shared_inter} call {rep}")


@pytest.mark.parametrize("E,shared_inter,mode", [(300, 128, 1), (300, 0, 2), (40, 128, 1)])
def test_moe_one_token_routing_launch(cl, orc, E, shared_inter, mode):
    """One token: more than 256 experts route in a launch of their own (the
    gate/up GEMV reads its slots), 256 or fewer inside the GEMV; with a shared
    expert the routed down writes the weighted sum and the finish adds
    residual + shared after the join."""
    k, h, i, g, T = 8, 256, 256, 32, 1
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 27, shared_inter, True)
    logits = orc.fill_normal_f32(28, T, T * E).reshape(T, E)
    bias = orc.fill_normal_f32(29, 1, E) * np.float32(0.1)
    x = orc.fill_normal_f32(30, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    kw = dict(bias=dev(bias), scale=2.5, normalize=True) if mode == 1 else {}
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=mode, residual=xd,
                   ids_out=ids_o, weights_out=w_o, **kw)
    ids, w = host(ids_o), host(w_o)
    want_ids, want_w = route_oracle(orc, logits, bias if mode == 1 else None, k, mode,
                                    2.5 if mode == 1 else 1.0, True)
    assert np.array_equal(ids, want_ids), "routing ids differ"
    check_layer(orc, host(out), x, blob, shared, shared_inter, E, h, i, g, F16, ids, w, 0.0,
                f"one token E={E} shared={shared_inter} mode={mode}")


@pytest.mark.parametrize("sh_mode", ["0", "1", "2"])
@pytest.mark.parametrize("E,h,i,g,mode,si", [(24, 7168, 2048, 32, 1, 256), (260, 4608, 128, 128, 1, 256),
                                             (24, 7168, 2048, 32, 1, 2048), (260, 4608, 128, 128, 1, 128)])
def test_moe_one_token_wide_hidden(cl, orc, tuning, E, h, i, g, mode, si, sh_mode):
    """One token with more 16-row output tiles than CUs (hidden > 4096): the
    gate/up launch leaves a chunk table of one row per slot, the grouped down
    and the combine kernel follow; config 4 dims (G32, shared expert) on a
    24-expert subset, and 260 experts (routing in a launch of its own).  A
    shared expert of the routed experts' inter size runs as an always-on slot
    of both launches (f32 x as hi / lo planes, f32 out); another size runs as
    its own FFN beside them.  CASCADIA_INT4_MOE1_SHARED picks how a shared
    expert of the routed shape runs: 1 (the default) both halves as slots, 2
    the gate/up as a GEMV beside the routed one and the down as a slot, 0 its
    own FFN."""
    if si != i and sh_mode != "2":
        pytest.skip("the mode applies to a shared expert of the routed shape")
    tuning("CASCADIA_INT4_MOE1_SHARED", sh_mode)
    k, T = 8, 1
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 33, si, True)
    logits = orc.fill_normal_f32(34, T, T * E).reshape(T, E)
    bias = orc.fill_normal_f32(35, 1, E) * np.float32(0.1)
    x = orc.fill_normal_f32(36, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), bias=dev(bias), mode=mode,
                   scale=2.827, normalize=True, residual=xd, ids_out=ids_o, weights_out=w_o)
    check_layer(orc, host(out), x, blob, shared, si, E, h, i, g, F16, host(ids_o), host(w_o),
                0.0, f"one token E={E} h={h} shared={si}")


@pytest.mark.parametrize("T", [24, 70])
def test_moe_given_ids_and_determinism(cl, orc, T):
    """ROUTE_IDS with repeated experts across tokens; two calls bit-identical."""
    E, k, h, i, g = 8, 3, 128, 64, 32
    blob, _, ex = build(cl, orc, E, h, i, g, F16, 21)
    rng = np.random.default_rng(5)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
    ids[:, 1] = 2  # one hot expert: many tokens, several chunks
    w = rng.random((T, k)).astype(np.float32)
    x = orc.fill_normal_f32(22, T, T * h).reshape(T, h)
    xd = dev(x)
    o1 = torch.empty((T, h), dtype=torch.float32, device="cuda")
    o2 = torch.empty((T, h), dtype=torch.float32, device="cuda")
    for o in (o1, o2):
        cl.moe_forward(ex, xd, o, top_k=k, mode=cl.ROUTE_IDS, ids=dev(ids), weights=dev(w),
                       residual=xd)
    a, b = host(o1), host(o2)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "not deterministic"
    check_layer(orc, a, x, blob, None, 0, E, h, i, g, F16, ids, w, 0.0, "given ids")


@pytest.mark.parametrize("T", [1, 2, 8])
def test_moe_config3_minimax_shape(cl, orc, T):
    """Config 3 dims (H 3072, I 1536, G128 fp16, softmax over the top 8) on a
    64-expert subset."""
    E, k, h, i, g = 64, 8, 3072, 1536, 128
    blob, _, ex = build(cl, orc, E, h, i, g, F16, 31)
    logits = orc.fill_normal_f32(32, T, T * E).reshape(T, E)
    x = orc.fill_normal_bf16(33, T, T * h)
    x = (x.astype(np.uint32) << 16).view(np.float32).reshape(T, h)  # bf16 activations
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=cl.ROUTE_SOFTMAX_TOPK,
                   residual=xd, ids_out=ids_o, weights_out=w_o)
    check_layer(orc, host(out), x, blob, None, 0, E, h, i, g, F16, host(ids_o), host(w_o), 0.0,
                f"config3 T={T}")


@pytest.mark.parametrize("T", [2, 3])
def test_moe_config4_kimi_shape(cl, orc, T):
    """Config 4 dims (H 7168, I 2048, G32 fp16, sigmoid routing renormalised
    x 2.827, one shared expert) on a 24-expert subset, Zipf-skewed logits; two
    tokens run as one-row chunks on the grouped one-token GEMV."""
    E, k, h, i, g = 24, 8, 7168, 2048, 32
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 41, shared_inter=2048)
    perm = np.random.default_rng(1).permutation(E)
    logits = (-1.1 * np.log1p(perm)[None, :] + orc.fill_normal_f32(42, T, T * E).reshape(T, E)).astype(np.float32)
    x = orc.fill_normal_f32(43, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=cl.ROUTE_SIGMOID_BIAS,
                   scale=2.827, normalize=True, residual=xd, ids_out=ids_o, weights_out=w_o)
    check_layer(orc, host(out), x, blob, shared, 2048, E, h, i, g, F16, host(ids_o), host(w_o),
                0.0, "config4")
