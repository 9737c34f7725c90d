"""GPU parity of the load-time quantiser (cascadia_int4_quantize_bf16, the
crate's quantize_int4_group, shell_int4.rs:148-212) against the oracle:
packed nibbles and bf16 scales bit-identical; then the quantised weights
through the one-token GEMV against the oracle GEMV on the oracle's bytes."""
import numpy as np
import pytest
import torch

from conftest import MAX_ABS_TOL, REL_L2_TOL, max_abs, rel_l2

pytestmark = pytest.mark.gpu
BF16 = 0


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


def weights_bf16(orc, n, k, g, seed):
    """bf16 bits of N(0, 0.05) weights, with an all-zero group, a group of
    exact rounding ties (max 0.875: scale 0.125 exactly, so w * 8 lands on
    k + 0.5) and a group of signed zeros."""
    rng = np.random.default_rng(seed)
    w = rng.normal(0, 0.05, (n, k)).astype(np.float32)
    w[0, :g] = 0.0
    if n > 1:
        ties = (np.arange(g) % 7 * 2 + 1) * 0.0625 * np.where(np.arange(g) % 2, -1.0, 1.0)
        ties[0] = 0.875
        w[1, :g] = ties.astype(np.float32)
    wb = orc.f32_to_bf16(w).reshape(n, k)
    if n > 2:
        wb[2, :g] = np.where(np.arange(g) % 2, 0x8000, 0).astype(np.uint16)
    return wb.reshape(-1)


@pytest.mark.parametrize("n,k,g", [(16, 256, 32), (300, 7168, 32), (130, 1024, 128), (64, 4096, 64),
                                   (7, 96, 96), (33, 2048, 256)])
def test_quantize_bit_identical_to_oracle(cl, orc, n, k, g):
    wb = weights_bf16(orc, n, k, g, n + k + g)
    packed, scales = cl.quantize_int4_group(dev(wb.view(np.int16)), n, k, g)
    want_p, want_s = orc.quantize_int4_group(wb, n, k, g)
    got_p, got_s = host(packed), host(scales)
    assert np.array_equal(got_s, want_s.view(np.uint8).reshape(-1)), f"scales differ {n}x{k} G{g}"
    assert np.array_equal(got_p, want_p.reshape(-1)), f"codes differ {n}x{k} G{g}"
    # the tie group: codes 7 and +-1, +-2, ... (round half away from zero), nibble q + 8
    if n > 1 and g >= 32:
        row = got_p[(k // 2):(k // 2) + g // 2]
        q = np.stack([row & 15, row >> 4], 1).reshape(-1).astype(np.int32) - 8
        j = np.arange(g)
        want_q = (j % 7 + 1) * np.where(j % 2, -1, 1)
        want_q[0] = 7
        assert np.array_equal(q, want_q), "rounding ties"


def test_quantize_then_gemv(cl, orc):
    """GPU-quantised weights, tiled, through the one-token GEMV: the oracle
    GEMV on the oracle's bytes."""
    n, k, g = 1024, 4096, 32
    wb = weights_bf16(orc, n, k, g, 5)
    packed, scales = cl.quantize_int4_group(dev(wb.view(np.int16)), n, k, g)
    pt, st = cl.tile_weights(packed, scales, n, k, g)
    x = orc.fill_normal_f32(3, 41, k)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    cl.dequant_gemm_int4_multi_auto(pt, st, dev(x), n, k, 1, y, group_size=g,
                                    scale_dtype=cl.SCALE_BF16, tiling=cl.TILING_MFMA)
    want_p, want_s = orc.quantize_int4_group(wb, n, k, g)
    want = orc.gemm_multi(want_p, want_s.view(np.uint8), x, n, k, 1, g, BF16).reshape(-1)
    got = host(y)
    assert rel_l2(got, want) <= REL_L2_TOL and max_abs(got, want) <= MAX_ABS_TOL


def test_quantize_rejects_bad_shapes(cl):
    w = torch.zeros(8 * 96, dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError):
        cl.quantize_int4_group(w, 8, 96, 32 + 16)  # group not a multiple of 32
    with pytest.raises(ValueError):
        cl.quantize_int4_group(w, 8, 96, 64)  # k_cols not a multiple of the group
    with pytest.raises(ValueError):
        cl.quantize_int4_group(w, 8, 128, 32)  # length mismatch (kernel.rs-style assert)


def test_quantised_expert_vs_fp32_swiglu(cl, orc):
    """ov_moe.rs:888-920 on the device: the crate's test expert (hidden 64,
    inter 32, its hashed weights in [-0.1, 0.1)) quantised by the GPU
    quantiser from bf16, then expert_forward on the GPU, within rel-L2 0.1 of
    the fp32 SwiGLU of the unquantised weights -- the crate's bar (this case
    measures 0.084 through the oracle); and equal to the oracle's expert on
    the oracle's bytes at the parity bars."""
    h, m, g = 64, 32, 32

    def mk(n, seed):  # the crate test's generator (ov_moe.rs:888-920)
        i = np.arange(n, dtype=np.uint64)
        v = ((i * 2654435761 + seed) & 0xFFFFFFFF) % 1000
        return ((v.astype(np.float32) / np.float32(1000) - np.float32(0.5)) *
                np.float32(0.2)).astype(np.float32)

    gate, up, down, x = mk(m * h, 1), mk(m * h, 2), mk(h * m, 3), mk(h, 4)
    parts, want_flat = [], []
    for w, n, k in ((gate, m, h), (up, m, h), (down, h, m)):
        wb = orc.f32_to_bf16(w).reshape(-1)
        p, s = cl.quantize_int4_group(dev(wb.view(np.int16)), n, k, g)
        parts += [p, s]
        op, os_ = orc.quantize_int4_group(wb, n, k, g)
        want_flat += [op.view(np.uint8).reshape(-1), os_.view(np.uint8).reshape(-1)]
    xb = orc.f32_to_bf16(x)
    out = torch.empty(h, dtype=torch.int16, device="cuda")
    cl.expert_forward(dev(xb.view(np.int16)), *parts, out, group_size=g, scale_dtype=cl.SCALE_BF16)
    got = orc.bf16_to_f32(host(out).view(np.uint16))
    G, U, D = (a.astype(np.float64) for a in (gate.reshape(m, h), up.reshape(m, h), down.reshape(h, m)))
    gg, uu = G @ x, U @ x
    fp32 = D @ ((gg / (1 + np.exp(-gg))) * uu)
    assert rel_l2(got, fp32) < 0.1, f"int4 expert vs fp32 SwiGLU rel_l2={rel_l2(got, fp32):.3g}"
    want = orc.bf16_to_f32(orc.expert_forward(xb, np.concatenate(want_flat), h, m, g, BF16))
    assert rel_l2(got, want) <= REL_L2_TOL and max_abs(got, want) <= MAX_ABS_TOL
