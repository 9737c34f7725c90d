"""GPU parity of the OpenVINO CascadiaInt4Gemv format
(crates/cascadia-ov-genai-shim/cpp/gemv_offload.cpp:150-340, 413-660):
two's-complement nibbles converted once to the crate's offset nibbles
(bit-exact: every byte XOR 0x88), then the op's evaluate() -- segments of
output rows concatenated, f16 or f32 activations and outputs -- against the
oracle's restatement of its scalar path (oracle.ov_gemv, pinned on the CPU by
a sign-extension closed form and an f64 brute force).  Bars: f32 outputs
rel-L2 <= 1e-3 and max-abs <= 2e-2; f16 outputs rel-L2 <= 1e-3 and within
one f16 ulp of the oracle's f32 result rounded (+ 1e-5 max|y|)."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import assert_f32_close

pytestmark = pytest.mark.gpu


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


def ov_matrix(orc, n, k, g, seed):
    packed = orc.fill_bytes(seed, 90, n * k // 2)
    scales = orc.fill_scales(seed, 91, n * (k // g), 1)  # f16 bits
    return packed, scales


def test_ov_to_crate_bit_exact(cl, orc):
    packed = orc.fill_bytes(3, 1, 4099)  # a tail past whole words
    got = host(cl.ov_to_crate(dev(packed)))
    assert np.array_equal(got, packed ^ 0x88)
    t = dev(packed)
    cl.ov_to_crate(t, t)  # in place
    assert np.array_equal(host(t), packed ^ 0x88)


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("k,g", [(4096, 128), (2048, 32), (1536, 64)])
def test_ov_gemv_one_row(cl, orc, k, g, tiled):
    n = 1000
    packed, scales = ov_matrix(orc, n, k, g, k + g)
    p = cl.ov_to_crate(dev(packed))
    s = dev(scales.view(np.uint8))
    if tiled:
        p, s = cl.tile_weights(p, s, n, k, g)
    a = orc.fill_normal_f32(4, k, k)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    cl.ov_gemv([(p, s, n, cl.TILING_MFMA if tiled else cl.TILING_CRATE)], k, g, dev(a), out)
    assert_f32_close(host(out), orc.ov_gemv(packed, scales, a, n, k, g), f"ov {k} G{g}")


@pytest.mark.parametrize("rows", [1, 3, 16])
def test_ov_gemv_segments_f16(cl, orc, rows):
    """Three fused segments (q/k/v-like: 1024 + 256 + 256 rows), f16
    activations and output, tiled weights."""
    k, g = 2048, 128
    ns = [1024, 256, 256]
    mats = [ov_matrix(orc, n, k, g, 10 + j) for j, n in enumerate(ns)]
    segs = []
    for (packed, scales), n in zip(mats, ns):
        p, s = cl.tile_weights(cl.ov_to_crate(dev(packed)), dev(scales.view(np.uint8)), n, k, g)
        segs.append((p, s, n, cl.TILING_MFMA))
    a16 = orc.fill_normal_f32(5, rows, rows * k).astype(np.float16).reshape(rows, k)
    out = torch.empty((rows, sum(ns)), dtype=torch.float16, device="cuda")
    cl.ov_gemv(segs, k, g, dev(a16), out)
    got = host(out).astype(np.float64)
    want = np.concatenate([np.stack([orc.ov_gemv(p_, s_, a16[r].astype(np.float32), n, k, g)
                                     for r in range(rows)]) for (p_, s_), n in zip(mats, ns)],
                          axis=1)
    w16 = want.astype(np.float16).astype(np.float64)
    ulp = np.spacing(np.abs(want.astype(np.float16))).astype(np.float64)
    assert np.all(np.abs(got - w16) <= ulp + 1e-5 * np.max(np.abs(want)))
    r = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert r <= 1e-3
