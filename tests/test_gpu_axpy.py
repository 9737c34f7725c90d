"""GPU parity of the AXPY form of the sparse down projection (ffn_axpy.rs):
transpose_requantize_down bit-identical to the oracle, dequant_axpy_int4_active
against the oracle's sums (rel-L2 / max-abs tolerance: the GPU adds the active
rows in another order)."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import assert_f32_close

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


def crate_down(orc, h, i, seed):
    packed = orc.fill_bytes(seed, 70, h * i // 2)
    scales = orc.fill_scales(seed, 71, h * (i // 32), BF16).reshape(h, i // 32)
    scales[:32, 1] = 0  # zero scales: destination groups of zeros (scale 1.0, code 0)
    return packed, scales.view(np.uint8).reshape(-1)


@pytest.mark.parametrize("h,i", [(96, 64), (512, 256), (7168, 2048), (4096, 1536)])
def test_transpose_requantize_bit_identical(cl, orc, h, i):
    packed, scales = crate_down(orc, h, i, h + i)
    pt, st = cl.transpose_requantize_down(dev(packed), dev(scales), h, i)
    want_p, want_s = orc.transpose_requantize_down(packed, scales, h, i)
    assert np.array_equal(host(st), want_s), f"scales {h}x{i}"
    assert np.array_equal(host(pt), want_p), f"codes {h}x{i}"


@pytest.mark.parametrize("h,i,n_act", [(512, 256, 40), (7168, 2048, 300), (4096, 14336, 1900),
                                       (7168, 2048, 2048), (96, 64, 1)])
def test_axpy_matches_oracle(cl, orc, h, i, n_act):
    packed, scales = crate_down(orc, h, i, 3 * h + i)
    want_p, want_s = orc.transpose_requantize_down(packed, scales, h, i)
    pt, st = cl.transpose_requantize_down(dev(packed), dev(scales), h, i)
    rng = np.random.default_rng(n_act)
    s = rng.normal(0, 1, i).astype(np.float32)
    active = np.sort(rng.choice(i, n_act, replace=False)).astype(np.uint32)
    y0 = rng.normal(0, 1, h).astype(np.float32)
    y = dev(y0)
    cl.dequant_axpy_int4_active(pt, st, dev(s), dev(active.view(np.int32)), i, h, y)
    want = orc.dequant_axpy_active(want_p, want_s, s, active, i, h, y=y0)
    assert_f32_close(host(y), want, f"axpy {h}x{i} n={n_act}")


def test_axpy_order_empty_and_bad_ids(cl, orc):
    h, i = 512, 256
    packed, scales = crate_down(orc, h, i, 9)
    pt, st = cl.transpose_requantize_down(dev(packed), dev(scales), h, i)
    want_p, want_s = orc.transpose_requantize_down(packed, scales, h, i)
    s = orc.fill_normal_f32(9, 72, i)
    rng = np.random.default_rng(9)
    act = rng.permutation(i)[:50].astype(np.uint32)  # unsorted
    y = torch.zeros(h, dtype=torch.float32, device="cuda")
    cl.dequant_axpy_int4_active(pt, st, dev(s), dev(act.view(np.int32)), i, h, y)
    assert_f32_close(host(y), orc.dequant_axpy_active(want_p, want_s, s, act, i, h), "unsorted")
    # empty list: y unchanged
    y1 = dev(np.arange(h, dtype=np.float32))
    cl.dequant_axpy_int4_active(pt, st, dev(s), torch.empty(0, dtype=torch.int32, device="cuda"),
                                i, h, y1)
    assert np.array_equal(host(y1), np.arange(h, dtype=np.float32))
    # ids past the intermediate size are skipped
    bad = np.concatenate([act[:10], np.array([i, i + 7, 0xFFFFFFFF], np.uint32)])
    y2 = torch.zeros(h, dtype=torch.float32, device="cuda")
    cl.dequant_axpy_int4_active(pt, st, dev(s), dev(bad.view(np.int32)), i, h, y2)
    assert_f32_close(host(y2), orc.dequant_axpy_active(want_p, want_s, s, act[:10], i, h), "bad ids")
    with pytest.raises(ValueError):
        cl.transpose_requantize_down(dev(packed), dev(scales), h + 16, i)
