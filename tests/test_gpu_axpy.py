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


def test_transpose_requantize_f32_inverse(cl, orc):
    """The closed form of test_oracle's f32-inverse pin on the GPU: a group
    holding -8 and 4 at source scale 0.125 transposes to codes -7 and 3 (not
    4, which 1 / bf16(scale) would give), scale bits 0x3E12."""
    from test_oracle import _crate_down
    h, i = 64, 32
    codes = np.zeros((h, i), np.int64)
    codes[0, :] = -8
    codes[1, :] = 4
    codes[2, :] = 3
    packed, scales = _crate_down(orc, h, i, codes, np.full((h, i // 32), 0x3E00))
    pt, st = cl.transpose_requantize_down(dev(packed), dev(scales), h, i)
    pt, st = host(pt), host(st)
    got = np.stack([pt & 15, pt >> 4], -1).reshape(i, h).astype(np.int64) - 8
    assert np.all(got[:, 0] == -7) and np.all(got[:, 1] == 3) and np.all(got[:, 2] == 3)
    assert np.all(st.view(np.uint16).reshape(i, h // 32)[:, 0] == 0x3E12)


def test_transpose_requantize_g128_f16(cl, orc):
    """The generalised source format (G 128 along intermediate, fp16 scales:
    config 1's down, which the crate's G 32 / bf16 function does not take):
    the GPU codes and scales equal the crate's re-quantisation (restated in
    numpy above) applied to the source dequantised bit-exactly."""
    h, i, g = 512, 1024, 128
    packed = orc.fill_bytes(4, 80, h * i // 2)
    scales = orc.fill_scales(4, 81, h * (i // g), 1).view(np.uint8).copy()
    from test_oracle import np_requantize
    w = orc.dequant(packed, scales, h, i, g, 1)  # pinned bit-exact dequantisation
    want_q, want_s = np_requantize(w)
    pt, st = cl.transpose_requantize_down(dev(packed), dev(scales), h, i, group_size=g,
                                          scale_dtype=1)
    pt, st = host(pt), host(st)
    got_q = np.stack([pt & 15, pt >> 4], -1).reshape(i, h).astype(np.int64) - 8
    assert np.array_equal(st.view(np.uint16).reshape(i, h // 32), want_s)
    assert np.array_equal(got_q, want_q)


def test_capture_refuses_library_workspace_growth(cl, orc):
    """Inside a HIP graph capture, a call that would grow the library's own
    workspace (a device synchronisation and a reallocation) is refused with
    ERR_ARG before anything is launched; with a caller workspace the same
    call captures, and its replays give the eager result."""
    h, i, n = 32768, 32, 131072  # 4096 slices x 32768 x 4 B = 512 MiB of partials
    pt = torch.full((i * h // 2,), 0x99, dtype=torch.uint8, device="cuda")
    st = dev(np.full(i * (h // 32), 0x3F80, np.uint16).view(np.uint8))
    s = torch.ones(i, dtype=torch.float32, device="cuda")
    act = torch.zeros(n, dtype=torch.int32, device="cuda")  # row 0, n times
    y = torch.zeros(h, dtype=torch.float32, device="cuda")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with pytest.raises(cl.CascadiaInt4Error) as ei:
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                cl.dequant_axpy_int4_active(pt, st, s, act, i, h, y)
    assert ei.value.rc == -2
    del g
    torch.cuda.synchronize()
    small = act[:100]
    ws = torch.empty(cl.lib().cascadia_int4_axpy_workspace_bytes(h, 100), dtype=torch.uint8,
                     device="cuda")
    y_eager = torch.zeros(h, dtype=torch.float32, device="cuda")
    cl.dequant_axpy_int4_active(pt, st, s, small, i, h, y_eager, workspace=ws)
    g = torch.cuda.CUDAGraph()
    y.zero_()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cl.dequant_axpy_int4_active(pt, st, s, small, i, h, y, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), f"replay {rep}"
    # 0x99: codes 1, scale 1.0, each of 100 active rows adds 1
    assert float(y_eager[0]) == 100.0


def test_capture_on_library_workspace_survives_growth(cl, orc):
    """A graph captured on the library's own (already large enough) workspace
    keeps replaying the eager result after a later, larger eager call has
    grown that workspace: the growth keeps the old buffer alive instead of
    freeing it under the graph.  Torch allocations made after the growth
    must not alias the captured buffer either, so the replay's result is
    compared after fresh allocations have been written."""
    h, i = 4096, 64
    pt = dev(orc.fill_bytes(6, 90, i * h // 2))
    st = dev(np.full(i * (h // 32), 0x3F80, np.uint16).view(np.uint8))
    s = torch.linspace(-1.0, 1.0, i, dtype=torch.float32, device="cuda")
    small = torch.arange(0, i, 3, dtype=torch.int32, device="cuda")
    y_eager = torch.zeros(h, dtype=torch.float32, device="cuda")
    cl.dequant_axpy_int4_active(pt, st, s, small, i, h, y_eager)  # warms the workspace
    y = torch.zeros(h, dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            cl.dequant_axpy_int4_active(pt, st, s, small, i, h, y)
    torch.cuda.current_stream().wait_stream(side)
    # a much larger eager call grows the library workspace past the captured one
    big = torch.zeros(1 << 18, dtype=torch.int32, device="cuda")
    y_big = torch.zeros(h, dtype=torch.float32, device="cuda")
    cl.dequant_axpy_int4_active(pt, st, s, big, i, h, y_big)
    torch.cuda.synchronize()
    junk = [torch.full((1 << 22,), 7.0, device="cuda") for _ in range(8)]
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), f"replay {rep} after growth"
    assert all(float(j[-1]) == 7.0 for j in junk), "a replay wrote into later allocations"
