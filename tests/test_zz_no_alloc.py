"""The allocation-free expert FFN entry point (cascadia_int4_expert_forward_noalloc)
against cascadia_int4_expert_forward_device with a caller workspace: same
kernels, so the bf16 outputs must be bit-identical.  Two calls in a row, the
second with a smaller input, since every call shares the one static scratch.
The first case is also checked against the CPU oracle (rel-L2 <= 1e-3)."""
import ctypes as C

import numpy as np
import pytest
import torch

from conftest import REL_L2_TOL, rel_l2

pytestmark = pytest.mark.gpu
BF16, F16 = 0, 1
TILING_CRATE, TILING_MFMA = 0, 1


@pytest.fixture(scope="module")
def cl():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import cascadia_amd

    return cascadia_amd


def make_expert(cl, orc, h, i, g, sdt, seed, tiled):
    flat = orc.fill_bytes(seed, 31, orc.expert_bytes(h, i, g)).copy()
    offs, sizes = orc.expert_offsets(h, i, g)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 32 + s_, sizes[s_] // 2,
                                                              sdt).view(np.uint8)
    W = cl.ExpertWeights(torch.from_numpy(flat).cuda(), h, i, g, sdt)
    return flat, (W.tiled() if tiled else W)


def call_noalloc(cl, h, i, g, sdt, W, tiling, x, n, out):
    ex = cl._lib.Expert(*(t.data_ptr() for t in W.slices()), tiling)
    return cl.lib().cascadia_int4_expert_forward_noalloc(
        h, i, g, sdt, C.byref(ex), x.data_ptr(), n, out.data_ptr(),
        torch.cuda.current_stream().cuda_stream)


def call_device(cl, h, i, g, sdt, W, tiling, x, n, out):
    ex = cl._lib.Expert(*(t.data_ptr() for t in W.slices()), tiling)
    ws = torch.empty(max(cl.lib().cascadia_int4_ffn_workspace_bytes(h, i, g, n), 16),
                     dtype=torch.uint8, device="cuda")
    rc = cl.lib().cascadia_int4_expert_forward_device(
        h, i, g, sdt, C.byref(ex), x.data_ptr(), n, out.data_ptr(), ws.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return rc


# (hidden, inter, group, scale dtype, tiled, first n_tokens, second n_tokens)
CASES = [
    (4096, 14336, 128, F16, True, 16, 4),   # config 1 (Llama-3-8B FFN), MFMA-tiled
    (7168, 2048, 32, BF16, False, 8, 1),    # K2.6 expert dims, the crate's layout
    (3072, 1536, 128, F16, True, 16, 1),    # config 3 expert dims
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"h{c[0]}_i{c[1]}_g{c[2]}_n{c[5]}-{c[6]}")
def test_noalloc_matches_device_entry(cl, orc, case):
    h, i, g, sdt, tiled, n1, n2 = case
    print(f"noalloc case {case}", flush=True)
    flat, W = make_expert(cl, orc, h, i, g, sdt, 5, tiled)
    tiling = TILING_MFMA if tiled else TILING_CRATE
    assert cl.lib().cascadia_int4_ffn_workspace_bytes(h, i, g, n1) <= (8 << 20)
    for call, n in enumerate((n1, n2)):
        x = cl.fill_normal(torch.empty((n, h), dtype=torch.bfloat16, device="cuda"), 9, 40 + call)
        got = torch.full((n, h), -7.0, dtype=torch.bfloat16, device="cuda")
        want = torch.empty((n, h), dtype=torch.bfloat16, device="cuda")
        assert call_noalloc(cl, h, i, g, sdt, W, tiling, x, n, got) == 0
        torch.cuda.synchronize()
        assert call_device(cl, h, i, g, sdt, W, tiling, x, n, want) == 0
        g_bits = got.view(torch.int16).cpu().numpy()
        w_bits = want.view(torch.int16).cpu().numpy()
        assert np.array_equal(g_bits, w_bits), f"call {call} (n={n}): outputs differ"
        if call == 0:
            xb = x.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
            ref = orc.bf16_to_f32(orc.cpu_expert_forward(xb, n, flat, h, i, g, sdt))
            gf = orc.bf16_to_f32(g_bits.view(np.uint16))
            assert rel_l2(gf, ref) <= REL_L2_TOL


def test_noalloc_rejects_oversize(cl, orc):
    """A call whose workspace exceeds the static scratch is refused on the host
    (no kernel runs), and a following in-bounds call still works."""
    h, i, g, sdt = 4096, 14336, 128, F16
    n_big = 512  # [512, 14336] hi/lo planes alone are 28 MiB > 8 MiB
    assert cl.lib().cascadia_int4_ffn_workspace_bytes(h, i, g, n_big) > (8 << 20)
    _, W = make_expert(cl, orc, h, i, g, sdt, 6, True)
    x = cl.fill_normal(torch.empty((n_big, h), dtype=torch.bfloat16, device="cuda"), 9, 50)
    out = torch.empty((n_big, h), dtype=torch.bfloat16, device="cuda")
    assert call_noalloc(cl, h, i, g, sdt, W, TILING_MFMA, x, n_big, out) == -2
    got = torch.empty((2, h), dtype=torch.bfloat16, device="cuda")
    want = torch.empty((2, h), dtype=torch.bfloat16, device="cuda")
    assert call_noalloc(cl, h, i, g, sdt, W, TILING_MFMA, x[:2], 2, got) == 0
    torch.cuda.synchronize()
    assert call_device(cl, h, i, g, sdt, W, TILING_MFMA, x[:2], 2, want) == 0
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
