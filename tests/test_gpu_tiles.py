"""GPU parity of the MFMA-tile GEMMs (grouped.hip) against the CPU oracle.

They run an expert FFN of many tokens (65 and more; expert_forward for bf16
rows, ffn_forward_sparse_f32 at tau 0 for f32 rows: the shared expert) and
every MoE layer of 65 tokens or more: routing, grouping into 128-row chunks,
the grouped gate/up with the SwiGLU epilogue into hi / lo planes, the grouped
down, the slot-order combine.  Groups of 32 and 64 columns take the
transposed-fragment steps, 128 the plain ones.  Bars as for the other
kernels: bf16 outputs rel-L2 <= 1e-3 and within one bf16 ulp of the oracle
(+ 1e-5 max|y|); f32 outputs rel-L2 <= 1e-3, max-abs <= 2e-2; MoE layers as in
test_gpu_moe.check_layer.
"""
import numpy as np
import pytest
import torch

from conftest import REL_L2_TOL, rel_l2
from test_gpu_gemm import assert_bf16_close, assert_f32_close
from test_gpu_moe import build, check_layer

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


def expert(orc, h, i, g, sdt, seed):
    flat = orc.fill_bytes(seed, 50, orc.expert_bytes(h, i, g)).copy()
    offs, sizes = orc.expert_offsets(h, i, g)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 51 + s_, sizes[s_] // 2,
                                                              sdt).view(np.uint8)
    return flat


@pytest.mark.parametrize("M", [65, 130, 257])
@pytest.mark.parametrize("h,i,g,sdt", [(512, 384, 32, F16), (1024, 768, 64, BF16),
                                       (768, 1280, 128, F16), (512, 256, 256, BF16)])
def test_expert_forward_tiles(cl, orc, tuning, M, h, i, g, sdt):
    """expert_forward over M rows on the tile GEMMs (bf16 rows, bf16 out;
    the tile threshold lowered to 65 rows)."""
    tuning("CASCADIA_INT4_FFN_TILE_TOKENS", "65")
    flat = expert(orc, h, i, g, sdt, M + g)
    W = cl.ExpertWeights(dev(flat), h, i, g, sdt).tiled()
    xb = orc.fill_normal_bf16(M, 52, M * h)
    out = torch.empty(M * h, dtype=torch.int16, device="cuda")
    cl.expert_forward(dev(xb.view(np.int16).reshape(M, h)), *W.slices(), out, group_size=g,
                      scale_dtype=sdt, tiling=cl.TILING_MFMA)
    want = orc.cpu_expert_forward(xb, M, flat, h, i, g, sdt)
    assert_bf16_close(host(out).view(np.uint16).reshape(M, h), want, f"tiles M{M} G{g}")


@pytest.mark.parametrize("M,g", [(65, 32), (100, 64), (200, 128)])
def test_ffn_f32_tiles(cl, orc, tuning, M, g):
    """The f32-in / f32-out FFN (the shared expert) over M rows: x split into
    hi / lo planes, both planes through every MFMA."""
    tuning("CASCADIA_INT4_FFN_TILE_TOKENS", "65")
    h, i, sdt = 512, 384, F16
    flat = expert(orc, h, i, g, sdt, 7 + g)
    W = cl.ExpertWeights(dev(flat), h, i, g, sdt).tiled()
    x = orc.fill_normal_f32(8, M, M * h).reshape(M, h)
    out = torch.empty((M, h), dtype=torch.float32, device="cuda")
    cl.ffn_forward_sparse_f32(dev(x), h, i, *W.slices(), out, 0.0, group_size=g, scale_dtype=sdt,
                              tiling=cl.TILING_MFMA)
    want = np.stack([orc.ffn_forward_f32(x[t], flat, h, i, g, sdt)[0] for t in range(M)])
    assert_f32_close(host(out), want, f"ffn f32 tiles M{M} G{g}")


@pytest.mark.parametrize("hot_rows", ["1", "48"])
@pytest.mark.parametrize("T", [65, 200])
@pytest.mark.parametrize("g,mode,shared_inter,thr", [(32, 1, 256, 0.0), (128, 2, 0, 0.0),
                                                     (64, 1, 128, 0.2)])
def test_moe_tiles(cl, orc, tuning, T, g, mode, shared_inter, thr, hot_rows):
    """MoE layers of 65+ tokens (routing by logits; the tile thresholds
    lowered to 65 tokens): every expert on the tile GEMMs (hot_rows 1), or the
    hybrid split -- experts with 48+ rows on tiles, the others on the skinny
    kernels' 16-row chunks."""
    tuning("CASCADIA_INT4_MOE_TILE_TOKENS", "65")
    tuning("CASCADIA_INT4_FFN_TILE_TOKENS", "65")
    tuning("CASCADIA_INT4_MOE_TILE_ROWS", hot_rows)
    E, k, h, i, sdt = 12, 4, 512, 256, F16
    blob, shared, ex = build(cl, orc, E, h, i, g, sdt, 61 + g, shared_inter, True)
    logits = orc.fill_normal_f32(62, T, T * E).reshape(T, E)
    x = orc.fill_normal_f32(63, T, T * h).reshape(T, h)
    out = torch.empty((T, h), dtype=torch.float32, device="cuda")
    ids_o = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w_o = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = dev(x)
    cl.moe_forward(ex, xd, out, top_k=k, logits=dev(logits), mode=mode, scale=1.0,
                   threshold=thr, residual=xd, ids_out=ids_o, weights_out=w_o)
    check_layer(orc, host(out), x, blob, shared, shared_inter, E, h, i, g, sdt, host(ids_o),
                host(w_o), thr, f"tiles T={T} G{g} mode={mode}")


def test_moe_tiles_hot_expert(cl, orc, tuning):
    """Given ids sending every token to one expert (300 rows: three 128-row
    chunks, the last partial) plus scattered ones; two calls bit-identical."""
    tuning("CASCADIA_INT4_MOE_TILE_TOKENS", "65")
    E, k, h, i, g, T = 9, 3, 384, 256, 32, 300
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 71, 128, True)
    rng = np.random.default_rng(3)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
    ids[:, 0] = 4
    ids[:, 1] = np.where(ids[:, 1] == 4, 5, ids[:, 1])
    ids[:, 2] = np.where((ids[:, 2] == 4) | (ids[:, 2] == ids[:, 1]), 0, ids[:, 2])
    ids[:, 1] = np.where(ids[:, 1] == ids[:, 2], 1, ids[:, 1])
    w = rng.random((T, k)).astype(np.float32)
    x = orc.fill_normal_f32(72, T, T * h).reshape(T, h)
    xd = dev(x)
    outs = []
    for _ in range(2):
        o = torch.empty((T, h), dtype=torch.float32, device="cuda")
        cl.moe_forward(ex, xd, o, top_k=k, mode=cl.ROUTE_IDS, ids=dev(ids), weights=dev(w),
                       residual=xd)
        outs.append(host(o))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "not deterministic"
    check_layer(orc, outs[0], x, blob, shared, 128, E, h, i, g, F16, ids, w, 0.0, "hot expert")


def test_tiles_match_skinny_path(cl, orc, tuning):
    """The same 80-token layer through both paths (the skinny grouped kernels
    forced by a high tile threshold): both within the bar of the oracle and of
    each other."""
    E, k, h, i, g, T = 10, 4, 512, 384, 32, 80
    blob, shared, ex = build(cl, orc, E, h, i, g, F16, 81, 128, True)
    logits = orc.fill_normal_f32(82, T, T * E).reshape(T, E)
    x = orc.fill_normal_f32(83, T, T * h).reshape(T, h)
    xd = dev(x)
    res = []
    for thr_tokens in ("65", "100000"):
        tuning("CASCADIA_INT4_MOE_TILE_TOKENS", thr_tokens)
        tuning("CASCADIA_INT4_FFN_TILE_TOKENS", thr_tokens)
        o = torch.empty((T, h), dtype=torch.float32, device="cuda")
        cl.moe_forward(ex, xd, o, top_k=k, logits=dev(logits), mode=1, scale=2.5,
                       residual=xd)
        res.append(host(o))
    d0, d1 = res[0] - x, res[1] - x
    assert rel_l2(d0, d1) <= REL_L2_TOL
