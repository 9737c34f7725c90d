"""Calls on two streams at once, each with its own workspace and outputs,
equal the same calls made one after another, bit for bit.

The header promises that calls are reentrant for distinct output buffers
when each brings its own workspace (include/cascadia_int4.h).  Here the
expert FFN at one and four tokens (at four tokens both projections split K
across workgroups into partials in the workspace), the f32-in FFN at three
tokens, and MoE layers at
5 and 70 tokens (one prep launch, then separate routing / grouping launches;
the shared expert forks onto the library's side stream) are enqueued on two
streams, alternating, with no synchronisation between them, and every output
is compared with the serial result.
"""
import numpy as np
import pytest
import torch

from test_gpu_moe import build

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


def expert(orc, h, i, g, sdt, seed):
    flat = orc.fill_bytes(seed, 60, orc.expert_bytes(h, i, g)).copy()
    offs, sizes = orc.expert_offsets(h, i, g)
    for s_ in (1, 3, 5):
        flat[offs[s_]:offs[s_] + sizes[s_]] = orc.fill_scales(seed, 61 + s_, sizes[s_] // 2,
                                                              sdt).view(np.uint8)
    return flat


def test_two_streams_equal_serial(cl, orc):
    print("two streams: expert FFN M1/M4, f32 FFN, MoE T5/T70", flush=True)
    h, i, g = 1024, 3072, 128
    W = cl.ExpertWeights(dev(expert(orc, h, i, g, F16, 5)), h, i, g, F16).tiled()
    E, mh, mi, k, si = 16, 512, 384, 4, 128
    _, _, ex = build(cl, orc, E, mh, mi, 32, F16, 6, shared_inter=si, tiled=True)

    # each job: (a closure issuing the call on the current stream into its
    # outputs with its workspace, the output tensors)
    def make_jobs():
        jobs = []
        for T in (1, 4):
            x = cl.fill_normal(torch.empty((T, h), dtype=torch.bfloat16, device="cuda"), 7, T)
            out = torch.empty((T, h), dtype=torch.bfloat16, device="cuda")
            ws = torch.empty(cl.ffn_workspace_bytes(h, i, T, g), dtype=torch.uint8, device="cuda")
            jobs.append((lambda x=x, out=out, ws=ws: cl.expert_forward(
                x, *W.slices(), out, group_size=g, scale_dtype=F16, workspace=ws,
                tiling=cl.TILING_MFMA), [out]))
        xf = cl.fill_normal(torch.empty((3, h), dtype=torch.float32, device="cuda"), 8, 3)
        of = torch.empty((3, h), dtype=torch.float32, device="cuda")
        wsf = torch.empty(cl.ffn_sparse_workspace_bytes(h, i, 3, g), dtype=torch.uint8,
                          device="cuda")
        jobs.append((lambda: cl.ffn_forward_sparse_f32(
            xf, h, i, *W.slices(), of, 0.0, group_size=g, scale_dtype=F16, workspace=wsf,
            tiling=cl.TILING_MFMA), [of]))
        for T in (5, 70):
            x = cl.fill_normal(torch.empty((T, mh), dtype=torch.float32, device="cuda"), 9, T)
            lg = cl.fill_normal(torch.empty((T, E), dtype=torch.float32, device="cuda"), 10, T)
            out = torch.empty((T, mh), dtype=torch.float32, device="cuda")
            ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
            wts = torch.empty((T, k), dtype=torch.float32, device="cuda")
            ws = torch.empty(cl.moe_workspace_bytes(ex, k, T), dtype=torch.uint8, device="cuda")
            jobs.append((lambda x=x, lg=lg, out=out, ids=ids, wts=wts, ws=ws: cl.moe_forward(
                ex, x, out, top_k=k, logits=lg, mode=cl.ROUTE_SIGMOID_BIAS, scale=2.5,
                residual=x, ids_out=ids, weights_out=wts, workspace=ws), [out, ids, wts]))
        return jobs

    serial = make_jobs()
    for fn, _ in serial:
        fn()
        torch.cuda.synchronize()
    want = [[t.clone() for t in outs] for _, outs in serial]

    a_jobs, b_jobs = make_jobs(), make_jobs()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for rep in range(6):
        for j in range(len(a_jobs)):
            with torch.cuda.stream(sa):
                a_jobs[j][0]()
            with torch.cuda.stream(sb):
                b_jobs[(j + rep) % len(b_jobs)][0]()
    torch.cuda.synchronize()
    for jobs, name in ((a_jobs, "stream a"), (b_jobs, "stream b")):
        for j, (_, outs) in enumerate(jobs):
            for t, w in zip(outs, want[j]):
                assert torch.equal(t, w), f"{name}, job {j}: differs from the serial call"
