"""Benchmark of the INT4 weight-only matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--no-cpu] [--headline-only]
    python bench.py --profile | --profile-gemv | --profile-prefill | --profile-moe | --profile-sparse
                    | --profile-batches
        (launch one workload eagerly, untimed, for rocprofv3)

Headline: the Llama-3-8B-shaped decode FFN chain,
gate/up 14336x4096 + down 4096x14336, INT4 group 128 with fp16 scales, bf16
activations, M tokens.  One step = one expert_forward chain (two kernels:
fused gate/up/SiLU*up, then down with the bf16 output rounding) over one
batch of M tokens.  The weights are synthetic (seeded), made in the crate's
layout and converted once to the MFMA-tiled device layout (the upload step,
outside the timed region); steps rotate through enough distinct copies that
each matrix alone spans more than 2 x the 256 MB Infinity Cache, and that
cache is flushed before the timed replay, so every step streams its weights
from HBM.  The K timed steps are captured once as a HIP graph and replayed
once, bracketed by synchronisations, as a server's decode loop would run them.

`value` = algorithmic bytes per step (3 x (packed + scales) + M*H*2*2: the
weights read once plus activations in and out) x steps / wall time of the
timed region -> GB/s.  The roofline object covers the dominant kernel (the
fused gate/up kernel), timed with HIP events recorded on the stream the
kernels run on.  The CPU baseline is the oracle's AVX-512 port of the crate's
kernels on the host cores, on a bounded sample of the same workload.

`extra` (unless --headline-only) measures every other BASELINE config the
same way -- config 0 GEMV, config 1 at M 4 / 16, the four config 2 prefill
GEMMs, config 3 MoE at T 1 / 32 / 256, config 4 (four stacked layers) at T 1
/ 8 / 64 / 1024 -- each with event-timed GPU time, algorithmic bytes or flops,
the roofline fraction, and a CPU baseline of the crate's own dispatch on a
bounded sample (the per-token loop for seq > 64; the runner's per-(token,
slot) loop for MoE); plus the box's measured copy / read ceilings and the
f1 / f3 paths (shell projections, activation-sparse expert, AXPY down).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MALL_BYTES = 256 << 20
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "config1_gate_up_traffic.json")
# counter-measured HBM bytes / algorithmic bytes of the other decode workloads
# (rocprofv3 FETCH_SIZE + WRITE_SIZE passes over the bench's profile modes)
TRAFFIC_ALL = os.path.join(ROOT, "profiles", "traffic.json")
PREFILL_SHAPES = [(512, 4096), (512, 14336), (2048, 4096), (2048, 14336)]
CPU_SAMPLE_S = 2.0  # CPU seconds per secondary baseline


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--m", type=int, default=1, help="decode batch (tokens) of the headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--headline-only", action="store_true", help="skip the other configs")
    ap.add_argument("--extra", action="store_true", help="(default behaviour; kept for scripts)")
    ap.add_argument("--profile-gemv", action="store_true",
                    help="launch the config 0 GEMV 200 times over rotating copies, for rocprofv3")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="launch the config 2 prefill GEMMs eagerly, without timing, for rocprofv3")
    ap.add_argument("--profile-batches", action="store_true",
                    help="run the config 1 chain at M = 4 and 16, 40 eager calls each, for "
                         "rocprofv3")
    ap.add_argument("--profile-sparse", action="store_true",
                    help="launch the config 1 activation-sparse expert (tau 0.3) 50 times "
                         "eagerly, for rocprofv3")
    ap.add_argument("--profile-moe", action="store_true",
                    help="run configs 3 and 4 at T=--moe-tokens (a few steps), for rocprofv3")
    ap.add_argument("--moe-tokens", type=int, default=1, help="tokens of --profile-moe")
    ap.add_argument("--moe-config", type=int, default=0, choices=(0, 3, 4),
                    help="--profile-moe: config 3 or 4 only (0: both)")
    ap.add_argument("--profile", action="store_true",
                    help="launch the headline kernels and a 256 MiB copy (counter calibration) "
                         "eagerly, without timing, for rocprofv3")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def ffn_bytes(h, i, g, m):
    w = 3 * (i * h // 2 + i * (h // g) * 2)
    return w + m * h * 2 * 2


def gate_up_bytes(h, i, g, m):
    return 2 * (i * h // 2 + i * (h // g) * 2) + m * h * 2 + m * i * 4


def host_cpu():
    """nproc, the OpenMP threads the CPU port uses, and the CPU model."""
    import oracle as orc

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "threads": orc.cpu_threads(), "model": model,
            "isa": {2: "avx512", 1: "avx2", 0: "scalar"}[orc.cpu_isa()]}


def cpu_loop(fn, seconds):
    """Call fn(n) for n = 0, 1, ... for about `seconds` (one untimed warm-up
    call first); returns (calls, elapsed)."""
    fn(0)
    n = 0
    t0 = time.perf_counter()
    while True:
        fn(n)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return n, dt


def chain_copies(cl, h, i, g):
    """Distinct expert copies a rotating decode chain needs so that each of its
    matrices alone (the down, 1/3 of an expert, is the smallest) spans more
    than twice the Infinity Cache: no matrix is re-read from it, whichever of
    the chain's loads allocate there."""
    smallest = h * i // 2 + h * (i // g) * 2
    return math.ceil(2 * MALL_BYTES / smallest) + 1


class Copies:
    """`n` distinct synthetic experts: crate layout, tiled once for the GPU."""

    def __init__(self, cl, torch, h, i, g, sdt, n, seed=1, keep_crate=3):
        self.h, self.i, self.g = h, i, g
        nb = cl.expert_bytes(h, i, g)
        self.crate = []  # a few crate-layout blobs for the CPU baseline
        self.w = []
        for c in range(n):
            f = torch.empty(nb, dtype=torch.uint8, device="cuda")
            cl.fill_bytes(f, seed, 100 + c)
            W = cl.ExpertWeights(f, h, i, g, sdt)
            for j, s in enumerate((W.gate_scale_bits(), W.up_scale_bits(), W.down_scale_bits())):
                cl.fill_scales(s, seed, 1000 + 10 * c + j, sdt)
            self.w.append(W.tiled())
            if len(self.crate) < keep_crate:
                self.crate.append(f)
            del W, f
        torch.cuda.synchronize()


_MALL_FLUSH = []


def flush_mall(torch):
    """Read four times the Infinity Cache's size of other data, so that no
    weight bytes are left in it from setup or an earlier replay (loads that do
    not allocate in it, such as non-temporal ones, could otherwise keep hitting
    what setup left there).  A read leaves clean lines: the timed region does
    not pay for writing them back."""
    if not _MALL_FLUSH:
        buf = torch.empty(MALL_BYTES, dtype=torch.float32, device="cuda")
        buf.fill_(1.0)
        _MALL_FLUSH.append(buf)
    _MALL_FLUSH[0].sum()


def graph_time(torch, fn, steps):
    """Capture `steps` calls as one HIP graph and time one replay: wall clock
    between synchronisations, and HIP events on the replay stream.  The
    Infinity Cache is flushed between the upload replay and the timed one."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for k in range(steps):
                fn(k)
        g.replay()  # the first replay uploads the graph
        flush_mall(torch)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(s)
        g.replay()
        e1.record(s)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    torch.cuda.current_stream().wait_stream(s)
    del g
    return t1 - t0, e0.elapsed_time(e1) / 1e3


def chain_fn(cl, copies, x, out, sdt):
    nc = len(copies.w)

    def fn(k):
        cl.expert_forward(x, *copies.w[k % nc].slices(), out, group_size=copies.g,
                          scale_dtype=sdt, tiling=cl.TILING_MFMA)
    return fn


def gate_up_fn(cl, copies, x, inter, sdt):
    nc = len(copies.w)

    def fn(k):
        W = copies.w[k % nc]
        cl.gate_up_silu(x, W.gate_packed_bytes(), W.gate_scale_bits(), W.up_packed_bytes(),
                        W.up_scale_bits(), inter, group_size=copies.g, scale_dtype=sdt,
                        tiling=cl.TILING_MFMA)
    return fn


def cpu_chain_baseline(torch, copies, x, m, seconds):
    """expert_forward chains on the host (the crate's dispatch: a4 at one
    token, the blocked / multi tiles at 4..64), rotating the host copies."""
    import numpy as np

    import oracle as orc

    h, i, g = copies.h, copies.i, copies.g
    host = [c.cpu().numpy() for c in copies.crate]
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    out = np.empty((m, h), np.uint16)

    def run(n):
        orc.cpu_expert_forward(xb, m, host[n % len(host)], h, i, g, orc.SCALE_F16, out)
    n, dt = cpu_loop(run, seconds)
    isa = {2: "avx512", 1: "avx2", 0: "scalar"}[orc.cpu_isa()]
    return {
        "value": round(ffn_bytes(h, i, g, m) * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": orc.cpu_threads(),
        "kind": "port",
        "sample": f"{n} expert_forward chains (config1 M={m}) over {len(host)} host weight copies "
                  f"in {dt:.1f}s, {isa} kernels of the crate's dispatch, OpenMP",
        "tokens_per_s": round(m * n / dt, 3),
    }


def read_traffic(m):
    """HBM bytes per launch of the gate/up kernel from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), if present."""
    try:
        with open(TRAFFIC_FILE) as f:
            d = json.load(f)
        v = d.get(f"M{m}", {}).get("hbm_bytes_per_launch")
        return None if v is None else int(v)
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------
# the other BASELINE configs
# ---------------------------------------------------------------------------

def hbm_ceiling(cl, torch):
    """The box's measured streaming ceilings: a 1 GiB device copy (read +
    write bytes counted) and this library's streaming-read kernel
    (cascadia_int4_stream_read: the decode GEMV's weight-stream pattern
    without its arithmetic) over 60 MiB -- the size of config 1's gate/up --
    rotating through 16 buffers (more than twice the Infinity Cache), and over
    1 GiB; HIP events on the launch stream."""
    a = torch.ones(256 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    reps = 20
    e[0].record()
    for _ in range(reps):
        b.copy_(a)
    e[1].record()
    torch.cuda.synchronize()
    nb = a.numel() * 4
    tc = e[0].elapsed_time(e[1]) / 1e3 / reps
    del b
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    out = {"copy_GBps": round(2 * nb / tc / 1e9, 1)}
    small = [cl.fill_bytes(torch.empty(60 << 20, dtype=torch.uint8, device="cuda"), 9, j)
             for j in range(16)]
    for name, bufs, steps in (("read_60MiB_GBps", small, 320), ("read_1GiB_GBps", [a], 20)):
        def rd(r, bufs=bufs):
            cl.stream_read(bufs[r % len(bufs)], sink)
        for r in range(len(bufs)):
            rd(r)
        _, ev = graph_time(torch, rd, steps)
        out[name] = round(bufs[0].numel() * bufs[0].element_size() / (ev / steps) / 1e9, 1)
    del a, small
    torch.cuda.empty_cache()
    out["read_us_by_bytes"] = read_floor(cl, torch, sink)
    return out


# The byte counts the decode entries are set against: a 64 KiB read (the
# floor of one launch in a graph replay), config 0's GEMV, config 1's down and
# its fused gate/up.
READ_FLOOR_BYTES = {"64KiB": 64 << 10, "config0": 4096 * 4096 // 2 + 4096 * 32 * 2,
                    "config1_down": 4096 * 14336 // 2 + 4096 * 112 * 2,
                    "config1_gate_up": 2 * (14336 * 4096 // 2 + 14336 * 32 * 2)}


def read_floor(cl, torch, sink):
    """Microseconds per launch of the streaming-read kernel over each size of
    READ_FLOOR_BYTES (graph replays, buffers rotating past twice the Infinity
    Cache): what a plain read of a workload's weight bytes costs on this box,
    launch and first-byte latency included."""
    out = {}
    for name, nbytes in READ_FLOOR_BYTES.items():
        nb = (nbytes + 8191) // 8192 * 8192
        nbuf = max(2, min(64, math.ceil(2 * MALL_BYTES / nb) + 1))
        bufs = [cl.fill_bytes(torch.empty(nb, dtype=torch.uint8, device="cuda"), 9, j)
                for j in range(nbuf)]

        def rd(r, bufs=bufs):
            cl.stream_read(bufs[r % len(bufs)], sink)
        for r in range(nbuf):
            rd(r)
        steps = 1000 if nb < (32 << 20) else 300
        _, ev = graph_time(torch, rd, steps)
        out[name] = round(ev / steps * 1e6, 3)
        del bufs
    torch.cuda.empty_cache()
    return out


def config0(cl, torch, sdt, cpu):
    """Config 0: one 4096x4096 GEMV, f32 x, G128 fp16, over > 2x MALL of
    rotating weight copies."""
    import numpy as np

    import oracle as orc

    n = k = 4096
    g = 128
    nb, nsb = n * k // 2, n * (k // g) * 2
    ncp = math.ceil(2 * MALL_BYTES / (nb + nsb)) + 1
    PS = []
    for c in range(ncp):
        p = cl.fill_bytes(torch.empty(nb, dtype=torch.uint8, device="cuda"), 0, 200 + c)
        s = cl.fill_scales(torch.empty(nsb, dtype=torch.uint8, device="cuda"), 0, 300 + c, sdt)
        PS.append(cl.tile_weights(p, s, n, k, g))
        del p, s
    x = cl.fill_normal(torch.empty(k, dtype=torch.float32, device="cuda"), 0, 13)
    y = torch.empty(n, dtype=torch.float32, device="cuda")

    def gemv(r):
        pt, st = PS[r % ncp]
        cl.dequant_gemv_int4(pt, st, x, n, k, y, group_size=g, scale_dtype=sdt,
                             tiling=cl.TILING_MFMA)
    for r in range(10):
        gemv(r)
    steps = 1000
    wall, ev = graph_time(torch, gemv, steps)
    t = ev / steps
    b = nb + nsb + k * 4 + n * 4
    res = {"us_per_call": round(t * 1e6, 3), "wall_us_per_call": round(wall / steps * 1e6, 3),
           "GB/s": round(b / t / 1e9, 1), "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_bytes": b, "copies": ncp}
    del PS
    if cpu:
        hc = 16  # 139 MB of host copies: more than the host's last-level cache
        hp = [orc.fill_bytes(0, 200 + c, nb) for c in range(hc)]
        hs = [orc.fill_scales(0, 300 + c, nsb // 2, sdt).view(np.uint8).copy() for c in range(hc)]
        xh = x.cpu().numpy()
        yh = np.empty(n, np.float32)

        def run(r):
            orc.cpu_gemm(hp[r % hc], hs[r % hc], xh, n, k, 1, g, sdt, yh)
        cnt, dt = cpu_loop(run, CPU_SAMPLE_S)
        res["cpu_baseline"] = {"value": round(b * cnt / dt / 1e9, 3), "unit": "GB/s",
                               "cores": orc.cpu_threads(), "kind": "port",
                               "sample": f"{cnt} GEMVs, {hc} host copies, {dt:.1f}s"}
    return res


def config1_batches(cl, torch, sdt, copies, cpu):
    """Config 1 at M = 4 and 16: chain time, the fused gate/up kernel's
    event-timed duration and roofline fraction, CPU chains on the host."""
    res = {}
    h, i, g = copies.h, copies.i, copies.g
    for mm in (4, 16):
        xm = cl.fill_normal(torch.empty((mm, h), dtype=torch.bfloat16, device="cuda"), 0, 22)
        om = torch.empty((mm, h), dtype=torch.bfloat16, device="cuda")
        im = torch.empty((mm, i), dtype=torch.float32, device="cuda")
        fn = chain_fn(cl, copies, xm, om, sdt)
        gu = gate_up_fn(cl, copies, xm, im, sdt)
        for k in range(10):
            fn(k)
            gu(k)
        steps = 200
        wall, ev = graph_time(torch, fn, steps)
        _, ev_gu = graph_time(torch, gu, steps)
        t_gu = ev_gu / steps
        gub = gate_up_bytes(h, i, g, mm)
        e = {"us_per_chain": round(ev / steps * 1e6, 2),
             "wall_us_per_chain": round(wall / steps * 1e6, 2),
             "GB/s": round(ffn_bytes(h, i, g, mm) * steps / ev / 1e9, 1),
             "hbm_frac": round(ffn_bytes(h, i, g, mm) * steps / ev / 1e9 / HBM_PEAK_GBS, 4),
             "tokens_per_s": round(mm * steps / ev, 1),
             "gate_up_kernel": {"us": round(t_gu * 1e6, 2), "algorithmic_bytes": gub,
                                "frac": round(gub / t_gu / 1e9 / HBM_PEAK_GBS, 4)}}
        if cpu:
            e["cpu_baseline"] = cpu_chain_baseline(torch, copies, xm, mm, CPU_SAMPLE_S)
        res[f"config1_M{mm}"] = e
    return res


def prefill_setup(cl, torch, m, nn, kk, g, sdt, keep_host=False):
    """One config 2 prefill GEMM (bf16 x, MFMA-tiled weights, bf16 out)."""
    pk = cl.fill_bytes(torch.empty(nn * kk // 2, dtype=torch.uint8, device="cuda"), 2, 1)
    sc = cl.fill_scales(torch.empty(nn * (kk // g) * 2, dtype=torch.uint8, device="cuda"), 2, 2,
                        sdt)
    pt, st = cl.tile_weights(pk, sc, nn, kk, g)
    hostw = (pk.cpu().numpy(), sc.cpu().numpy()) if keep_host else None
    del pk, sc
    xb = cl.fill_normal(torch.empty(m * kk, dtype=torch.bfloat16, device="cuda"), 2, 3)
    yb = torch.empty(m * nn, dtype=torch.bfloat16, device="cuda")

    def pre(r):
        cl.gemm_int4_bf16(pt, st, xb, nn, kk, m, yb, group_size=g, scale_dtype=sdt,
                          tiling=cl.TILING_MFMA)
    return pre, xb, hostw


def config2(cl, torch, sdt, cpu):
    """Config 2 prefill GEMMs: TFLOP/s against the 2.5 PF bf16 dense peak;
    the CPU runs the crate's per-token GEMV loop (seq > 64) on 128 tokens."""
    import numpy as np

    import oracle as orc

    res = {}
    kk, g = 4096, 128
    for (m, nn) in PREFILL_SHAPES:
        pre, xb, hostw = prefill_setup(cl, torch, m, nn, kk, g, sdt, keep_host=cpu)
        pre(0)
        reps = 20
        wall, ev = graph_time(torch, pre, reps)
        t = ev / reps
        fl = 2.0 * m * nn * kk
        e = {"us_per_call": round(t * 1e6, 1), "TFLOP/s": round(fl / t / 1e12, 1),
             "mfma_frac": round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 4), "flops": fl}
        if cpu:
            ns = 128
            xs = orc.bf16_to_f32(xb[:ns * kk].view(torch.int16).cpu().numpy().view(np.uint16))
            ys = np.empty((ns, nn), np.float32)

            def run(r):
                orc.cpu_gemm(hostw[0], hostw[1], xs, nn, kk, ns, g, sdt, ys)
            cnt, dt = cpu_loop(run, CPU_SAMPLE_S)
            cfl = 2.0 * nn * kk * ns * cnt
            e["cpu_baseline"] = {"value": round(cfl / dt / 1e12, 4), "unit": "TFLOP/s",
                                 "cores": orc.cpu_threads(), "kind": "port",
                                 "sample": f"{cnt}x{ns} tokens, per-token loop, {dt:.1f}s"}
        res[f"config2_prefill_M{m}_N{nn}"] = e
        del pre, xb, hostw
        torch.cuda.empty_cache()
    return res


def make_experts_dev(cl, torch, E, h, i, g, sdt, seed):
    """E synthetic experts (crate layout, seeded): (crate blob, stride, tiled)."""
    per = cl.expert_bytes(h, i, g)
    stride = (per + 255) // 256 * 256
    crate = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    cl.fill_bytes(crate, seed, 7)
    for e in range(E):
        W = cl.ExpertWeights(crate[e * stride:e * stride + per], h, i, g, sdt)
        for j, s in enumerate((W.gate_scale_bits(), W.up_scale_bits(), W.down_scale_bits())):
            cl.fill_scales(s, seed, 100000 + 3 * e + j, sdt)
    ex = cl.MoEExperts.from_crate(crate, E, h, i, g, sdt, stride=stride, tiled=True)
    torch.cuda.synchronize()
    return crate, stride, ex


def marker(cl, torch):
    """A dispatch that brackets a profiled region: one streaming read of 64 KiB
    (its kernel runs nowhere else in the profile modes)."""
    if not _MARK:
        _MARK.append(torch.zeros(1 << 14, dtype=torch.float32, device="cuda"))
        _MARK.append(torch.zeros(1024, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    cl.stream_read(_MARK[0], _MARK[1])
    torch.cuda.synchronize()


_MARK = []


def calibrate(cl, torch):
    """Counter calibration after a profiled region: five 256 MiB streaming
    reads (true bytes read known) and five 256 MiB device copies (256 MiB
    read, 256 MiB written), each its own dispatch."""
    a = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    for _ in range(5):
        cl.stream_read(a, sink)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def bench_moe(cl, torch, E, h, i, g, k, T, layers, mode, scale, shared_inter, steps,
              zipf=None, nsets=64, cpu=False, cpu_tokens=4, replicas=1, profile_steps=0):
    """MoE layer(s) for T tokens; steps rotate through `nsets` routing-logit
    sets so that consecutive steps touch different experts, and through
    `replicas` copies of every layer's experts (so that no expert a step
    selects can still be in the Infinity Cache from a recent step).  With
    `cpu`, the runner's per-(token, slot) loop on the host over the first
    `cpu_tokens` tokens, through every layer, with the routing the GPU used.
    With `profile_steps`, no timing: that many eager steps between two
    marker dispatches, then the counter calibration; returns each step's
    algorithmic bytes."""
    import numpy as np

    import oracle as orc

    sdt = cl.SCALE_F16
    stacks, crates, shared_host = [], [], []
    for layer in range(layers * replicas):
        crate, stride, ex = make_experts_dev(cl, torch, E, h, i, g, sdt, 50 + layer)
        sh_host = None
        if shared_inter:
            per = cl.expert_bytes(h, shared_inter, g)
            f = cl.fill_bytes(torch.empty(per, dtype=torch.uint8, device="cuda"), 60 + layer, 1)
            W = cl.ExpertWeights(f, h, shared_inter, g, sdt)
            for j, s in enumerate((W.gate_scale_bits(), W.up_scale_bits(), W.down_scale_bits())):
                cl.fill_scales(s, 60 + layer, 10 + j, sdt)
            sh_host = f.cpu().numpy() if cpu else None
            ex = cl.MoEExperts(ex.blobs, E, h, i, g, sdt, cl.TILING_MFMA, ex.stride, W.tiled())
        stacks.append(ex)
        crates.append((crate, stride) if cpu and layer < layers else None)
        shared_host.append(sh_host)
        if not cpu:
            del crate
    logits = []
    for sidx in range(nsets):
        l = cl.fill_normal(torch.empty((T, E), dtype=torch.float32, device="cuda"), 70 + sidx, 1)
        if zipf is not None:
            perm = torch.randperm(E, generator=torch.Generator().manual_seed(1))
            l += (-zipf * torch.log1p(perm.float())).cuda()[None, :]
        logits.append(l)
    xb = cl.fill_normal(torch.empty((T, h), dtype=torch.bfloat16, device="cuda"), 80, 1)
    xs = [xb.float()] + [torch.empty((T, h), dtype=torch.float32, device="cuda") for _ in range(layers)]
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, k), dtype=torch.float32, device="cuda")
    # unique experts per step and layer (routing only depends on the logits)
    uniq = []
    for sidx in range(nsets):
        cl.moe_forward(stacks[0], xs[0], xs[1], top_k=k, logits=logits[sidx], mode=mode,
                       scale=scale, residual=xs[0], ids_out=ids)
        uniq.append(len(set(ids.cpu().flatten().tolist())))
    u_avg = sum(uniq) / len(uniq)

    def step(r):
        rep = (r % replicas) * layers
        for layer in range(layers):
            cl.moe_forward(stacks[rep + layer], xs[layer], xs[layer + 1], top_k=k,
                           logits=logits[(r + 7 * layer) % nsets], mode=mode, scale=scale,
                           residual=xs[layer])
    for r in range(5):
        step(r)
    per_expert = 3 * (i * h // 2 + i * (h // g) * 2)
    per_shared = 3 * (shared_inter * h // 2 + shared_inter * (h // g) * 2) if shared_inter else 0
    fixed = per_shared + T * h * 6 + T * E * 4 + T * k * 8
    if profile_steps:
        marker(cl, torch)
        for r in range(profile_steps):
            step(r)
        marker(cl, torch)
        calibrate(cl, torch)
        per_step = [sum(uniq[(r + 7 * layer) % nsets] * per_expert + fixed
                        for layer in range(layers)) for r in range(profile_steps)]
        del stacks, logits, crates, xs
        torch.cuda.empty_cache()
        return {"T": T, "layers": layers, "replicas": replicas, "steps": profile_steps,
                "algorithmic_bytes_per_step": per_step,
                "unique_experts": [uniq[(r + 7 * layer) % nsets] for r in range(profile_steps)
                                   for layer in range(layers)]}
    wall, ev = graph_time(torch, step, steps)
    t = ev / steps
    byts = layers * (u_avg * per_expert + fixed)
    flops = layers * 2.0 * T * (k + (1 if shared_inter else 0)) * 3 * h * i
    res = {"T": T, "layers": layers, "us_per_step": round(t * 1e6, 2),
           "wall_us_per_step": round(wall / steps * 1e6, 2),
           "tokens_per_s": round(T / t, 1), "GB/s": round(byts / t / 1e9, 1),
           "hbm_frac": round(byts / t / 1e9 / HBM_PEAK_GBS, 4),
           "TFLOP/s": round(flops / t / 1e12, 2),
           "mfma_frac": round(flops / t / 1e12 / BF16_PEAK_TFLOPS, 4),
           "unique_experts_avg": round(u_avg, 1), "algorithmic_bytes_per_step": int(byts),
           "replicas": replicas}
    if cpu:
        S = min(T, cpu_tokens)
        plan = []
        for layer in range(layers):
            cl.moe_forward(stacks[layer], xs[0], xs[1], top_k=k, logits=logits[(7 * layer) % nsets],
                           mode=mode, scale=scale, residual=xs[0], ids_out=ids, weights_out=wts)
            li = ids.cpu().numpy()[:S].astype(np.int64)
            lw = wts.cpu().numpy()[:S].copy()
            crate, stride = crates[layer]
            used = sorted({int(e) for e in li.ravel()})
            blob = np.concatenate([crate[e * stride:(e + 1) * stride].cpu().numpy() for e in used])
            remap = np.vectorize({e: j for j, e in enumerate(used)}.get)(li).astype(np.int64)
            plan.append((blob, len(used), stride, remap, lw, shared_host[layer]))
        x0 = xb[:S].float().cpu().numpy()

        def run(r):
            xr = x0
            for blob, ne, stride, rid, lw, shh in plan:
                xr = orc.cpu_moe_layer(xr, blob, ne, shh, shared_inter, h, i, g, sdt, rid, lw,
                                       0.0, stride=stride)
        cnt, dt = cpu_loop(run, CPU_SAMPLE_S)
        res["cpu_baseline"] = {"value": round(S * cnt / dt, 2), "unit": "tokens/s",
                               "cores": orc.cpu_threads(), "kind": "port",
                               "sample": f"{cnt}x{S} tokens x {layers} layers, {dt:.1f}s"}
    del stacks, logits, crates, xs
    torch.cuda.empty_cache()
    return res


def f_rows(cl, torch, sdt, copies):
    """f1 / f3 paths at one token: the K2.6 shell projections, the
    activation-sparse expert at tau 0.1 / 0.3, the AXPY down."""
    import ctypes as C

    res = {}
    h, i, g = copies.h, copies.i, copies.g
    # the K2.6 shell projections at one token (q_a, q_b, kv_a, kv_b, o_proj,
    # router; shell_int4.rs:404-660) in the crate's format (G = 32, bf16
    # scales): six one-token GEMVs per step over rotating weight copies
    shapes = [(1536, 7168), (12288, 1536), (576, 7168), (16384, 512), (7168, 8192), (384, 7168)]
    gs, sbf = 32, cl.SCALE_BF16
    per = sum(nn * kk // 2 + nn * (kk // gs) * 2 for nn, kk in shapes)
    ncs = math.ceil(2 * MALL_BYTES / per) + 1
    SH = []
    for c in range(ncs):
        mats = []
        for j, (nn, kk) in enumerate(shapes):
            p = cl.fill_bytes(torch.empty(nn * kk // 2, dtype=torch.uint8, device="cuda"), 1, 400 + 8 * c + j)
            sc = cl.fill_scales(torch.empty(nn * (kk // gs) * 2, dtype=torch.uint8, device="cuda"),
                                1, 500 + 8 * c + j, sbf)
            mats.append(cl.tile_weights(p, sc, nn, kk, gs))
            del p, sc
        SH.append(mats)
    xs_ = {kk: cl.fill_normal(torch.empty(kk, dtype=torch.float32, device="cuda"), 1, kk)
           for _, kk in shapes}
    ys_ = [torch.empty(nn, dtype=torch.float32, device="cuda") for nn, _ in shapes]

    def shell(r):
        for j, (nn, kk) in enumerate(shapes):
            pt, st = SH[r % ncs][j]
            cl.dequant_gemv_int4(pt, st, xs_[kk], nn, kk, ys_[j], group_size=gs, scale_dtype=sbf,
                                 tiling=cl.TILING_MFMA)
    for r in range(5):
        shell(r)
    steps = 200
    _, ev = graph_time(torch, shell, steps)
    t = ev / steps
    b = per + sum(kk * 4 + nn * 4 for nn, kk in shapes)
    res["shell_projections_M1"] = {"us_per_step": round(t * 1e6, 2), "GB/s": round(b / t / 1e9, 1),
                                   "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                                   "bytes_per_step": b, "copies": ncs}
    del SH
    # The activation-sparse FFN at one token, tau 0.1 / 0.3, in the layout made
    # for it (TILING_MFMA_UP_ROWS: gate and down tiled, up rows contiguous, so
    # only the active up rows are read); the AXPY form also over the all-tiled
    # layout (up read in 16-byte pieces of its tiles), for comparison.  One
    # crate-layout up per weight copy (synthetic, seeded), so the up rows
    # rotate with the rest.
    nc = len(copies.w)
    mat = i * h // 2 + i * (h // g) * 2
    UPS = [(cl.fill_bytes(torch.empty(i * h // 2, dtype=torch.uint8, device="cuda"), 3, 800 + c),
            cl.fill_scales(torch.empty(i * (h // g) * 2, dtype=torch.uint8, device="cuda"), 3,
                           900 + c, sdt)) for c in range(nc)]
    xs1 = cl.fill_normal(torch.empty(h, dtype=torch.bfloat16, device="cuda"), 0, 23)
    os1 = torch.empty(h, dtype=torch.bfloat16, device="cuda")
    for tau in (0.1, 0.3):
        ex = [cl._lib.Expert(W.gate_packed_bytes().data_ptr(), W.gate_scale_bits().data_ptr(),
                             UPS[c][0].data_ptr(), UPS[c][1].data_ptr(),
                             W.down_packed_bytes().data_ptr(), W.down_scale_bits().data_ptr(),
                             cl.TILING_MFMA_UP_ROWS) for c, W in enumerate(copies.w)]
        W0 = copies.w[0]
        fr = cl.expert_forward_sparse(xs1.view(torch.int16), W0.gate_packed_bytes(),
                                      W0.gate_scale_bits(), UPS[0][0], UPS[0][1],
                                      W0.down_packed_bytes(), W0.down_scale_bits(),
                                      os1.view(torch.int16), tau, group_size=g, scale_dtype=sdt,
                                      tiling=cl.TILING_MFMA_UP_ROWS)

        def sparse(r, tau=tau):
            cl.check("cascadia_int4_expert_forward_sparse", cl.lib().cascadia_int4_expert_forward_sparse(
                h, i, g, sdt, C.byref(ex[r % nc]), xs1.data_ptr(), 1, tau, None, os1.data_ptr(),
                None, None, torch.cuda.current_stream().cuda_stream))
        for r in range(10):
            sparse(r)
        steps = 200
        _, ev = graph_time(torch, sparse, steps)
        t = ev / steps
        na = int(round(fr * i))
        # the crate's reads: gate and down in full, the active up rows
        b = 2 * mat + na * (h // 2 + (h // g) * 2) + h * 2 * 2
        res[f"sparse_expert_M1_tau{tau}"] = {"us_per_call": round(t * 1e6, 2),
                                             "active_frac": round(fr, 4),
                                             "GB/s": round(b / t / 1e9, 1),
                                             "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                                             "layout": "mfma_up_rows"}
    # the composed AXPY-form sparse FFN (ffn_sparsity.rs:638-740): f32 in /
    # out, gate + mask + rows-subset up + AXPY down over config 1's
    # transposed down
    src = cl.ExpertWeights(copies.crate[0], h, i, g, sdt)
    ptc, stc = cl.transpose_requantize_down(src.down_packed_bytes(), src.down_scale_bits(), h, i,
                                            group_size=g, scale_dtype=sdt)
    # one transposed down per weight copy, so that the active rows rotate too
    # (synthetic codes and bf16 scales of the transposed shape; the first is
    # copy 0's true transpose)
    PTS = [(ptc, stc)] + [
        (cl.fill_bytes(torch.empty(i * h // 2, dtype=torch.uint8, device="cuda"), 2, 600 + c),
         cl.fill_scales(torch.empty(i * (h // 32) * 2, dtype=torch.uint8, device="cuda"), 2,
                        700 + c, cl.SCALE_BF16))
        for c in range(1, nc)]
    xf1 = xs1.float()
    of1 = torch.empty(h, dtype=torch.float32, device="cuda")
    wsx = torch.empty(cl.ffn_sparse_axpy_workspace_bytes(h, i, 1, g), dtype=torch.uint8,
                      device="cuda")
    for tau, lay in ((0.1, "up_rows"), (0.3, "up_rows"), (0.3, "tiled")):
        W0 = copies.w[0]
        rows = lay == "up_rows"
        til = cl.TILING_MFMA_UP_ROWS if rows else cl.TILING_MFMA
        up0 = UPS[0] if rows else (W0.up_packed_bytes(), W0.up_scale_bits())
        fr = cl.ffn_forward_sparse_axpy_f32(xf1, h, i, W0.gate_packed_bytes(), W0.gate_scale_bits(),
                                            *up0, ptc, stc, of1, tau, group_size=g,
                                            scale_dtype=sdt, workspace=wsx, tiling=til)
        exa = [cl._lib.Expert(W.gate_packed_bytes().data_ptr(), W.gate_scale_bits().data_ptr(),
                              (UPS[c][0] if rows else W.up_packed_bytes()).data_ptr(),
                              (UPS[c][1] if rows else W.up_scale_bits()).data_ptr(),
                              PTS[c][0].data_ptr(), PTS[c][1].data_ptr(), til)
               for c, W in enumerate(copies.w)]

        def axffn(r, tau=tau, exa=exa):
            cl.check("cascadia_int4_ffn_forward_sparse_axpy_f32",
                     cl.lib().cascadia_int4_ffn_forward_sparse_axpy_f32(
                         h, i, g, sdt, C.byref(exa[r % nc]), xf1.data_ptr(), 1, tau, None,
                         of1.data_ptr(), None, wsx.data_ptr(),
                         torch.cuda.current_stream().cuda_stream))
        for r in range(10):
            axffn(r)
        steps = 200
        _, ev = graph_time(torch, axffn, steps)
        t = ev / steps
        na = int(round(fr * i))
        # algorithmic: the crate's reads (gate, the active up and transposed-down rows)
        b = mat + na * (h // 2 + (h // g) * 2) + na * (h // 2 + (h // 32) * 2) + h * 4 * 2
        key = f"sparse_axpy_ffn_M1_tau{tau}" + ("" if rows else "_tiled_up")
        res[key] = {"us_per_call": round(t * 1e6, 2), "active_frac": round(fr, 4),
                    "GB/s": round(b / t / 1e9, 1),
                    "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                    "layout": "mfma_up_rows" if rows else "mfma"}
    del ptc, stc, wsx, PTS, UPS
    # the AXPY form of the sparse down (ffn_axpy.rs:82-160): config 1's down
    # transposed to [inter, hidden], 13.4 % of the rows active (what tau 0.3
    # selects above), over rotating copies larger than 2x the Infinity Cache
    I1, H1 = i, h
    ptb, stb = I1 * H1 // 2, I1 * (H1 // 32) * 2
    nca = math.ceil(2 * MALL_BYTES / (ptb + stb)) + 1
    AX = []
    for c in range(nca):
        p = cl.fill_bytes(torch.empty(H1 * I1 // 2, dtype=torch.uint8, device="cuda"), 2, 600 + c)
        sc = cl.fill_scales(torch.empty(H1 * (I1 // 32) * 2, dtype=torch.uint8, device="cuda"),
                            2, 700 + c, cl.SCALE_BF16)
        AX.append(cl.transpose_requantize_down(p, sc, H1, I1))
        del p, sc
    n_act = int(round(0.1344 * I1))
    act = torch.sort(torch.randperm(I1, device="cuda")[:n_act])[0].to(torch.int32)
    sca = cl.fill_normal(torch.empty(I1, dtype=torch.float32, device="cuda"), 2, 11)
    ya = torch.zeros(H1, dtype=torch.float32, device="cuda")
    wsa = torch.empty(cl.lib().cascadia_int4_axpy_workspace_bytes(H1, n_act), dtype=torch.uint8,
                      device="cuda")

    def axpy(r):
        pt_, st_ = AX[r % nca]
        cl.dequant_axpy_int4_active(pt_, st_, sca, act, I1, H1, ya, workspace=wsa)
    for r in range(5):
        axpy(r)
    steps = 200
    _, ev = graph_time(torch, axpy, steps)
    t = ev / steps
    b = n_act * (H1 // 2 + (H1 // 32) * 2 + 8) + 2 * H1 * 4
    res["axpy_down_config1_13pct"] = {"us_per_call": round(t * 1e6, 2), "active_rows": n_act,
                                      "GB/s": round(b / t / 1e9, 1),
                                      "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                                      "copies": nca}
    del AX
    return res


def all_configs(cl, torch, sdt, copies, cpu):
    ex = {"hbm_ceiling": hbm_ceiling(cl, torch)}
    if cpu:
        ex["cpu_host"] = host_cpu()
    ex["config0_gemv"] = config0(cl, torch, sdt, cpu)
    ex.update(config1_batches(cl, torch, sdt, copies, cpu))
    ex.update(config2(cl, torch, sdt, cpu))
    for T in (1, 32, 256):
        # one token's 8 experts (58 MB) fit the Infinity Cache a few steps over:
        # eight copies of the layer rotate, so no step finds its experts there
        ex[f"config3_moe_T{T}"] = bench_moe(
            cl, torch, 256, 3072, 1536, 128, 8, T, 1, cl.ROUTE_SOFTMAX_TOPK, 1.0, 0,
            200 if T < 256 else 40, cpu=cpu, cpu_tokens=8, replicas=8 if T == 1 else 1)
    for T in (1, 8, 64, 1024):
        ex[f"config4_moe_T{T}"] = bench_moe(
            cl, torch, 384, 7168, 2048, 32, 8, T, 4, cl.ROUTE_SIGMOID_BIAS, 2.827, 2048,
            50 if T < 64 else (20 if T == 64 else 5), zipf=1.1, nsets=16 if T == 1024 else 64,
            cpu=cpu, cpu_tokens=4)
    ex.update(f_rows(cl, torch, sdt, copies))
    try:
        with open(TRAFFIC_ALL) as f:
            tr = json.load(f)
        for key, e in ex.items():
            if key in tr and isinstance(e, dict):
                e["traffic_ratio"] = tr[key]["ratio"]  # HBM bytes / algorithmic, counters
    except (OSError, ValueError, KeyError):
        pass
    return ex


def summary(line):
    """The figures of every config in a few hundred characters, for the end of
    the JSON line (a reader that keeps only the tail of the output still gets
    them): [µs, fraction of roofline] per workload -- HBM for decode / MoE, bf16
    MFMA for prefill; MoE entries [µs per step, HBM frac, MFMA frac, tokens/s]."""
    ex = line.get("extra", {})
    out = {"c1_M1": [round(line["ms_per_step"] * 1e3, 2), line["roofline"]["frac"]]}
    c = ex.get("config0_gemv")
    if c:
        out["c0"] = [c["us_per_call"], c["hbm_frac"]]
    for m in (4, 16):
        c = ex.get(f"config1_M{m}")
        if c:
            out[f"c1_M{m}"] = [c["us_per_chain"], c["hbm_frac"]]
    for (pm, pn) in PREFILL_SHAPES:
        c = ex.get(f"config2_prefill_M{pm}_N{pn}")
        if c:
            out[f"c2_{pm}x{pn}"] = [c["us_per_call"], c["mfma_frac"]]
    for cfg, ts in ((3, (1, 32, 256)), (4, (1, 8, 64, 1024))):
        for T in ts:
            c = ex.get(f"config{cfg}_moe_T{T}")
            if c:
                out[f"c{cfg}_T{T}"] = [c["us_per_step"], c["hbm_frac"], c["mfma_frac"],
                                       c["tokens_per_s"]]
    c = ex.get("sparse_axpy_ffn_M1_tau0.3")
    if c:
        out["axpy_tau0.3"] = [c["us_per_call"], round(c["us_per_call"] / out["c1_M1"][0], 3)]
    c = ex.get("hbm_ceiling")
    if c:
        out["read_ceiling_GBps"] = c.get("read_60MiB_GBps")
        rf = c.get("read_us_by_bytes")
        if rf:
            # time of a plain read of the same bytes / the workload's time
            out["vs_same_bytes_read"] = {
                "c0": round(rf["config0"] / out["c0"][0], 3) if "c0" in out else None,
                "c1_M1_chain": round((rf["config1_gate_up"] + rf["config1_down"]) /
                                     out["c1_M1"][0], 3),
                "floor_64KiB_us": rf["64KiB"]}
    return out


# ---------------------------------------------------------------------------
# main
# ---------------------------------------------------------------------------

def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; --gpus N > 1 is not supported "
                                   "(value is one GPU's throughput; the path is not sharded)"}))
        sys.exit(2)
    import torch

    import cascadia_amd as cl

    sdt = cl.SCALE_F16
    if args.profile_gemv:
        n = k = 4096
        g = 128
        nb, nsb = n * k // 2, n * (k // g) * 2
        ncp = math.ceil(2 * MALL_BYTES / (nb + nsb)) + 1
        PS = []
        for c in range(ncp):
            p = cl.fill_bytes(torch.empty(nb, dtype=torch.uint8, device="cuda"), 0, 200 + c)
            s = cl.fill_scales(torch.empty(nsb, dtype=torch.uint8, device="cuda"), 0, 300 + c, sdt)
            PS.append(cl.tile_weights(p, s, n, k, g))
        x = cl.fill_normal(torch.empty(k, dtype=torch.float32, device="cuda"), 0, 13)
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        for r in range(20):
            pt, st = PS[r % ncp]
            cl.dequant_gemv_int4(pt, st, x, n, k, y, group_size=g, scale_dtype=sdt,
                                 tiling=cl.TILING_MFMA)
        marker(cl, torch)  # the 200 launches between the markers are the profiled ones
        for r in range(200):
            pt, st = PS[r % ncp]
            cl.dequant_gemv_int4(pt, st, x, n, k, y, group_size=g, scale_dtype=sdt,
                                 tiling=cl.TILING_MFMA)
        marker(cl, torch)
        calibrate(cl, torch)
        print(json.dumps({"profile": "gemv", "launches": 200, "copies": ncp,
                          "algorithmic_bytes": nb + nsb + k * 4 + n * 4}), flush=True)
        return
    if args.profile_prefill:
        for (pm, pn) in PREFILL_SHAPES:
            pre, _, _ = prefill_setup(cl, torch, pm, pn, 4096, 128, sdt)
            for r in range(5):
                pre(r)
            torch.cuda.synchronize()
            del pre
        print(json.dumps({"profile": "prefill", "shapes": PREFILL_SHAPES, "launches": 5}),
              flush=True)
        return
    if args.profile_batches:
        # the config 1 chain at M = 4 and 16 (the skinny kernels, the down's K
        # split and its reduce), 40 eager calls each over rotating copies
        h, i, g = 4096, 14336, 128
        copies = Copies(cl, torch, h, i, g, sdt, chain_copies(cl, h, i, g), keep_crate=0)
        for mm in (4, 16):
            xm = cl.fill_normal(torch.empty((mm, h), dtype=torch.bfloat16, device="cuda"), 0, 22)
            om = torch.empty((mm, h), dtype=torch.bfloat16, device="cuda")
            fn = chain_fn(cl, copies, xm, om, sdt)
            for k in range(40):
                fn(k)
        torch.cuda.synchronize()
        print(json.dumps({"profile": "config1_batches", "M": [4, 16], "launches": 40,
                          "copies": len(copies.w)}), flush=True)
        return
    if args.profile_sparse:
        # 50 calls each of the GEMV form (expert_forward_sparse) and the AXPY
        # form (ffn_forward_sparse_axpy_f32) at tau 0.3 on the layout the
        # default run times (gate and down tiled, up rows contiguous), weight
        # copies rotating past the Infinity Cache
        import ctypes as C

        h, i, g = 4096, 14336, 128
        nc = chain_copies(cl, h, i, g)
        copies = Copies(cl, torch, h, i, g, sdt, nc, keep_crate=1)
        UPS = [(cl.fill_bytes(torch.empty(i * h // 2, dtype=torch.uint8, device="cuda"), 3, 800 + c),
                cl.fill_scales(torch.empty(i * (h // g) * 2, dtype=torch.uint8, device="cuda"), 3,
                               900 + c, sdt)) for c in range(nc)]
        xs1 = cl.fill_normal(torch.empty(h, dtype=torch.bfloat16, device="cuda"), 0, 23)
        os1 = torch.empty(h, dtype=torch.bfloat16, device="cuda")
        st = torch.cuda.current_stream().cuda_stream
        ex = [cl._lib.Expert(W.gate_packed_bytes().data_ptr(), W.gate_scale_bits().data_ptr(),
                             UPS[c][0].data_ptr(), UPS[c][1].data_ptr(),
                             W.down_packed_bytes().data_ptr(), W.down_scale_bits().data_ptr(),
                             cl.TILING_MFMA_UP_ROWS) for c, W in enumerate(copies.w)]
        for r in range(50):
            cl.check("cascadia_int4_expert_forward_sparse", cl.lib().cascadia_int4_expert_forward_sparse(
                h, i, g, sdt, C.byref(ex[r % nc]), xs1.data_ptr(), 1, 0.3, None, os1.data_ptr(),
                None, None, st))
        src = cl.ExpertWeights(copies.crate[0], h, i, g, sdt)
        pts = [cl.transpose_requantize_down(src.down_packed_bytes(), src.down_scale_bits(), h, i,
                                            group_size=g, scale_dtype=sdt)]
        pts += [(cl.fill_bytes(torch.empty(i * h // 2, dtype=torch.uint8, device="cuda"), 2, 600 + c),
                 cl.fill_scales(torch.empty(i * (h // 32) * 2, dtype=torch.uint8, device="cuda"), 2,
                                700 + c, cl.SCALE_BF16)) for c in range(1, nc)]
        xf1, of1 = xs1.float(), torch.empty(h, dtype=torch.float32, device="cuda")
        ws = torch.empty(cl.ffn_sparse_axpy_workspace_bytes(h, i, 1, g), dtype=torch.uint8,
                         device="cuda")
        exa = [cl._lib.Expert(W.gate_packed_bytes().data_ptr(), W.gate_scale_bits().data_ptr(),
                              UPS[c][0].data_ptr(), UPS[c][1].data_ptr(), pts[c][0].data_ptr(),
                              pts[c][1].data_ptr(), cl.TILING_MFMA_UP_ROWS)
               for c, W in enumerate(copies.w)]
        for r in range(50):
            cl.check("cascadia_int4_ffn_forward_sparse_axpy_f32",
                     cl.lib().cascadia_int4_ffn_forward_sparse_axpy_f32(
                         h, i, g, sdt, C.byref(exa[r % nc]), xf1.data_ptr(), 1, 0.3, None,
                         of1.data_ptr(), None, ws.data_ptr(), st))
        torch.cuda.synchronize()
        print(json.dumps({"profile": "sparse_expert+sparse_axpy_ffn", "tau": 0.3,
                          "layout": "mfma_up_rows", "launches": 50, "copies": nc}), flush=True)
        return
    if args.profile_moe:
        # eager steps between two marker dispatches (then the counter
        # calibration), with the default bench's weight rotation; prints each
        # step's algorithmic bytes
        T = args.moe_tokens
        out = {"profile": "moe"}
        if args.moe_config in (0, 3):
            out[f"config3_T{T}"] = bench_moe(
                cl, torch, 256, 3072, 1536, 128, 8, T, 1, cl.ROUTE_SOFTMAX_TOPK, 1.0, 0, 0,
                nsets=16, replicas=8 if T == 1 else 1, profile_steps=16 if T < 256 else 4)
        if args.moe_config in (0, 4):
            out[f"config4_T{T}"] = bench_moe(
                cl, torch, 384, 7168, 2048, 32, 8, T, 4, cl.ROUTE_SIGMOID_BIAS, 2.827, 2048, 0,
                zipf=1.1, nsets=16, profile_steps=8 if T < 256 else 2)
        print(json.dumps(out), flush=True)
        return
    h, i, g, m = 4096, 14336, 128, args.m
    ncopies = chain_copies(cl, h, i, g)
    copies = Copies(cl, torch, h, i, g, sdt, ncopies)
    x = cl.fill_normal(torch.empty((m, h), dtype=torch.bfloat16, device="cuda"), 0, 22)
    out = torch.empty((m, h), dtype=torch.bfloat16, device="cuda")
    inter = torch.empty((m, i), dtype=torch.float32, device="cuda")
    fn = chain_fn(cl, copies, x, out, sdt)
    gu = gate_up_fn(cl, copies, x, inter, sdt)

    if args.profile:
        for k in range(args.steps):
            fn(k)
        for k in range(args.steps):
            gu(k)
        a = torch.zeros(64 << 20, dtype=torch.float32, device="cuda")  # 256 MiB
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)  # calibration: reads 256 MiB, writes 256 MiB per launch
        torch.cuda.synchronize()
        print(json.dumps({"profile": "done", "steps": args.steps, "M": m}), flush=True)
        return

    for k in range(args.warmup):
        fn(k)
    torch.cuda.synchronize()
    wall, ev = graph_time(torch, fn, args.steps)
    value = ffn_bytes(h, i, g, m) * args.steps / wall / 1e9

    for k in range(args.warmup):
        gu(k)
    _, ev_gu = graph_time(torch, gu, args.steps)
    t_gu = ev_gu / args.steps
    gu_bytes = gate_up_bytes(h, i, g, m)
    achieved = gu_bytes / t_gu / 1e9

    line = {
        "metric": "INT4 GEMV/MoE-layer achieved HBM GB/s + tokens/s; prefill GEMM TFLOP/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4*bf16->f32 (f32 accumulation; the SwiGLU intermediate as bf16 hi+lo "
                 "planes, about 17 significant bits)",
        "data": "synthetic",
        "config": {"workload": "config1_llama3_8b_decode_ffn_chain", "M": m, "hidden": h,
                   "inter": i, "group": g, "scales": "fp16", "weight_copies": ncopies,
                   "weight_layout": "mfma_tiled, converted once from the crate layout",
                   "timing": "one HIP-graph replay of the K steps",
                   "tokens_per_s": round(m * args.steps / wall, 1),
                   "event_ms_per_step": round(ev / args.steps * 1e3, 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(m),
                     "kernel": "gemv_kernel<2,0,4,1> fused gate/up",
                     "algorithmic_bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(t_gu * 1e6, 3)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_chain_baseline(torch, copies, x, m, args.cpu_seconds)
    if not args.headline_only:
        line["extra"] = all_configs(cl, torch, sdt, copies, not args.no_cpu)
        ceil = line["extra"]["hbm_ceiling"].get("read_60MiB_GBps")
        if ceil:
            line["roofline"]["frac_of_read_ceiling"] = round(achieved / ceil, 4)
        line["summary"] = summary(line)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
