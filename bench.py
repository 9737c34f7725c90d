"""Benchmark of the INT4 weight-only matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--m 1] [--no-cpu] [--extra]

Headline: the Llama-3-8B-shaped decode FFN chain,
gate/up 14336x4096 + down 4096x14336, INT4 group 128 with fp16 scales, bf16
activations, M tokens.  One step = one expert_forward chain (two kernels:
fused gate/up/SiLU*up, then down with the bf16 output rounding) over one
batch of M tokens, with the weights rotated through enough distinct copies
(> 2 x 256 MB Infinity Cache) that every step streams its weights from HBM.

`value` = algorithmic bytes per step (3 x (packed + scales) + M*H*2*2, the
weights read once plus activations in and out) x steps / wall time of the
timed region -> GB/s.  The roofline object covers the dominant kernel (the
fused gate/up kernel), timed with HIP events on the stream it runs on.  The
CPU baseline is the oracle's AVX-512 port of the crate's kernels on the host
cores, on a bounded sample of the same workload (same bytes, copied back).
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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--m", type=int, default=1, help="decode batch (tokens) of the headline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--extra", action="store_true", help="also time configs 0 and 2, M=4/16")
    return ap.parse_args()


def ffn_bytes(h, i, g, m):
    w = 3 * (i * h // 2 + i * (h // g) * 2)
    return w + m * h * 2 * 2


def gate_up_bytes(h, i, g, m):
    return 2 * (i * h // 2 + i * (h // g) * 2) + m * h * 2 + m * i * 4


class Copies:
    """`n` distinct synthetic experts resident in HBM."""

    def __init__(self, cl, torch, h, i, g, sdt, n, seed=1):
        self.h, self.i, self.g = h, i, g
        nb = cl.expert_bytes(h, i, g)
        self.flat = []
        self.w = []
        for c in range(n):
            f = torch.empty(nb, dtype=torch.uint8, device="cuda")
            cl.fill_bytes(f, seed, 100 + c)
            W = cl.ExpertWeights(f, h, i, g, sdt)
            for j, s in enumerate((W.gate_scale_bits(), W.up_scale_bits(), W.down_scale_bits())):
                cl.fill_scales(s, seed, 1000 + 10 * c + j, sdt)
            self.flat.append(f)
            self.w.append(W)
        torch.cuda.synchronize()


def time_chain(cl, torch, copies, x, out, steps, warmup, sdt):
    nc = len(copies.w)
    for s in range(warmup):
        cl.expert_forward(x, *copies.w[s % nc].slices(), out, group_size=copies.g, scale_dtype=sdt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for s in range(steps):
        cl.expert_forward(x, *copies.w[s % nc].slices(), out, group_size=copies.g, scale_dtype=sdt)
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0), e0.elapsed_time(e1) / 1e3


def time_gate_up(cl, torch, copies, x, inter, steps, warmup, sdt):
    """Average duration of the fused gate/up kernel alone (HIP events on the
    current stream, which is the stream the kernel is launched on)."""
    nc = len(copies.w)
    for s in range(warmup):
        W = copies.w[s % nc]
        cl.gate_up_silu(x, W.gate_packed_bytes(), W.gate_scale_bits(), W.up_packed_bytes(),
                        W.up_scale_bits(), inter, group_size=copies.g, scale_dtype=sdt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for s in range(steps):
        W = copies.w[s % nc]
        cl.gate_up_silu(x, W.gate_packed_bytes(), W.gate_scale_bits(), W.up_packed_bytes(),
                        W.up_scale_bits(), inter, group_size=copies.g, scale_dtype=sdt)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / steps


def cpu_baseline(cl, torch, copies, x, m, seconds):
    import numpy as np

    import oracle as orc

    h, i, g = copies.h, copies.i, copies.g
    host = [c.cpu().numpy() for c in copies.flat[:3]]
    xb = x.view(torch.int16).cpu().numpy().view(np.uint16)
    out = np.empty((m, h), np.uint16)
    orc.cpu_expert_forward(xb, m, host[0], h, i, g, orc.SCALE_F16, out)  # warm-up
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        orc.cpu_expert_forward(xb, m, host[n % len(host)], h, i, g, orc.SCALE_F16, out)
        n += 1
    dt = time.perf_counter() - t0
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


def extra_measurements(cl, torch, args, sdt):
    """Secondary numbers (not the headline): config 0 GEMV, M=4/16 chains,
    prefill GEMM."""
    import numpy as np

    res = {}
    # config 0: 4096x4096 GEMV, f32 x, rotate > 2x MALL of weight copies
    n = k = 4096
    g = 128
    nb = n * k // 2
    nsb = n * (k // g) * 2
    ncp = math.ceil(2 * MALL_BYTES / (nb + nsb)) + 1
    P = [cl.fill_bytes(torch.empty(nb, dtype=torch.uint8, device="cuda"), 0, 200 + c) for c in range(ncp)]
    S = [cl.fill_scales(torch.empty(nsb, dtype=torch.uint8, device="cuda"), 0, 300 + c, sdt) for c in range(ncp)]
    x = cl.fill_normal(torch.empty(k, dtype=torch.float32, device="cuda"), 0, 13)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    for s in range(20):
        cl.dequant_gemv_int4(P[s % ncp], S[s % ncp], x, n, k, y, group_size=g, scale_dtype=sdt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    steps = 2000
    e0.record()
    for s in range(steps):
        cl.dequant_gemv_int4(P[s % ncp], S[s % ncp], x, n, k, y, group_size=g, scale_dtype=sdt)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / steps
    b = nb + nsb + k * 4 + n * 4
    res["config0_gemv"] = {"us_per_call": round(t * 1e6, 3), "GB/s": round(b / t / 1e9, 1),
                           "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4), "copies": ncp}
    del P, S
    # config 2: prefill GEMM M=512, N=4096, K=4096 (bf16 in/out)
    for (m, nn) in [(512, 4096), (2048, 14336)]:
        kk = 4096
        pk = cl.fill_bytes(torch.empty(nn * kk // 2, dtype=torch.uint8, device="cuda"), 2, 1)
        sc = cl.fill_scales(torch.empty(nn * (kk // g) * 2, dtype=torch.uint8, device="cuda"), 2, 2, sdt)
        xb = cl.fill_normal(torch.empty(m * kk, dtype=torch.bfloat16, device="cuda"), 2, 3)
        yb = torch.empty(m * nn, dtype=torch.bfloat16, device="cuda")
        for _ in range(3):
            cl.gemm_int4_bf16(pk, sc, xb, nn, kk, m, yb, group_size=g, scale_dtype=sdt)
        torch.cuda.synchronize()
        reps = 10
        e0.record()
        for _ in range(reps):
            cl.gemm_int4_bf16(pk, sc, xb, nn, kk, m, yb, group_size=g, scale_dtype=sdt)
        e1.record()
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) / 1e3 / reps
        tf = 2.0 * m * nn * kk / t / 1e12
        res[f"config2_prefill_M{m}_N{nn}"] = {"us_per_call": round(t * 1e6, 1), "TFLOP/s": round(tf, 1),
                                              "mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)}
        del pk, sc, xb, yb
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU; --gpus N > 1 is not supported "
                                   "(the path is single-GPU; sharding is documented in DESIGN.md)"}))
        sys.exit(2)
    import torch

    import cascadia_amd as cl

    sdt = cl.SCALE_F16
    h, i, g, m = 4096, 14336, 128, args.m
    per_copy = cl.expert_bytes(h, i, g)
    ncopies = math.ceil(2 * MALL_BYTES / per_copy) + 1
    copies = Copies(cl, torch, h, i, g, sdt, ncopies)
    x = cl.fill_normal(torch.empty((m, h), dtype=torch.bfloat16, device="cuda"), 0, 22)
    out = torch.empty((m, h), dtype=torch.bfloat16, device="cuda")

    wall, ev = time_chain(cl, torch, copies, x, out, args.steps, args.warmup, sdt)
    step_bytes = ffn_bytes(h, i, g, m)
    value = step_bytes * args.steps / wall / 1e9

    inter = torch.empty((m, i), dtype=torch.float32, device="cuda")
    t_gu = time_gate_up(cl, torch, copies, x, inter, args.steps, args.warmup, sdt)
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
        "dtype": "int4*bf16->f32",
        "data": "synthetic",
        "config": {"workload": "config1_llama3_8b_decode_ffn_chain", "M": m, "hidden": h,
                   "inter": i, "group": g, "scales": "fp16", "weight_copies": ncopies,
                   "tokens_per_s": round(m * args.steps / wall, 1),
                   "event_ms_per_step": round(ev / args.steps * 1e3, 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "skinny_kernel (fused gate/up + SiLU*up)",
                     "algorithmic_bytes_per_launch": gu_bytes,
                     "avg_launch_us": round(t_gu * 1e6, 3)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cl, torch, copies, x, m, args.cpu_seconds)
    if args.extra:
        for mm in (4, 16):
            xm = cl.fill_normal(torch.empty((mm, h), dtype=torch.bfloat16, device="cuda"), 0, 22)
            om = torch.empty((mm, h), dtype=torch.bfloat16, device="cuda")
            w2, _ = time_chain(cl, torch, copies, xm, om, args.steps, args.warmup, sdt)
            line.setdefault("extra", {})[f"config1_M{mm}"] = {
                "GB/s": round(ffn_bytes(h, i, g, mm) * args.steps / w2 / 1e9, 1),
                "us_per_chain": round(w2 / args.steps * 1e6, 2),
                "tokens_per_s": round(mm * args.steps / w2, 1)}
        line.setdefault("extra", {}).update(extra_measurements(cl, torch, args, sdt))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
