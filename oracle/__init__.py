"""ctypes wrapper over the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py -- as the checker or the timed CPU reference,
never as a product path.  The product library (cascadia_amd) never imports
this package.

Each wrapper takes/returns numpy arrays and follows the C restatement in
int4_oracle.c, which cites the reference crate file:line it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

SCALE_BF16 = 0
SCALE_F16 = 1
ORDER_SCALAR = 0
ORDER_AVX512 = 1

_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, no GPU needed)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _declare(L):
    vp, sz, i32, f32, u64, f64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint64, C.c_double
    sig = {
        "or_bf16_to_f32": (f32, [C.c_uint16]),
        "or_f32_to_bf16": (C.c_uint16, [f32]),
        "or_f16_to_f32": (f32, [C.c_uint16]),
        "or_f32_to_f16": (C.c_uint16, [f32]),
        "or_expert_bytes": (sz, [sz, sz, sz]),
        "or_dequant": (None, [vp, vp, sz, sz, sz, i32, vp]),
        "or_gemv": (None, [vp, vp, vp, sz, sz, sz, i32, i32, vp]),
        "or_gemm_multi": (None, [vp, vp, vp, sz, sz, sz, sz, i32, i32, vp]),
        "or_gemv_rows_subset": (None, [vp, vp, vp, sz, sz, sz, i32, i32, vp, sz, vp]),
        "or_expert_forward": (None, [vp, sz, sz, sz, i32, i32, vp, vp]),
        "or_ffn_forward_f32": (f32, [vp, sz, sz, sz, i32, i32, vp, f32, vp]),
        "or_expert_forward_sparse": (f32, [vp, sz, sz, sz, i32, i32, vp, f32, vp]),
        "or_build_active_mask": (sz, [vp, sz, f32, vp, vp]),
        "or_transpose_requantize_down": (None, [vp, vp, sz, sz, vp, vp]),
        "or_dequant_axpy_active": (None, [vp, vp, vp, vp, sz, sz, sz, vp]),
        "or_build_active_mask_mode": (sz, [vp, sz, f32, vp, vp, vp]),
        "or_ffn_forward_f32_mode": (f32, [vp, sz, sz, sz, i32, i32, vp, f32, vp, vp]),
        "or_expert_forward_sparse_mode": (f32, [vp, sz, sz, sz, i32, i32, vp, f32, vp, vp]),
        "or_route_sigmoid_bias": (None, [vp, vp, sz, sz, f32, i32, vp, vp]),
        "or_route_softmax_topk": (None, [vp, sz, sz, vp, vp]),
        "or_moe_routed": (None, [vp, sz, sz, sz, sz, i32, i32, vp, sz, sz, vp, vp, sz, f32, vp]),
        "or_moe_layer": (None, [vp, sz, sz, sz, sz, i32, i32, vp, sz, sz, vp, sz, vp, vp, sz, f32, vp]),
        "or_quantize_int4_group": (None, [vp, sz, sz, sz, vp, vp]),
        "or_rng_u64": (u64, [u64, u64, u64]),
        "or_rng_normal": (f64, [u64, u64, u64]),
        "or_fill_bytes": (None, [u64, u64, sz, vp]),
        "or_fill_scales": (None, [u64, u64, sz, i32, f64, f64, vp]),
        "or_fill_normal_f32": (None, [u64, u64, sz, vp]),
        "or_fill_normal_bf16": (None, [u64, u64, sz, vp]),
        "or_cpu_isa": (i32, []),
        "or_cpu_threads": (i32, []),
        "or_cpu_gemm": (None, [vp, vp, vp, sz, sz, sz, sz, i32, vp]),
        "or_cpu_expert_forward": (None, [vp, sz, sz, sz, sz, i32, vp, vp]),
        "or_cpu_moe_layer": (None, [vp, sz, sz, sz, sz, i32, vp, sz, sz, vp, sz, vp, vp, sz, f32, vp]),
        "or_ffn_forward_sparse_axpy_f32_mode": (f32, [vp, sz, sz, sz, i32, i32, vp, vp, vp, vp, vp,
                                                      vp, f32, vp, vp]),
        "or_ov_gemv": (None, [vp, vp, vp, sz, sz, sz, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


# ---------------- conversions ----------------

def f32_to_bf16(x) -> np.ndarray:
    """RNE f32 -> bf16 bits, NaN kept quiet (format.rs:151-160), vectorised."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((b[nan] >> 16) | 0x0040).astype(np.uint16)
    return r


def bf16_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def scale_to_f32(bits, scale_dtype: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    if scale_dtype == SCALE_F16:
        return bits.view(np.float16).astype(np.float32)
    return bf16_to_f32(bits)


# ---------------- layout ----------------

def expert_bytes(hidden, inter, group) -> int:
    return int(lib().or_expert_bytes(hidden, inter, group))


def expert_offsets(hidden, inter, group):
    gp = inter * hidden // 2
    gs = inter * (hidden // group) * 2
    dp = hidden * inter // 2
    ds = hidden * (inter // group) * 2
    o = [0, gp, gp + gs, 2 * gp + gs, 2 * (gp + gs), 2 * (gp + gs) + dp]
    return o, [gp, gs, gp, gs, dp, ds]


def dequant(packed, scales, n, k, group, sdt) -> np.ndarray:
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    out = np.empty((n, k), np.float32)
    lib().or_dequant(_p(packed), _p(scales), n, k, group, sdt, _p(out))
    return out


# ---------------- GEMV / GEMM ----------------

def gemv(packed, scales, x, n, k, group, sdt, order=ORDER_AVX512) -> np.ndarray:
    packed, scales, x = _c(packed, np.uint8), _c(scales, np.uint8), _c(x, np.float32)
    assert packed.size == n * k // 2 and scales.size == n * (k // group) * 2 and x.size == k
    y = np.empty(n, np.float32)
    lib().or_gemv(_p(packed), _p(scales), _p(x), n, k, group, sdt, order, _p(y))
    return y


def gemm_multi(packed, scales, xs, n, k, seq, group, sdt, order=ORDER_AVX512) -> np.ndarray:
    packed, scales, xs = _c(packed, np.uint8), _c(scales, np.uint8), _c(xs, np.float32)
    assert xs.size == seq * k
    ys = np.empty((seq, n), np.float32)
    lib().or_gemm_multi(_p(packed), _p(scales), _p(xs), n, k, seq, group, sdt, order, _p(ys))
    return ys


def gemv_rows_subset(packed, scales, x, n, k, group, sdt, rows, y, order=ORDER_AVX512):
    packed, scales, x = _c(packed, np.uint8), _c(scales, np.uint8), _c(x, np.float32)
    rows = _c(rows, np.uint32)
    assert y.dtype == np.float32 and y.flags.c_contiguous and y.size == n
    lib().or_gemv_rows_subset(_p(packed), _p(scales), _p(x), n, k, group, sdt, order,
                              _p(rows), rows.size, _p(y))
    return y


# ---------------- expert FFN ----------------

def expert_forward(x_bf16, flat, hidden, inter, group, sdt, order=ORDER_AVX512) -> np.ndarray:
    x_bf16, flat = _c(x_bf16, np.uint16), _c(flat, np.uint8)
    out = np.empty(hidden, np.uint16)
    lib().or_expert_forward(_p(x_bf16), hidden, inter, group, sdt, order, _p(flat), _p(out))
    return out


def _thr(thresholds, n):
    if thresholds is None:
        return None, None
    t = _c(thresholds, np.float32)
    assert t.size == n, "one threshold per intermediate lane"
    return t, _p(t)


def ffn_forward_f32(x, flat, hidden, inter, group, sdt, tau=0.0, order=ORDER_AVX512,
                    thresholds=None):
    x, flat = _c(x, np.float32), _c(flat, np.uint8)
    t, tp = _thr(thresholds, inter)
    out = np.empty(hidden, np.float32)
    frac = lib().or_ffn_forward_f32_mode(_p(x), hidden, inter, group, sdt, order, _p(flat),
                                         tau, tp, _p(out))
    return out, float(frac)


def expert_forward_sparse(x_bf16, flat, hidden, inter, group, sdt, tau, order=ORDER_AVX512,
                          thresholds=None):
    x_bf16, flat = _c(x_bf16, np.uint16), _c(flat, np.uint8)
    t, tp = _thr(thresholds, inter)
    out = np.empty(hidden, np.uint16)
    frac = lib().or_expert_forward_sparse_mode(_p(x_bf16), hidden, inter, group, sdt, order,
                                               _p(flat), tau, tp, _p(out))
    return out, float(frac)


def transpose_requantize_down(packed, scales, hidden, inter):
    """ffn_axpy.rs:342: -> (packed_t u8[inter * hidden / 2], scale_t u8[inter * hidden / 32 * 2])."""
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    pt = np.empty(inter * hidden // 2, np.uint8)
    st = np.empty(inter * (hidden // 32) * 2, np.uint8)
    lib().or_transpose_requantize_down(_p(packed), _p(scales), hidden, inter, _p(pt), _p(st))
    return pt, st


def dequant_axpy_active(packed_t, scale_t, scalars, active, inter, hidden, y=None):
    """ffn_axpy.rs:82: y (f32 [hidden], default zeros) += sum over active rows."""
    packed_t, scale_t = _c(packed_t, np.uint8), _c(scale_t, np.uint8)
    scalars, active = _c(scalars, np.float32), _c(active, np.uint32)
    y = np.zeros(hidden, np.float32) if y is None else _c(y, np.float32).copy()
    lib().or_dequant_axpy_active(_p(packed_t), _p(scale_t), _p(scalars), _p(active), active.size,
                                 inter, hidden, _p(y))
    return y


def ffn_forward_sparse_axpy_f32(x, flat, down_pt, down_st, hidden, inter, group, sdt, tau,
                                thresholds=None, order=ORDER_AVX512):
    """ffn_sparsity.rs:638-740: gate / up from the crate-layout expert blob
    `flat`, down from transpose_requantize_down's (down_pt, down_st);
    returns (out f32 [hidden], active fraction)."""
    x, flat = _c(x, np.float32), _c(flat, np.uint8)
    pt, st = _c(down_pt, np.uint8), _c(down_st, np.uint8)
    t, tp = _thr(thresholds, inter)
    offs, _ = expert_offsets(hidden, inter, group)
    base = flat.ctypes.data
    out = np.empty(hidden, np.float32)
    frac = lib().or_ffn_forward_sparse_axpy_f32_mode(
        _p(x), hidden, inter, group, sdt, order, C.c_void_p(base + offs[0]),
        C.c_void_p(base + offs[1]), C.c_void_p(base + offs[2]), C.c_void_p(base + offs[3]),
        _p(pt), _p(st), tau, tp, _p(out))
    return out, float(frac)


def build_active_mask(gate_out, tau, thresholds=None):
    g = _c(gate_out, np.float32)
    t, tp = _thr(thresholds, g.size)
    silu = np.empty_like(g)
    act = np.empty(g.size, np.uint32)
    n = lib().or_build_active_mask_mode(_p(g), g.size, tau, tp, _p(silu), _p(act))
    return silu, act[:n].copy()


# ---------------- routing / MoE ----------------

def route_sigmoid_bias(logits, bias, top_k, scale, norm=True):
    logits = _c(logits, np.float32)
    E = logits.size
    b = None if bias is None else _c(bias, np.float32)
    ids = np.empty(top_k, np.int64)
    w = np.empty(top_k, np.float32)
    lib().or_route_sigmoid_bias(_p(logits), None if b is None else _p(b), E, top_k, scale,
                                1 if norm else 0, _p(ids), _p(w))
    return ids, w


def route_softmax_topk(logits, top_k):
    logits = _c(logits, np.float32)
    ids = np.empty(top_k, np.int64)
    w = np.empty(top_k, np.float32)
    lib().or_route_softmax_topk(_p(logits), logits.size, top_k, _p(ids), _p(w))
    return ids, w


def moe_routed(x, experts, n_experts, hidden, inter, group, sdt, ids, weights, threshold=0.0,
               order=ORDER_AVX512):
    x = _c(x, np.float32)
    T = x.size // hidden
    experts = _c(experts, np.uint8)
    stride = experts.size // n_experts
    ids, weights = _c(ids, np.int64), _c(weights, np.float32)
    k = ids.size // T
    out = np.empty((T, hidden), np.float32)
    lib().or_moe_routed(_p(x), T, hidden, inter, group, sdt, order, _p(experts), stride,
                        n_experts, _p(ids), _p(weights), k, threshold, _p(out))
    return out


def moe_layer(x, experts, n_experts, shared, shared_inter, hidden, inter, group, sdt, ids,
              weights, threshold=0.0, order=ORDER_AVX512):
    x = _c(x, np.float32)
    T = x.size // hidden
    experts = _c(experts, np.uint8)
    stride = experts.size // n_experts
    ids, weights = _c(ids, np.int64), _c(weights, np.float32)
    k = ids.size // T
    sh = None if shared is None else _c(shared, np.uint8)
    out = np.empty((T, hidden), np.float32)
    lib().or_moe_layer(_p(x), T, hidden, inter, group, sdt, order, _p(experts), stride,
                       n_experts, None if sh is None else _p(sh), shared_inter, _p(ids),
                       _p(weights), k, threshold, _p(out))
    return out


def quantize_int4_group(w_bf16, n, k, group):
    w = _c(w_bf16, np.uint16)
    packed = np.empty(n * k // 2, np.uint8)
    scales = np.empty(n * (k // group) * 2, np.uint8)
    lib().or_quantize_int4_group(_p(w), n, k, group, _p(packed), _p(scales))
    return packed, scales


# ---------------- generators ----------------

def fill_bytes(seed, stream, n):
    out = np.empty(n, np.uint8)
    lib().or_fill_bytes(seed, stream, n, _p(out))
    return out


def fill_scales(seed, stream, n, sdt, sigma=0.02, offset=1e-3):
    out = np.empty(n, np.uint16)
    lib().or_fill_scales(seed, stream, n, sdt, sigma, offset, _p(out))
    return out


def fill_normal_f32(seed, stream, n):
    out = np.empty(n, np.float32)
    lib().or_fill_normal_f32(seed, stream, n, _p(out))
    return out


def fill_normal_bf16(seed, stream, n):
    out = np.empty(n, np.uint16)
    lib().or_fill_normal_bf16(seed, stream, n, _p(out))
    return out


# ---------------- CPU baseline (timed) ----------------

def cpu_isa() -> int:
    return int(lib().or_cpu_isa())


def cpu_threads() -> int:
    return int(lib().or_cpu_threads())


def cpu_gemm(packed, scales, xs, n, k, seq, group, sdt, out=None):
    xs = _c(xs, np.float32)
    if out is None:
        out = np.empty((seq, n), np.float32)
    lib().or_cpu_gemm(_p(packed), _p(scales), _p(xs), n, k, seq, group, sdt, _p(out))
    return out


def cpu_expert_forward(x_bf16, n_tokens, flat, hidden, inter, group, sdt, out=None):
    x_bf16 = _c(x_bf16, np.uint16)
    if out is None:
        out = np.empty((n_tokens, hidden), np.uint16)
    lib().or_cpu_expert_forward(_p(x_bf16), n_tokens, hidden, inter, group, sdt, _p(flat), _p(out))
    return out


def cpu_moe_layer(x, experts, n_experts, shared, shared_inter, hidden, inter, group, sdt, ids,
                  weights, threshold=0.0, stride=None):
    """The runner's per-(token, slot) MoE loop on the crate-dispatch CPU
    kernels (timed baseline; bit-identical per token to moe_layer)."""
    x = _c(x, np.float32)
    T = x.size // hidden
    experts = _c(experts, np.uint8)
    stride = experts.size // n_experts if stride is None else stride
    ids, weights = _c(ids, np.int64), _c(weights, np.float32)
    k = ids.size // T
    sh = None if shared is None else _c(shared, np.uint8)
    out = np.empty((T, hidden), np.float32)
    lib().or_cpu_moe_layer(_p(x), T, hidden, inter, group, sdt, _p(experts), stride, n_experts,
                           None if sh is None else _p(sh), shared_inter, _p(ids), _p(weights), k,
                           threshold, _p(out))
    return out


def ov_gemv(packed, scale_f16_bits, act, n, k, gsize):
    """gemv_offload.cpp:623-638: the CascadiaInt4Gemv op's scalar path, one
    activation row; two's-complement nibbles, f16 scales, any even group."""
    packed = _c(packed, np.uint8)
    sc = _c(scale_f16_bits, np.uint16)
    act = _c(act, np.float32)
    out = np.empty(n, np.float32)
    lib().or_ov_gemv(_p(packed), _p(sc), _p(act), n, k, gsize, _p(out))
    return out
