"""ctypes binding of libcascadia_int4_hip.so (the C ABI in include/cascadia_int4.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
# the in-tree build; CASCADIA_INT4_LIB names another build of the same ABI
LIB_PATH = os.environ.get("CASCADIA_INT4_LIB") or os.path.join(PKG, "lib",
                                                               "libcascadia_int4_hip.so")

OK = 0
ERR_NULL = -1
ERR_ARG = -2
ERR_DEVICE = -3
ERR_NOMEM = -4
SCALE_BF16 = 0
SCALE_F16 = 1
TILING_CRATE = 0
TILING_MFMA = 1
TILING_MFMA_UP_ROWS = 2

_ERRS = {ERR_NULL: "null pointer", ERR_ARG: "invalid argument (shape/length/alignment)",
         ERR_DEVICE: "HIP device error", ERR_NOMEM: "device allocation failed"}


class CascadiaInt4Error(RuntimeError):
    def __init__(self, fn: str, rc: int):
        super().__init__(f"{fn} returned {rc} ({_ERRS.get(rc, 'unknown')})")
        self.rc = rc


class Layout(C.Structure):
    _fields_ = [("n_rows", C.c_uint32), ("k_cols", C.c_uint32),
                ("group_size", C.c_uint32), ("scale_dtype", C.c_uint32),
                ("tiling", C.c_uint32)]


class Expert(C.Structure):
    _fields_ = [("gate_packed", C.c_void_p), ("gate_scale", C.c_void_p),
                ("up_packed", C.c_void_p), ("up_scale", C.c_void_p),
                ("down_packed", C.c_void_p), ("down_scale", C.c_void_p),
                ("tiling", C.c_uint32)]


ROUTE_IDS = 0
ROUTE_SIGMOID_BIAS = 1
ROUTE_SOFTMAX_TOPK = 2


class MoeLayer(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("inter", C.c_uint32), ("group_size", C.c_uint32),
                ("scale_dtype", C.c_uint32), ("tiling", C.c_uint32), ("n_experts", C.c_uint32),
                ("experts", C.c_void_p), ("expert_stride", C.c_size_t), ("shared", Expert),
                ("shared_inter", C.c_uint32)]


class OvSegment(C.Structure):
    _fields_ = [("packed", C.c_void_p), ("scale_f16", C.c_void_p), ("n_rows", C.c_uint32),
                ("tiling", C.c_uint32)]


class Routing(C.Structure):
    _fields_ = [("mode", C.c_uint32), ("top_k", C.c_uint32), ("logits", C.c_void_p),
                ("bias", C.c_void_p), ("scale", C.c_float), ("normalize", C.c_uint32),
                ("ids", C.c_void_p), ("weights", C.c_void_p), ("threshold", C.c_float)]


_vp, _u32, _u64, _sz, _f64, _i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_size_t, C.c_double, C.c_int
_LP, _EP = C.POINTER(Layout), C.POINTER(Expert)
_MP, _RP = C.POINTER(MoeLayer), C.POINTER(Routing)

# Every symbol declared in include/cascadia_int4.h: (restype, argtypes).
SIGNATURES = {
    "cascadia_int4_version": (C.c_char_p, []),
    "cascadia_int4_synchronize": (_i32, [_vp]),
    "cascadia_int4_reload_tuning": (None, []),
    "cascadia_int4_dequant_gemv": (_i32, [_LP, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_dequant_gemv_rows_subset": (_i32, [_LP, _vp, _vp, _vp, _vp, _vp, _u32, _vp]),
    "cascadia_int4_build_active_mask": (_i32, [_vp, _u32, C.c_float, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_f32_to_bf16": (_i32, [_vp, _sz, _vp, _vp]),
    "cascadia_int4_bf16_to_f32": (_i32, [_vp, _sz, _vp, _vp]),
    "cascadia_int4_dequant_gemm_multi": (_i32, [_LP, _vp, _vp, _vp, _u32, _vp, _vp]),
    "cascadia_int4_dequant_gemm_bf16in": (_i32, [_LP, _vp, _vp, _vp, _u32, _vp, _vp]),
    "cascadia_int4_gemm_bf16": (_i32, [_LP, _vp, _vp, _vp, _u32, _vp, _vp]),
    "cascadia_int4_tiled_sizes": (_i32, [_LP, C.POINTER(_sz), C.POINTER(_sz)]),
    "cascadia_int4_tile_weights": (_i32, [_LP, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_expert_bytes": (_sz, [_u32, _u32, _u32]),
    "cascadia_int4_expert_tiled_bytes": (_sz, [_u32, _u32, _u32]),
    "cascadia_int4_tile_expert": (_i32, [_u32, _u32, _u32, _EP, _vp, _EP, _vp]),
    "cascadia_int4_expert_from_flat": (_i32, [_vp, _u32, _u32, _u32, _EP]),
    "cascadia_int4_ffn_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32]),
    "cascadia_int4_expert_forward_device": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, _vp, _vp, _vp]),
    "cascadia_int4_expert_forward_noalloc": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, _vp, _vp]),
    "cascadia_int4_ffn_forward_f32": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, _vp, _vp, _vp]),
    "cascadia_int4_gate_up_silu": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, _u32, _vp, _vp]),
    "cascadia_int4_moe_workspace_bytes": (_sz, [_MP, _u32, _u32]),
    "cascadia_int4_moe_forward": (_i32, [_MP, _RP, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_debug_dequant": (_i32, [_LP, _vp, _vp, _vp, _vp]),
    "cascadia_int4_stream_read": (_i32, [_vp, _sz, _vp, _vp]),
    "cascadia_int4_fill_synthetic": (_i32, [_u32, _u64, _u64, _sz, _f64, _f64, _u32, _vp, _vp]),
    "cascadia_int4_transpose_requantize_down": (_i32, [_u32, _u32, _u32, _u32, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_axpy_workspace_bytes": (_sz, [_u32, _u32]),
    "cascadia_int4_dequant_axpy_active": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "cascadia_int4_ffn_sparse_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32]),
    "cascadia_int4_ffn_forward_sparse_f32": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, C.c_float,
                                                    _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_expert_forward_sparse": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32, C.c_float,
                                                   _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_ffn_sparse_axpy_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32]),
    "cascadia_int4_ffn_forward_sparse_axpy_f32": (_i32, [_u32, _u32, _u32, _u32, _EP, _vp, _u32,
                                                         C.c_float, _vp, _vp, _vp, _vp, _vp]),
    "cascadia_int4_ov_to_crate": (_i32, [_vp, _sz, _vp, _vp]),
    "cascadia_int4_ov_gemv_workspace_bytes": (_sz, [C.POINTER(OvSegment), _u32, _u32, _u32, _u32]),
    "cascadia_int4_ov_gemv": (_i32, [C.POINTER(OvSegment), _u32, _u32, _u32, _vp, _u32, _u32, _vp,
                                     _u32, _vp, _vp]),
    "cascadia_int4_quantize_bf16": (_i32, [_vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "cascadia_int4_open_source": (_i32, [C.c_char_p, C.POINTER(_vp)]),
    "cascadia_int4_destroy_source": (None, [_vp]),
    "cascadia_int4_prewarm": (_i32, [_vp, _u32, _u32]),
    "cascadia_int4_expert_forward": (_i32, [_vp, _u32, _u32, _vp, _vp]),
    "cascadia_int4_source_set_cache_limits": (_i32, [_vp, _u64, _u64]),
    "cascadia_int4_source_cache_stats": (_i32, [_vp, C.POINTER(_u64), C.POINTER(_u64),
                                                C.POINTER(_u64)]),
    "cascadia_int4_prefetch": (_i32, [_vp, _u32, _u32]),
    "cascadia_int4_prefetch_wait": (_i32, [_vp]),
    "cascadia_int4_prefetch_stats": (_i32, [_vp, C.POINTER(_u64), C.POINTER(_u64),
                                            C.POINTER(_u64), C.POINTER(_u64)]),
}

_lib = None


def lib():
    """Load the library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python cascadia_amd/build.py` "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, rc: int) -> None:
    if rc != OK:
        raise CascadiaInt4Error(fn, rc)
