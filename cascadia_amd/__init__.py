"""cascadia_amd -- MI355X (gfx950) implementation of cascadia-int4-gemm's INT4
weight-only matmul hot path, behind the C ABI of include/cascadia_int4.h.

Importing the package loads libcascadia_int4_hip.so; it raises if the library
was not built (``python cascadia_amd/build.py``).  There is no CPU fallback.
"""
# torch first: its HIP runtime must be the process's one before the library
# (linked against libamdhip64) is loaded, or a program importing this package
# before torch would hold two HIP runtimes and device pointers from one would be
# invalid in the other.
import torch  # noqa: F401

from ._lib import (ROUTE_IDS, ROUTE_SIGMOID_BIAS, ROUTE_SOFTMAX_TOPK, CascadiaInt4Error,
                   LIB_PATH, SCALE_BF16, SCALE_F16, SIGNATURES, TILING_CRATE, TILING_MFMA,
                   TILING_MFMA_UP_ROWS, check, lib)

lib()  # fail loudly at import when the HIP library is missing

from .api import (GROUP_SIZE, HIDDEN, INTERMEDIATE, NIBBLES_PER_INT32, ExpertSource,  # noqa: E402
                  ExpertWeights, GemmError, GemmTruncated, SparsityMode, bf16_bits_to_f32,
                  build_active_mask, build_active_mask_mode, build_active_mask_per_channel,
                  dequant_gemv_int4_rows_subset, dequant_gemv_int4_rows_subset_auto,
                  expert_forward_sparse_mode, f32_to_bf16_bits, ffn_forward_sparse_f32_mode,
                  stream_read,
                  debug_dequant, dequant_gemm_int4_multi_auto,
                  dequant_gemm_int4_multi_blocked_auto, dequant_gemv_int4,
                  dequant_gemv_int4_auto, expert_bytes, expert_forward, expert_forward_sparse,
                  expert_forward_sparse_per_channel, ffn_forward_sparse_f32,
                  ffn_forward_sparse_f32_per_channel, ffn_sparse_workspace_bytes,
                  ffn_forward_sparse_axpy_f32, ffn_forward_sparse_axpy_f32_mode,
                  ffn_forward_sparse_axpy_f32_per_channel, ffn_sparse_axpy_workspace_bytes,
                  ffn_workspace_bytes, transpose_requantize_down, dequant_axpy_int4_active,
                  dequant_axpy_int4_active_auto, fill_bytes, fill_normal,
                  fill_scales, gate_up_silu, gemm_int4_bf16, MoEExperts, moe_forward,
                  moe_workspace_bytes, ov_gemv, ov_to_crate, quantize_int4_group, tile_weights,
                  tiled_sizes)

__all__ = [
    "CascadiaInt4Error", "LIB_PATH", "SCALE_BF16", "SCALE_F16", "SIGNATURES", "check", "lib",
    "GROUP_SIZE", "HIDDEN", "INTERMEDIATE", "NIBBLES_PER_INT32", "ExpertSource", "ExpertWeights",
    "debug_dequant", "dequant_gemm_int4_multi_auto", "dequant_gemm_int4_multi_blocked_auto",
    "dequant_gemv_int4", "dequant_gemv_int4_auto", "expert_bytes", "expert_forward",
    "expert_forward_sparse", "expert_forward_sparse_per_channel", "ffn_forward_sparse_f32",
    "ffn_forward_sparse_f32_per_channel", "ffn_sparse_workspace_bytes", "ffn_workspace_bytes",
    "ffn_forward_sparse_axpy_f32", "ffn_forward_sparse_axpy_f32_mode",
    "ffn_forward_sparse_axpy_f32_per_channel", "ffn_sparse_axpy_workspace_bytes",
    "transpose_requantize_down", "dequant_axpy_int4_active", "dequant_axpy_int4_active_auto", "fill_bytes",
    "fill_normal", "fill_scales", "gate_up_silu", "gemm_int4_bf16", "tile_weights",
    "tiled_sizes", "TILING_CRATE", "TILING_MFMA", "MoEExperts", "moe_forward",
    "moe_workspace_bytes", "ov_gemv", "ov_to_crate", "quantize_int4_group", "ROUTE_IDS",
    "ROUTE_SIGMOID_BIAS",
    "ROUTE_SOFTMAX_TOPK", "TILING_MFMA_UP_ROWS", "GemmError", "GemmTruncated", "SparsityMode",
    "bf16_bits_to_f32", "f32_to_bf16_bits", "build_active_mask", "build_active_mask_mode",
    "build_active_mask_per_channel", "dequant_gemv_int4_rows_subset",
    "dequant_gemv_int4_rows_subset_auto", "expert_forward_sparse_mode",
    "ffn_forward_sparse_f32_mode", "stream_read",
]
