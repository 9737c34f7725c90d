"""Python mirror of cascadia-int4-gemm's public API over HBM-resident tensors.

Same function names, argument order and meaning as the crate
(crates/cascadia-int4-gemm/src/lib.rs:29-78), with torch device tensors in
place of Rust slices.  Where the crate panics on a length mismatch
(assert_eq!, kernel.rs:39-43) these raise ValueError before any GPU work.
Work is enqueued on torch's current stream; reading a result back (e.g.
``.cpu()``) waits for it, as the crate's synchronous call would.

torch is plumbing here (device memory, streams); every computation runs in
libcascadia_int4_hip.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import (ROUTE_IDS, ROUTE_SIGMOID_BIAS, ROUTE_SOFTMAX_TOPK, Expert, Layout, MoeLayer,
                   OvSegment, Routing, SCALE_BF16, SCALE_F16, TILING_CRATE, TILING_MFMA,
                   TILING_MFMA_UP_ROWS, check, lib)

# K2.6 constants of the crate (lib.rs:71-78)
HIDDEN = 7168
INTERMEDIATE = 2048
GROUP_SIZE = 32
NIBBLES_PER_INT32 = 8


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _dev(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a device (HBM) tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _expect(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _is_bf16_bits(t: torch.Tensor) -> bool:
    return t.dtype in (torch.bfloat16, torch.int16, torch.uint16)


def _layout(n_rows, k_cols, group_size, scale_dtype, tiling=TILING_CRATE) -> Layout:
    return Layout(n_rows, k_cols, group_size, scale_dtype, tiling)


def tiled_sizes(n_rows, k_cols, group_size=GROUP_SIZE):
    """(packed, scale) byte sizes of the MFMA-tiled copy of a matrix."""
    pb, sb = C.c_size_t(), C.c_size_t()
    L = _layout(n_rows, k_cols, group_size, SCALE_BF16)
    check("cascadia_int4_tiled_sizes", lib().cascadia_int4_tiled_sizes(C.byref(L), C.byref(pb), C.byref(sb)))
    return pb.value, sb.value


def _check_weights(packed, scale_bits, n_rows, k_cols, group_size, tiling=TILING_CRATE):
    _dev(packed, "packed")
    _dev(scale_bits, "scale_bits")
    _expect(group_size % 32 == 0 and k_cols % group_size == 0,
            f"k_cols {k_cols} must be a multiple of group_size {group_size} (a multiple of 32)")
    if tiling == TILING_MFMA:
        pb, sb = tiled_sizes(n_rows, k_cols, group_size)
    else:
        pb, sb = n_rows * (k_cols // 2), n_rows * (k_cols // group_size) * 2
    _expect(_nbytes(packed) == pb, f"packed has {_nbytes(packed)} bytes, expected {pb}")
    _expect(_nbytes(scale_bits) == sb, f"scale_bits has {_nbytes(scale_bits)} bytes, expected {sb}")


def tile_weights(packed, scale_bits, n_rows, k_cols, group_size=GROUP_SIZE):
    """MFMA-tiled copies (packed, scales) of a crate-layout matrix."""
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size)
    pb, sb = tiled_sizes(n_rows, k_cols, group_size)
    pt = torch.empty(pb, dtype=torch.uint8, device=packed.device)
    st = torch.empty(sb, dtype=torch.uint8, device=packed.device)
    L = _layout(n_rows, k_cols, group_size, SCALE_BF16)
    check("cascadia_int4_tile_weights", lib().cascadia_int4_tile_weights(
        C.byref(L), packed.data_ptr(), scale_bits.data_ptr(), pt.data_ptr(), st.data_ptr(),
        _stream()))
    return pt, st


# ---------------------------------------------------------------------------
# GEMV / GEMM
# ---------------------------------------------------------------------------

def dequant_gemv_int4(packed, scale_bits, x, n_rows, k_cols, y, group_size=GROUP_SIZE,
                      scale_dtype=SCALE_BF16, tiling=TILING_CRATE):
    """y = W x (kernel.rs:31-71).  x f32 [k_cols], y f32 [n_rows]."""
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size, tiling)
    _dev(x, "x"), _dev(y, "y")
    _expect(x.dtype == torch.float32 and x.numel() == k_cols, "x must be f32 [k_cols]")
    _expect(y.dtype == torch.float32 and y.numel() == n_rows, "y must be f32 [n_rows]")
    L = _layout(n_rows, k_cols, group_size, scale_dtype, tiling)
    check("cascadia_int4_dequant_gemv", lib().cascadia_int4_dequant_gemv(
        C.byref(L), packed.data_ptr(), scale_bits.data_ptr(), x.data_ptr(), y.data_ptr(),
        _stream()))
    return y


dequant_gemv_int4_auto = dequant_gemv_int4  # kernel_avx512.rs:274-297


def dequant_gemv_int4_rows_subset(packed, scale_bits, x, n_rows, k_cols, y, active_rows,
                                  group_size=GROUP_SIZE, scale_dtype=SCALE_BF16,
                                  tiling=TILING_CRATE):
    """y[r] = (W x)[r] for r in active_rows only (ffn_sparsity.rs:187-243); the
    other entries of y are not touched (pre-zero y where defined values are
    needed).  x f32 [k_cols], y f32 [n_rows], active_rows a device tensor of
    32-bit row ids (int32 or uint32); rows >= n_rows are skipped."""
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size, tiling)
    _dev(x, "x"), _dev(y, "y"), _dev(active_rows, "active_rows")
    _expect(x.dtype == torch.float32 and x.numel() == k_cols, "x must be f32 [k_cols]")
    _expect(y.dtype == torch.float32 and y.numel() == n_rows, "y must be f32 [n_rows]")
    _expect(active_rows.element_size() == 4 and not active_rows.is_floating_point(),
            "active_rows must hold 32-bit row ids")
    L = _layout(n_rows, k_cols, group_size, scale_dtype, tiling)
    check("cascadia_int4_dequant_gemv_rows_subset", lib().cascadia_int4_dequant_gemv_rows_subset(
        C.byref(L), packed.data_ptr(), scale_bits.data_ptr(), x.data_ptr(), y.data_ptr(),
        active_rows.data_ptr(), active_rows.numel(), _stream()))
    return y


dequant_gemv_int4_rows_subset_auto = dequant_gemv_int4_rows_subset  # ffn_sparsity.rs:317-348


# ---------------------------------------------------------------------------
# scalar conversions (format.rs:130-160)
# ---------------------------------------------------------------------------

def _as_device(v, dtype) -> tuple:
    """(device tensor, was_scalar) for a device tensor or a Python number."""
    if isinstance(v, torch.Tensor):
        return _dev(v, "x"), False
    return torch.tensor([v], dtype=dtype, device="cuda"), True


def f32_to_bf16_bits(x):
    """format.rs:151-160 (RNE, NaN kept quiet): f32 -> bf16 bits, on the device.
    x: an f32 device tensor (-> uint16 bits as int16 storage) or a Python
    float (-> int)."""
    t, scalar = _as_device(x, torch.float32)
    _expect(t.dtype == torch.float32, "x must be f32")
    out = torch.empty(t.shape, dtype=torch.int16, device=t.device)
    check("cascadia_int4_f32_to_bf16", lib().cascadia_int4_f32_to_bf16(
        t.data_ptr(), t.numel(), out.data_ptr(), _stream()))
    return int(out.cpu().view(torch.uint16).item()) if scalar else out


def bf16_bits_to_f32(bits):
    """format.rs:130-135: bf16 bits -> f32 (exact), on the device.  bits: a
    16-bit device tensor (-> f32 tensor) or a Python int (-> float)."""
    if not isinstance(bits, torch.Tensor):
        bits = torch.tensor([bits & 0xFFFF], dtype=torch.int32).to(torch.int16).cuda()
        scalar = True
    else:
        _dev(bits, "bits")
        scalar = False
    _expect(bits.element_size() == 2, "bits must be 16-bit")
    out = torch.empty(bits.shape, dtype=torch.float32, device=bits.device)
    check("cascadia_int4_bf16_to_f32", lib().cascadia_int4_bf16_to_f32(
        bits.data_ptr(), bits.numel(), out.data_ptr(), _stream()))
    return float(out.cpu().item()) if scalar else out


# ---------------------------------------------------------------------------
# activation masks (ffn_sparsity.rs:71-179)
# ---------------------------------------------------------------------------

class SparsityMode:
    """SparsityMode (ffn_sparsity.rs:71-91): Global(tau) -- one threshold for
    every lane -- or PerChannel(thresholds) -- a device f32 tensor of one
    threshold per intermediate lane."""

    __slots__ = ("tau", "thresholds")

    def __init__(self, tau: float = 0.0, thresholds: torch.Tensor | None = None):
        self.tau, self.thresholds = float(tau), thresholds

    @staticmethod
    def Global(tau: float) -> "SparsityMode":  # noqa: N802 (the crate's variant name)
        return SparsityMode(tau=tau)

    @staticmethod
    def PerChannel(thresholds: torch.Tensor) -> "SparsityMode":  # noqa: N802
        return SparsityMode(thresholds=thresholds)

    def is_dense(self) -> bool:
        """ffn_sparsity.rs:85-90 (a NaN tau is not dense).  PerChannel reads the
        thresholds back from the device."""
        if self.thresholds is None:
            return self.tau <= 0.0
        t = self.thresholds
        return t.numel() == 0 or bool((t <= 0.0).all().item())

    @staticmethod
    def of(mode) -> "SparsityMode":
        """A SparsityMode from itself, a float (Global) or a tensor (PerChannel)."""
        if isinstance(mode, SparsityMode):
            return mode
        if isinstance(mode, torch.Tensor):
            return SparsityMode.PerChannel(mode)
        return SparsityMode.Global(float(mode))


def build_active_mask_mode(gate_out, mode):
    """ffn_sparsity.rs:131-179 on one row: (silu_gate f32 [n], active u32
    ids ascending) with |silu| >= cutoff * max|silu| (every lane when the max
    is 0 or the mode is dense).  gate_out: f32 device tensor [n]; mode: a
    SparsityMode, a float or a per-channel tensor.  Waits for the device to
    size the list, as the crate returns a Vec."""
    m = SparsityMode.of(mode)
    _dev(gate_out, "gate_out")
    _expect(gate_out.dtype == torch.float32, "gate_out must be f32")
    n = gate_out.numel()
    thr = 0
    if m.thresholds is not None:
        _dev(m.thresholds, "thresholds")
        # ffn_sparsity.rs:116-123: one threshold per lane
        _expect(m.thresholds.dtype == torch.float32 and m.thresholds.numel() == n,
                f"per-channel thresholds length {m.thresholds.numel()} != gate_out length {n}")
        thr = m.thresholds.data_ptr()
    silu = torch.empty(n, dtype=torch.float32, device=gate_out.device)
    act = torch.empty(n, dtype=torch.int32, device=gate_out.device)
    cnt = torch.zeros(1, dtype=torch.int32, device=gate_out.device)
    if n:
        check("cascadia_int4_build_active_mask", lib().cascadia_int4_build_active_mask(
            gate_out.data_ptr(), n, m.tau, thr, silu.data_ptr(), act.data_ptr(), cnt.data_ptr(),
            _stream()))
    k = int(cnt.item())
    return silu, act[:k]


def build_active_mask(gate_out, threshold: float):
    """ffn_sparsity.rs:106-108 (SparsityMode::Global)."""
    return build_active_mask_mode(gate_out, SparsityMode.Global(threshold))


def build_active_mask_per_channel(gate_out, thresholds):
    """ffn_sparsity.rs:115-125 (SparsityMode::PerChannel)."""
    _expect(isinstance(thresholds, torch.Tensor) and thresholds.numel() == gate_out.numel(),
            f"per-channel thresholds length {getattr(thresholds, 'numel', lambda: -1)()} != "
            f"gate_out length {gate_out.numel()}")
    return build_active_mask_mode(gate_out, SparsityMode.PerChannel(thresholds))


def dequant_gemm_int4_multi_auto(packed, scale_bits, xs, n_rows, k_cols, seq, ys,
                                 group_size=GROUP_SIZE, scale_dtype=SCALE_BF16,
                                 tiling=TILING_CRATE):
    """ys[t*n_rows + r] for t < seq (kernel_avx512_multi.rs:207-245).
    xs f32 [seq, k_cols]; bf16 xs use the exact bf16 MFMA path."""
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size, tiling)
    _dev(xs, "xs"), _dev(ys, "ys")
    _expect(seq >= 1, "seq must be >= 1")
    _expect(xs.numel() == seq * k_cols, f"xs must hold seq*k_cols = {seq * k_cols} values")
    _expect(ys.dtype == torch.float32 and ys.numel() == seq * n_rows,
            f"ys must be f32 [seq*n_rows = {seq * n_rows}]")
    L = _layout(n_rows, k_cols, group_size, scale_dtype, tiling)
    if xs.dtype == torch.float32:
        fn = "cascadia_int4_dequant_gemm_multi"
    else:
        _expect(_is_bf16_bits(xs), "xs must be f32 or bf16")
        fn = "cascadia_int4_dequant_gemm_bf16in"
    check(fn, getattr(lib(), fn)(C.byref(L), packed.data_ptr(), scale_bits.data_ptr(),
                                 xs.data_ptr(), seq, ys.data_ptr(), _stream()))
    return ys


dequant_gemm_int4_multi_blocked_auto = dequant_gemm_int4_multi_auto  # _blocked.rs:295-347


def gemm_int4_bf16(packed, scale_bits, xs_bf16, n_rows, k_cols, seq, ys_bf16,
                   group_size=GROUP_SIZE, scale_dtype=SCALE_BF16, tiling=TILING_CRATE):
    """Prefill GEMM: bf16 [seq, k_cols] in, bf16 [seq, n_rows] out (f32 inside)."""
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size, tiling)
    _dev(xs_bf16, "xs_bf16"), _dev(ys_bf16, "ys_bf16")
    _expect(_is_bf16_bits(xs_bf16) and xs_bf16.numel() == seq * k_cols, "xs_bf16 [seq, k_cols] bf16")
    _expect(_is_bf16_bits(ys_bf16) and ys_bf16.numel() == seq * n_rows, "ys_bf16 [seq, n_rows] bf16")
    L = _layout(n_rows, k_cols, group_size, scale_dtype, tiling)
    check("cascadia_int4_gemm_bf16", lib().cascadia_int4_gemm_bf16(
        C.byref(L), packed.data_ptr(), scale_bits.data_ptr(), xs_bf16.data_ptr(), seq,
        ys_bf16.data_ptr(), _stream()))
    return ys_bf16


# ---------------------------------------------------------------------------
# expert FFN
# ---------------------------------------------------------------------------

def expert_bytes(hidden: int, inter: int, group_size: int = GROUP_SIZE) -> int:
    return int(lib().cascadia_int4_expert_bytes(hidden, inter, group_size))


class GemmError(RuntimeError):
    """GemmError (format.rs:28-33): an I/O failure opening an expert file."""


class GemmTruncated(GemmError):
    """GemmError::Truncated: the file holds fewer bytes than an expert."""

    def __init__(self, expected: int, actual: int):
        super().__init__(f"expert file truncated: expected {expected} bytes, got {actual}")
        self.expected, self.actual = expected, actual


def _section_sizes(hidden, inter, group_size, tiling):
    """Byte sizes of the six sections (gate p/s, up p/s, down p/s) of an
    expert in `tiling` (MFMA_UP_ROWS: gate and down tiled, up crate-layout)."""
    crate_g = (inter * hidden // 2, inter * (hidden // group_size) * 2)
    crate_d = (hidden * inter // 2, hidden * (inter // group_size) * 2)
    if tiling == TILING_CRATE:
        return [*crate_g, *crate_g, *crate_d]
    tg = tiled_sizes(inter, hidden, group_size)
    td = tiled_sizes(hidden, inter, group_size)
    up = crate_g if tiling == TILING_MFMA_UP_ROWS else tg
    return [*tg, *up, *td]


class ExpertWeights:
    """One expert's flat blob in HBM with the six slice accessors of
    format.rs:51-126 (any hidden / inter / group size).  In the crate layout
    the sections are contiguous (format.rs:35-47); tiled blobs hold each
    section 256-byte aligned."""

    def __init__(self, flat: torch.Tensor, hidden: int, inter: int, group_size: int = GROUP_SIZE,
                 scale_dtype: int = SCALE_BF16, tiling: int = TILING_CRATE):
        _dev(flat, "flat")
        _expect(flat.dtype == torch.uint8, "flat must be uint8")
        _expect(tiling in (TILING_CRATE, TILING_MFMA, TILING_MFMA_UP_ROWS), "tiling")
        self.flat, self.hidden, self.inter = flat, hidden, inter
        self.group_size, self.scale_dtype, self.tiling = group_size, scale_dtype, tiling
        sz = _section_sizes(hidden, inter, group_size, tiling)
        o = [0]
        if tiling == TILING_CRATE:
            for n in sz[:-1]:
                o.append(o[-1] + n)
            need = expert_bytes(hidden, inter, group_size)
        else:
            for n in sz[:-1]:
                o.append(o[-1] + _align256(n))
            need = o[-1] + sz[-1]
        _expect(flat.numel() >= need, f"flat expert too small: {flat.numel()} < {need}")
        self._slices = [flat[a:a + n] for a, n in zip(o, sz)]

    @staticmethod
    def open(path, hidden: int = HIDDEN, inter: int = INTERMEDIATE,
             group_size: int = GROUP_SIZE, scale_dtype: int = SCALE_BF16,
             device: str | torch.device = "cuda") -> "ExpertWeights":
        """ExpertWeights::open (format.rs:63-96): a flat expert file -- gate_p,
        gate_s, up_p, up_s, down_p, down_s -- read into HBM.  The crate's dims
        are K2.6's (HIDDEN x INTERMEDIATE, G 32, bf16 scales, lib.rs:71-78); a
        file shorter than one expert raises GemmTruncated, an unreadable one
        GemmError; extra bytes past the expert are ignored, as there."""
        need = expert_bytes(hidden, inter, group_size)
        try:
            with open(path, "rb") as f:
                f.seek(0, 2)
                size = f.tell()
                if size < need:
                    raise GemmTruncated(need, size)
                f.seek(0)
                host = torch.empty(need, dtype=torch.uint8, pin_memory=True)
                if f.readinto(memoryview(host.numpy())) != need:
                    raise GemmError(f"{path}: short read")
        except OSError as e:
            raise GemmError(f"{path}: {e}") from e
        flat = torch.empty(need + (-need) % 256, dtype=torch.uint8, device=device)
        flat[:need].copy_(host, non_blocking=True)
        torch.cuda.current_stream().synchronize()  # the pinned buffer is freed on return
        return ExpertWeights(flat, hidden, inter, group_size, scale_dtype)

    def tiled(self, up_rows: bool = False) -> "ExpertWeights":
        """The MFMA-tiled copy of this (crate-layout) expert.  up_rows: keep up
        in the crate layout (TILING_MFMA_UP_ROWS), for the activation-sparse
        forms, which read up one row at a time."""
        _expect(self.tiling == TILING_CRATE, "already tiled")
        if not up_rows:
            nb = int(lib().cascadia_int4_expert_tiled_bytes(self.hidden, self.inter,
                                                            self.group_size))
            dst = torch.empty(nb, dtype=torch.uint8, device=self.flat.device)
            src = _expert_struct(*self._slices)
            out = Expert()
            check("cascadia_int4_tile_expert", lib().cascadia_int4_tile_expert(
                self.hidden, self.inter, self.group_size, C.byref(src), dst.data_ptr(),
                C.byref(out), _stream()))
            return ExpertWeights(dst, self.hidden, self.inter, self.group_size,
                                 self.scale_dtype, TILING_MFMA)
        sz = _section_sizes(self.hidden, self.inter, self.group_size, TILING_MFMA_UP_ROWS)
        o = [0]
        for n in sz[:-1]:
            o.append(o[-1] + _align256(n))
        dst = torch.empty(o[-1] + _align256(sz[-1]), dtype=torch.uint8, device=self.flat.device)
        H, I, G = self.hidden, self.inter, self.group_size
        for src_i, (n, k) in ((0, (I, H)), (4, (H, I))):  # gate and down tiled
            L = _layout(n, k, G, self.scale_dtype)
            check("cascadia_int4_tile_weights", lib().cascadia_int4_tile_weights(
                C.byref(L), self._slices[src_i].data_ptr(), self._slices[src_i + 1].data_ptr(),
                dst.data_ptr() + o[src_i], dst.data_ptr() + o[src_i + 1], _stream()))
        for j in (2, 3):  # up as it is
            dst[o[j]:o[j] + sz[j]].copy_(self._slices[j])
        return ExpertWeights(dst, H, I, G, self.scale_dtype, TILING_MFMA_UP_ROWS)

    def gate_packed_bytes(self): return self._slices[0]
    def gate_scale_bits(self): return self._slices[1]
    def up_packed_bytes(self): return self._slices[2]
    def up_scale_bits(self): return self._slices[3]
    def down_packed_bytes(self): return self._slices[4]
    def down_scale_bits(self): return self._slices[5]

    def slices(self):
        return tuple(self._slices)


def _expert_struct(gp, gs, up, us, dp, ds, tiling=TILING_CRATE) -> Expert:
    for t, n in zip((gp, gs, up, us, dp, ds), ("gate_packed", "gate_scale", "up_packed",
                                                 "up_scale", "down_packed", "down_scale")):
        _dev(t, n)
    return Expert(gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(), dp.data_ptr(),
                  ds.data_ptr(), tiling)


def _ffn_dims(x, gate_packed, gate_scale, up_packed, up_scale, down_packed, down_scale,
              group_size, hidden=None, tiling=TILING_CRATE):
    hidden = hidden if hidden is not None else x.shape[-1]
    _expect(hidden % group_size == 0, "hidden must be a multiple of group_size")
    # kernel.rs:86: intermediate inferred from the gate scale length (a
    # tiled gate's scales cover inter rounded up to 16 rows; inter is a
    # multiple of the group, so of 32)
    inter = _nbytes(gate_scale) // 2 // (hidden // group_size)
    _expect(inter > 0 and inter % group_size == 0, "intermediate must be a multiple of group_size")
    gp, gs, up, us, dp, ds = _section_sizes(hidden, inter, group_size, tiling)
    _expect(_nbytes(gate_packed) == gp and _nbytes(up_packed) == up, "gate/up packed lengths")
    _expect(_nbytes(gate_scale) == gs and _nbytes(up_scale) == us, "gate/up scale lengths")
    _expect(_nbytes(down_packed) == dp, "down packed length")
    _expect(_nbytes(down_scale) == ds, "down scale length")
    return hidden, inter


def gate_up_silu(x, gate_packed, gate_scale, up_packed, up_scale, inter_out,
                 group_size=GROUP_SIZE, scale_dtype=SCALE_BF16, tiling=TILING_CRATE):
    """inter = silu(gate·x) ⊙ (up·x), f32 [n_tokens, inter] (kernel.rs:96-120).
    x: bf16 or f32 [n_tokens, hidden]."""
    _dev(x, "x"), _dev(inter_out, "inter_out")
    hidden = x.shape[-1]
    _expect(hidden % group_size == 0, "hidden must be a multiple of group_size")
    inter = _nbytes(gate_scale) // 2 // (hidden // group_size)
    gp = tiled_sizes(inter, hidden, group_size)[0] if tiling == TILING_MFMA else inter * hidden // 2
    _expect(_nbytes(gate_packed) == gp and _nbytes(up_packed) == gp
            and _nbytes(up_scale) == _nbytes(gate_scale), "gate/up slice lengths")
    T = x.numel() // hidden
    _expect(inter_out.dtype == torch.float32 and inter_out.numel() == T * inter, "inter_out f32 [T, inter]")
    xf32 = x.dtype == torch.float32
    _expect(xf32 or _is_bf16_bits(x), "x must be f32 or bf16")
    e = Expert(gate_packed.data_ptr(), gate_scale.data_ptr(), up_packed.data_ptr(),
               up_scale.data_ptr(), gate_packed.data_ptr(), gate_scale.data_ptr(), tiling)
    check("cascadia_int4_gate_up_silu", lib().cascadia_int4_gate_up_silu(
        hidden, inter, group_size, scale_dtype, C.byref(e), x.data_ptr(), 1 if xf32 else 0, T,
        inter_out.data_ptr(), _stream()))
    return inter_out


def ffn_workspace_bytes(hidden, inter, n_tokens, group_size=GROUP_SIZE) -> int:
    """Workspace bytes of expert_forward / ffn_forward_sparse_f32 for n_tokens
    rows on the current device."""
    return int(lib().cascadia_int4_ffn_workspace_bytes(hidden, inter, group_size, n_tokens))


def expert_forward(x_bf16, gate_packed, gate_scale, up_packed, up_scale, down_packed,
                   down_scale, out_bf16, group_size=GROUP_SIZE, scale_dtype=SCALE_BF16,
                   workspace=None, tiling=TILING_CRATE):
    """out = bf16(down · (silu(gate·x) ⊙ up·x)) (kernel.rs:75-136).
    x_bf16 / out_bf16: bf16 [hidden] or [n_tokens, hidden] (rows independent)."""
    _dev(x_bf16, "x_bf16"), _dev(out_bf16, "out_bf16")
    _expect(_is_bf16_bits(x_bf16) and _is_bf16_bits(out_bf16), "x and out must be bf16")
    hidden, inter = _ffn_dims(x_bf16, gate_packed, gate_scale, up_packed, up_scale, down_packed,
                              down_scale, group_size, tiling=tiling)
    T = x_bf16.numel() // hidden
    _expect(x_bf16.numel() == T * hidden and out_bf16.numel() == T * hidden,
            "x and out must both be [n_tokens, hidden]")
    e = _expert_struct(gate_packed, gate_scale, up_packed, up_scale, down_packed, down_scale,
                       tiling)
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    check("cascadia_int4_expert_forward_device", lib().cascadia_int4_expert_forward_device(
        hidden, inter, group_size, scale_dtype, C.byref(e), x_bf16.data_ptr(), T,
        out_bf16.data_ptr(), ws, _stream()))
    return out_bf16


def _sparse_call(x, weights, out, threshold, thresholds, group_size, scale_dtype, workspace,
                 tiling, x_f32, hidden=None, intermediate=None):
    """The shared body of the sparse entry points: returns the active
    fraction per token row (a float for a 1-D x, else a list)."""
    gate_packed, gate_scale, up_packed, up_scale, down_packed, down_scale = weights
    _dev(x, "x"), _dev(out, "out")
    if x_f32:
        _expect(x.dtype == torch.float32 and out.dtype == torch.float32, "f32 in/out")
    else:
        _expect(_is_bf16_bits(x) and _is_bf16_bits(out), "x and out must be bf16")
    h, inter = _ffn_dims(x, gate_packed, gate_scale, up_packed, up_scale, down_packed,
                         down_scale, group_size, hidden, tiling)
    if intermediate is not None:
        _expect(inter == intermediate,
                f"intermediate {intermediate} != {inter} implied by gate_scale")
    T = x.numel() // h
    _expect(x.numel() == T * h and out.numel() == T * h, "x and out must be [n_tokens, hidden]")
    thr = 0
    if thresholds is not None:
        _dev(thresholds, "thresholds")
        # ffn_sparsity.rs:116-123: one threshold per intermediate lane
        _expect(thresholds.dtype == torch.float32 and thresholds.numel() == inter,
                f"per-channel thresholds length {thresholds.numel()} != gate_out length {inter}")
        thr = thresholds.contiguous().data_ptr()
    e = _expert_struct(gate_packed, gate_scale, up_packed, up_scale, down_packed, down_scale,
                       tiling)
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    dense = thresholds is None and threshold <= 0.0  # SparsityMode::is_dense (NaN: sparse)
    counts = None if dense else torch.empty(T, dtype=torch.int32, device=x.device)
    name = "cascadia_int4_ffn_forward_sparse_f32" if x_f32 else "cascadia_int4_expert_forward_sparse"
    check(name, getattr(lib(), name)(h, inter, group_size, scale_dtype, C.byref(e), x.data_ptr(),
                                     T, float(threshold), thr, out.data_ptr(),
                                     0 if dense else counts.data_ptr(), ws, _stream()))
    # the dense branch returns 1.0 without a host round trip (ffn_sparsity.rs:465-496)
    # count / inter in f32, as the crate computes it (ffn_sparsity.rs:500)
    frac = [1.0] * T if dense else [
        float(np.float32(c) / np.float32(inter)) for c in counts.cpu().tolist()]
    return frac[0] if x.dim() == 1 else frac


def ffn_sparse_axpy_workspace_bytes(hidden, inter, n_tokens, group_size=GROUP_SIZE) -> int:
    return int(lib().cascadia_int4_ffn_sparse_axpy_workspace_bytes(hidden, inter, group_size,
                                                                    n_tokens))


def ffn_forward_sparse_axpy_f32_mode(x_f32, hidden, intermediate, gate_packed, gate_scale,
                                     up_packed, up_scale, down_packed_t, down_scale_t_bits,
                                     out_f32, mode, group_size=GROUP_SIZE,
                                     scale_dtype=SCALE_BF16, workspace=None,
                                     tiling=TILING_CRATE):
    """ffn_sparsity.rs:638-740: the AXPY-form sparse SwiGLU FFN, f32 in / out.
    down_packed_t / down_scale_t_bits: transpose_requantize_down's layout
    ([intermediate, hidden] codes, bf16 scales in groups of 32 along hidden).
    mode: a float (SparsityMode::Global) or a device f32 tensor of one
    threshold per intermediate lane (SparsityMode::PerChannel).  `workspace`
    plays the crate's FfnScratch (ffn_axpy.rs:452).  Returns the active
    fraction (a float for a 1-D x, else one per row)."""
    _dev(x_f32, "x"), _dev(out_f32, "out")
    _expect(x_f32.dtype == torch.float32 and out_f32.dtype == torch.float32, "f32 in/out")
    _expect(hidden % 32 == 0 and hidden % group_size == 0, "hidden: a multiple of 32 and of G")
    _check_weights(gate_packed, gate_scale, intermediate, hidden, group_size, tiling)
    _check_weights(up_packed, up_scale, intermediate, hidden, group_size, tiling)
    _dev(down_packed_t, "down_packed_t"), _dev(down_scale_t_bits, "down_scale_t_bits")
    _expect(_nbytes(down_packed_t) == intermediate * hidden // 2, "down_packed_t length")
    _expect(_nbytes(down_scale_t_bits) == intermediate * (hidden // 32) * 2,
            "down_scale_t_bits length")
    T = x_f32.numel() // hidden
    _expect(x_f32.numel() == T * hidden and out_f32.numel() == T * hidden,
            "x and out must be [n_tokens, hidden]")
    thr, tau = 0, 0.0
    m = SparsityMode.of(mode)
    if m.thresholds is not None:
        t = m.thresholds
        _dev(t, "thresholds")
        _expect(t.dtype == torch.float32 and t.numel() == intermediate,
                f"per-channel thresholds length {t.numel()} != intermediate {intermediate}")
        thr = t.data_ptr()
    else:
        tau = m.tau
    e = _expert_struct(gate_packed, gate_scale, up_packed, up_scale, down_packed_t,
                       down_scale_t_bits, tiling)
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    counts = torch.empty(T, dtype=torch.int32, device=x_f32.device)
    check("cascadia_int4_ffn_forward_sparse_axpy_f32",
          lib().cascadia_int4_ffn_forward_sparse_axpy_f32(
              hidden, intermediate, group_size, scale_dtype, C.byref(e), x_f32.data_ptr(), T,
              tau, thr, out_f32.data_ptr(), counts.data_ptr(), ws, _stream()))
    # count / intermediate in f32 (ffn_sparsity.rs:703)
    frac = [float(np.float32(c) / np.float32(intermediate)) for c in counts.cpu().tolist()]
    return frac[0] if x_f32.dim() == 1 else frac


def ffn_forward_sparse_axpy_f32(x_f32, hidden, intermediate, gate_packed, gate_scale, up_packed,
                                up_scale, down_packed_t, down_scale_t_bits, out_f32, threshold,
                                group_size=GROUP_SIZE, scale_dtype=SCALE_BF16, workspace=None,
                                tiling=TILING_CRATE):
    """ffn_sparsity.rs:569-600 (SparsityMode::Global)."""
    return ffn_forward_sparse_axpy_f32_mode(x_f32, hidden, intermediate, gate_packed, gate_scale,
                                            up_packed, up_scale, down_packed_t,
                                            down_scale_t_bits, out_f32, float(threshold),
                                            group_size, scale_dtype, workspace, tiling)


def ffn_forward_sparse_axpy_f32_per_channel(x_f32, hidden, intermediate, gate_packed,
                                            gate_scale, up_packed, up_scale, down_packed_t,
                                            down_scale_t_bits, out_f32, thresholds,
                                            group_size=GROUP_SIZE, scale_dtype=SCALE_BF16,
                                            workspace=None, tiling=TILING_CRATE):
    """ffn_sparsity.rs:605-633 (SparsityMode::PerChannel)."""
    return ffn_forward_sparse_axpy_f32_mode(x_f32, hidden, intermediate, gate_packed, gate_scale,
                                            up_packed, up_scale, down_packed_t,
                                            down_scale_t_bits, out_f32, thresholds, group_size,
                                            scale_dtype, workspace, tiling)


def transpose_requantize_down(src_packed, src_scale_bits, n_hidden, n_intermediate,
                              group_size=GROUP_SIZE, scale_dtype=SCALE_BF16):
    """ffn_axpy.rs:342-440: the down matrix [n_hidden, n_intermediate] (crate
    layout) -> (packed_t u8 [n_intermediate * n_hidden / 2], scale_t u8
    [n_intermediate * n_hidden / 32 * 2]), requantised in groups of 32 along
    hidden with bf16 scales, bit-identical to the crate."""
    _dev(src_packed, "src_packed"), _dev(src_scale_bits, "src_scale_bits")
    _expect(n_hidden % 32 == 0 and group_size % 32 == 0 and n_intermediate % group_size == 0,
            "hidden must be a multiple of 32 and the group a multiple of 32 dividing intermediate")
    _expect(src_packed.numel() * src_packed.element_size() == n_hidden * n_intermediate // 2,
            "src_packed length")
    _expect(src_scale_bits.numel() * src_scale_bits.element_size() ==
            n_hidden * (n_intermediate // group_size) * 2, "src_scale_bits length")
    pt = torch.empty(n_intermediate * n_hidden // 2, dtype=torch.uint8, device=src_packed.device)
    st = torch.empty(n_intermediate * (n_hidden // 32) * 2, dtype=torch.uint8,
                     device=src_packed.device)
    check("cascadia_int4_transpose_requantize_down", lib().cascadia_int4_transpose_requantize_down(
        n_hidden, n_intermediate, group_size, scale_dtype, src_packed.data_ptr(),
        src_scale_bits.data_ptr(), pt.data_ptr(), st.data_ptr(), _stream()))
    return pt, st


def dequant_axpy_int4_active(packed_t, scale_t_bits, scalars, active, n_intermediate, n_hidden,
                             y, workspace=None):
    """ffn_axpy.rs:82-160: y[n_hidden] += sum over r in active of scalars[r] *
    W_t[r, :] (device tensors; active int32/uint32 row ids)."""
    for t, n in ((packed_t, "packed_t"), (scale_t_bits, "scale_t_bits"), (scalars, "scalars"),
                 (active, "active"), (y, "y")):
        _dev(t, n)
    _expect(packed_t.numel() * packed_t.element_size() == n_intermediate * n_hidden // 2,
            "packed_t length")
    _expect(scale_t_bits.numel() * scale_t_bits.element_size() ==
            n_intermediate * (n_hidden // 32) * 2, "scale_t_bits length")
    _expect(scalars.dtype == torch.float32 and scalars.numel() == n_intermediate, "scalars")
    _expect(y.dtype == torch.float32 and y.numel() == n_hidden, "y")
    _expect(active.element_size() == 4, "active must hold 32-bit row ids")
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    check("cascadia_int4_dequant_axpy_active", lib().cascadia_int4_dequant_axpy_active(
        packed_t.data_ptr(), scale_t_bits.data_ptr(), scalars.data_ptr(), active.data_ptr(),
        active.numel(), n_intermediate, n_hidden, y.data_ptr(), ws, _stream()))
    return y


dequant_axpy_int4_active_auto = dequant_axpy_int4_active  # ffn_axpy.rs:274


def ffn_sparse_workspace_bytes(hidden, inter, n_tokens, group_size=GROUP_SIZE) -> int:
    """Workspace bytes of the sparse entry points for n_tokens rows."""
    return int(lib().cascadia_int4_ffn_sparse_workspace_bytes(hidden, inter, group_size,
                                                              n_tokens))


def expert_forward_sparse(x_bf16, gate_packed, gate_scale, up_packed, up_scale, down_packed,
                          down_scale, out_bf16, threshold, group_size=GROUP_SIZE,
                          scale_dtype=SCALE_BF16, workspace=None, tiling=TILING_CRATE):
    """ffn_sparsity.rs:756-783: bf16 in/out, activation-sparse with the global
    threshold (<= 0: expert_forward).  Returns the active fraction."""
    return _sparse_call(x_bf16, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                 down_scale), out_bf16, threshold, None, group_size,
                        scale_dtype, workspace, tiling, False)


def expert_forward_sparse_per_channel(x_bf16, gate_packed, gate_scale, up_packed, up_scale,
                                      down_packed, down_scale, out_bf16, thresholds,
                                      group_size=GROUP_SIZE, scale_dtype=SCALE_BF16,
                                      workspace=None, tiling=TILING_CRATE):
    """ffn_sparsity.rs:785-815: thresholds, device f32 [intermediate]."""
    return _sparse_call(x_bf16, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                 down_scale), out_bf16, 0.0, thresholds, group_size,
                        scale_dtype, workspace, tiling, False)


def ffn_forward_sparse_f32(x_f32, hidden, intermediate, gate_packed, gate_scale, up_packed,
                           up_scale, down_packed, down_scale, out_f32, threshold,
                           group_size=GROUP_SIZE, scale_dtype=SCALE_BF16, workspace=None,
                           tiling=TILING_CRATE):
    """SwiGLU FFN, f32 in/out (ffn_sparsity.rs:373-538): threshold <= 0 is the
    dense branch (the shared expert), > 0 the activation-sparse one.
    x_f32 / out_f32: [hidden] or [n_tokens, hidden].  Returns the active
    fraction."""
    return _sparse_call(x_f32, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                down_scale), out_f32, threshold, None, group_size, scale_dtype,
                        workspace, tiling, True, hidden, intermediate)


def ffn_forward_sparse_f32_mode(x_f32, hidden, intermediate, gate_packed, gate_scale, up_packed,
                                up_scale, down_packed, down_scale, out_f32, mode,
                                group_size=GROUP_SIZE, scale_dtype=SCALE_BF16, workspace=None,
                                tiling=TILING_CRATE):
    """ffn_sparsity.rs:438-538, the body of both f32 entry points: mode is a
    SparsityMode, a float (Global) or a per-channel device tensor."""
    m = SparsityMode.of(mode)
    return _sparse_call(x_f32, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                down_scale), out_f32, m.tau, m.thresholds, group_size,
                        scale_dtype, workspace, tiling, True, hidden, intermediate)


def expert_forward_sparse_mode(x_bf16, gate_packed, gate_scale, up_packed, up_scale, down_packed,
                               down_scale, out_bf16, mode, group_size=GROUP_SIZE,
                               scale_dtype=SCALE_BF16, workspace=None, tiling=TILING_CRATE):
    """ffn_sparsity.rs:812-867: bf16 in / out, mode a SparsityMode, a float or
    a per-channel device tensor; a dense mode is expert_forward."""
    m = SparsityMode.of(mode)
    return _sparse_call(x_bf16, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                 down_scale), out_bf16, m.tau, m.thresholds, group_size,
                        scale_dtype, workspace, tiling, False)


def ffn_forward_sparse_f32_per_channel(x_f32, hidden, intermediate, gate_packed, gate_scale,
                                       up_packed, up_scale, down_packed, down_scale, out_f32,
                                       thresholds, group_size=GROUP_SIZE,
                                       scale_dtype=SCALE_BF16, workspace=None,
                                       tiling=TILING_CRATE):
    """ffn_sparsity.rs:407-436: thresholds, device f32 [intermediate]."""
    return _sparse_call(x_f32, (gate_packed, gate_scale, up_packed, up_scale, down_packed,
                                down_scale), out_f32, 0.0, thresholds, group_size, scale_dtype,
                        workspace, tiling, True, hidden, intermediate)


# ---------------------------------------------------------------------------
# sparse-MoE layer
# ---------------------------------------------------------------------------

def _align256(n: int) -> int:
    return (n + 255) // 256 * 256


class MoEExperts:
    """The routed experts of one layer resident in HBM: expert e's blob at
    byte e * stride of one uint8 tensor, in the crate's flat layout
    (format.rs:35-47) or tiled (ExpertWeights.tiled()); plus an optional shared
    expert (an ExpertWeights of its own)."""

    def __init__(self, blobs: torch.Tensor, n_experts: int, hidden: int, inter: int,
                 group_size: int = GROUP_SIZE, scale_dtype: int = SCALE_BF16,
                 tiling: int = TILING_CRATE, stride: int | None = None,
                 shared: "ExpertWeights | None" = None):
        _dev(blobs, "blobs")
        _expect(blobs.dtype == torch.uint8, "blobs must be uint8")
        per = (int(lib().cascadia_int4_expert_tiled_bytes(hidden, inter, group_size))
               if tiling == TILING_MFMA else expert_bytes(hidden, inter, group_size))
        self.stride = stride if stride is not None else _align256(per)
        _expect(self.stride >= per and self.stride % 256 == 0, "stride: >= expert bytes, multiple of 256")
        _expect(blobs.numel() >= self.stride * (n_experts - 1) + per, "blobs too small")
        _expect(blobs.data_ptr() % 256 == 0, "blobs must be 256-byte aligned")
        if shared is not None:
            _expect(shared.hidden == hidden and shared.group_size == group_size
                    and shared.scale_dtype == scale_dtype, "shared expert dims")
        self.blobs, self.n_experts, self.hidden, self.inter = blobs, n_experts, hidden, inter
        self.group_size, self.scale_dtype, self.tiling, self.shared = group_size, scale_dtype, tiling, shared

    @staticmethod
    def from_crate(blobs: torch.Tensor, n_experts: int, hidden: int, inter: int,
                   group_size: int = GROUP_SIZE, scale_dtype: int = SCALE_BF16,
                   stride: int | None = None, shared=None, tiled: bool = True) -> "MoEExperts":
        """Experts given as crate-layout blobs at `stride`; tiled=True converts
        every expert (and the shared one) to the MFMA layout once."""
        crate = MoEExperts(blobs, n_experts, hidden, inter, group_size, scale_dtype,
                           TILING_CRATE, stride, shared)
        if not tiled:
            return crate
        per = int(lib().cascadia_int4_expert_tiled_bytes(hidden, inter, group_size))
        st = _align256(per)
        dst = torch.empty(st * n_experts, dtype=torch.uint8, device=blobs.device)
        for e in range(n_experts):
            src = ExpertWeights(blobs[e * crate.stride:e * crate.stride + expert_bytes(hidden, inter, group_size)],
                                hidden, inter, group_size, scale_dtype)
            out = Expert()
            check("cascadia_int4_tile_expert", lib().cascadia_int4_tile_expert(
                hidden, inter, group_size, C.byref(_expert_struct(*src.slices())),
                dst.data_ptr() + e * st, C.byref(out), _stream()))
        sh = shared.tiled() if (shared is not None and shared.tiling == TILING_CRATE) else shared
        return MoEExperts(dst, n_experts, hidden, inter, group_size, scale_dtype, TILING_MFMA, st, sh)

    def _struct(self) -> MoeLayer:
        L = MoeLayer()
        L.hidden, L.inter, L.group_size = self.hidden, self.inter, self.group_size
        L.scale_dtype, L.tiling, L.n_experts = self.scale_dtype, self.tiling, self.n_experts
        L.experts, L.expert_stride = self.blobs.data_ptr(), self.stride
        if self.shared is not None:
            L.shared = _expert_struct(*self.shared.slices(), self.shared.tiling)
            L.shared_inter = self.shared.inter
        return L


def moe_workspace_bytes(experts: MoEExperts, top_k: int, n_tokens: int) -> int:
    return int(lib().cascadia_int4_moe_workspace_bytes(C.byref(experts._struct()), top_k, n_tokens))


def moe_forward(experts: MoEExperts, x, out, *, top_k: int, logits=None, bias=None,
                mode: int = ROUTE_SIGMOID_BIAS, scale: float = 1.0, normalize: bool = True,
                ids=None, weights=None, threshold: float = 0.0, residual=None,
                ids_out=None, weights_out=None, workspace=None):
    """One MoE layer (runner.rs:1806-1832, batched over tokens):
    out = residual + shared(x) + sum_k w_k * bf16(expert_k(bf16(x))).
    x, out, residual: f32 [n_tokens, hidden] device tensors.  Routing from
    logits (f32 [n_tokens, n_experts]; sigmoid + bias, or softmax over the
    top-k) or given ids (int32) / weights (f32) [n_tokens, top_k]."""
    _dev(x, "x"), _dev(out, "out")
    H = experts.hidden
    _expect(x.dtype == torch.float32 and out.dtype == torch.float32, "x and out must be f32")
    T = x.numel() // H
    _expect(x.numel() == T * H and out.numel() == T * H and T >= 1, "x/out must be [n_tokens, hidden]")
    R = Routing()
    R.mode, R.top_k, R.scale, R.normalize, R.threshold = mode, top_k, scale, int(normalize), threshold
    if mode == ROUTE_IDS:
        _expect(ids is not None and weights is not None, "ROUTE_IDS needs ids and weights")
        _dev(ids, "ids"), _dev(weights, "weights")
        _expect(ids.dtype == torch.int32 and ids.numel() == T * top_k, "ids: int32 [n_tokens, top_k]")
        _expect(weights.dtype == torch.float32 and weights.numel() == T * top_k, "weights: f32 [n_tokens, top_k]")
        R.ids, R.weights = ids.data_ptr(), weights.data_ptr()
    else:
        _expect(logits is not None, "routing needs logits")
        _dev(logits, "logits")
        _expect(logits.dtype == torch.float32 and logits.numel() == T * experts.n_experts,
                "logits: f32 [n_tokens, n_experts]")
        R.logits = logits.data_ptr()
        if bias is not None:
            _dev(bias, "bias")
            _expect(bias.dtype == torch.float32 and bias.numel() == experts.n_experts, "bias: f32 [n_experts]")
            R.bias = bias.data_ptr()
    res = 0
    if residual is not None:
        _dev(residual, "residual")
        _expect(residual.dtype == torch.float32 and residual.numel() == T * H, "residual: f32 [n_tokens, hidden]")
        res = residual.data_ptr()
    io = wo = 0
    if ids_out is not None:
        _dev(ids_out, "ids_out")
        _expect(ids_out.dtype == torch.int32 and ids_out.numel() == T * top_k, "ids_out: int32 [n_tokens, top_k]")
        io = ids_out.data_ptr()
    if weights_out is not None:
        _dev(weights_out, "weights_out")
        _expect(weights_out.dtype == torch.float32 and weights_out.numel() == T * top_k, "weights_out: f32")
        wo = weights_out.data_ptr()
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    check("cascadia_int4_moe_forward", lib().cascadia_int4_moe_forward(
        C.byref(experts._struct()), C.byref(R), x.data_ptr(), res, T, out.data_ptr(), io, wo, ws,
        _stream()))
    return out


# ---------------------------------------------------------------------------
# the OpenVINO CascadiaInt4Gemv format (cascadia-ov-genai-shim/cpp/gemv_offload.cpp)
# ---------------------------------------------------------------------------

def ov_to_crate(packed_ov: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The op's two's-complement nibbles -> the crate's offset nibbles (every
    byte XOR 0x88; the same products).  out may be packed_ov (in place)."""
    _dev(packed_ov, "packed_ov")
    out = torch.empty_like(packed_ov) if out is None else _dev(out, "out")
    _expect(_nbytes(out) == _nbytes(packed_ov), "out size")
    check("cascadia_int4_ov_to_crate", lib().cascadia_int4_ov_to_crate(
        packed_ov.data_ptr(), _nbytes(packed_ov), out.data_ptr(), _stream()))
    return out


def ov_gemv(segments, k_cols: int, group_size: int, act, out, workspace=None):
    """The op's evaluate() (gemv_offload.cpp:413-660).  segments: a list of
    (packed, scale_f16, n_rows, tiling) with packed converted by ov_to_crate
    (and tiled, for TILING_MFMA); act: f16 or f32 [rows, k_cols]; out: f16 or
    f32 [rows, sum n_rows], the segments' outputs concatenated per row."""
    _dev(act, "act"), _dev(out, "out")
    _expect(act.dtype in (torch.float16, torch.float32) and out.dtype in (torch.float16,
                                                                          torch.float32),
            "act and out: f16 or f32")
    segs = (OvSegment * len(segments))()
    n_total = 0
    for j, (p, sc, n, tiling) in enumerate(segments):
        _check_weights(p, sc, n, k_cols, group_size, tiling)
        segs[j] = OvSegment(p.data_ptr(), sc.data_ptr(), n, tiling)
        n_total += n
    rows = act.numel() // k_cols
    _expect(act.numel() == rows * k_cols and rows >= 1, "act must be [rows, k_cols]")
    _expect(out.numel() == rows * n_total, "out must be [rows, sum of n_rows]")
    ws = 0 if workspace is None else _dev(workspace, "workspace").data_ptr()
    check("cascadia_int4_ov_gemv", lib().cascadia_int4_ov_gemv(
        segs, len(segments), k_cols, group_size, act.data_ptr(),
        int(act.dtype == torch.float16), rows, out.data_ptr(), int(out.dtype == torch.float16),
        ws, _stream()))
    return out


# ---------------------------------------------------------------------------
# debug / synthetic data
# ---------------------------------------------------------------------------

def debug_dequant(packed, scale_bits, n_rows, k_cols, group_size=GROUP_SIZE,
                  scale_dtype=SCALE_BF16, out=None):
    _check_weights(packed, scale_bits, n_rows, k_cols, group_size)
    if out is None:
        out = torch.empty((n_rows, k_cols), dtype=torch.float32, device=packed.device)
    L = _layout(n_rows, k_cols, group_size, scale_dtype)
    check("cascadia_int4_debug_dequant", lib().cascadia_int4_debug_dequant(
        C.byref(L), packed.data_ptr(), scale_bits.data_ptr(), out.data_ptr(), _stream()))
    return out


def quantize_int4_group(weight_bf16: torch.Tensor, n_rows: int, k_cols: int,
                        group_size: int = GROUP_SIZE):
    """Quantise bf16 weights [n_rows, k_cols] on the device into the crate
    layout: (packed u8 [n_rows * k_cols / 2], scales u8 [n_rows * k_cols /
    group_size * 2], bf16 little-endian).  shell_int4.rs:148-212, which asserts
    the length and that k_cols is a multiple of the group (32 there): those
    raise ValueError here.  `weight_bf16` holds the bf16 bits (bfloat16, int16
    or uint16 elements, or the raw bytes as uint8)."""
    _dev(weight_bf16, "weight_bf16")
    _expect(_nbytes(weight_bf16) == n_rows * k_cols * 2,
            f"weight_bf16 holds {_nbytes(weight_bf16)} bytes, expected {n_rows * k_cols * 2}")
    _expect(group_size > 0 and group_size % 32 == 0 and k_cols % group_size == 0,
            f"k_cols {k_cols} must be a multiple of group_size {group_size} (a multiple of 32)")
    _expect(weight_bf16.is_contiguous(), "weight_bf16 must be contiguous")
    packed = torch.empty(n_rows * k_cols // 2, dtype=torch.uint8, device=weight_bf16.device)
    scales = torch.empty(n_rows * (k_cols // group_size) * 2, dtype=torch.uint8,
                         device=weight_bf16.device)
    check("cascadia_int4_quantize_bf16", lib().cascadia_int4_quantize_bf16(
        weight_bf16.data_ptr(), n_rows, k_cols, group_size, packed.data_ptr(), scales.data_ptr(),
        _stream()))
    return packed, scales


class ExpertSource:
    """The crate's C handle API (c_ffi.rs:35-341) as its ctypes callers use it:
    a safetensors model directory, or an int4_bin one (manifest.json
    "experts_format": "int4_bin", experts/layer_LL/expert_EEE.bin), experts
    run one f32 vector at a time on host arrays of the model's hidden size.
    Experts are uploaded and tiled into HBM on first use (or by prewarm) and
    stay resident in an LRU cache (set_cache_limits; runner.rs:142-258) until
    evicted or close.  Errors raise CascadiaInt4Error with the crate's code
    (-1 null, -2 path or expert, -3 directory or HIP)."""

    def __init__(self, model_dir: str):
        h = C.c_void_p()
        check("cascadia_int4_open_source",
              lib().cascadia_int4_open_source(model_dir.encode(), C.byref(h)))
        self._h = h

    def prewarm(self, layer: int, expert: int) -> None:
        check("cascadia_int4_prewarm", lib().cascadia_int4_prewarm(self._h, layer, expert))

    def expert_forward(self, layer: int, expert: int, x_f32, out_f32) -> None:
        """x_f32, out_f32: contiguous host float32 numpy arrays of the hidden size."""
        import numpy as np

        _expect(isinstance(x_f32, np.ndarray) and x_f32.dtype == np.float32 and
                x_f32.flags.c_contiguous, "x_f32 must be a contiguous float32 numpy array")
        _expect(isinstance(out_f32, np.ndarray) and out_f32.dtype == np.float32 and
                out_f32.flags.c_contiguous and out_f32.size == x_f32.size,
                "out_f32 must be a contiguous float32 numpy array of x's size")
        check("cascadia_int4_expert_forward", lib().cascadia_int4_expert_forward(
            self._h, layer, expert, x_f32.ctypes.data, out_f32.ctypes.data))

    def set_cache_limits(self, max_experts: int = 0, max_bytes: int = 0) -> None:
        """Bound the resident experts (0 = unbounded); lowering evicts at once."""
        check("cascadia_int4_source_set_cache_limits",
              lib().cascadia_int4_source_set_cache_limits(self._h, max_experts, max_bytes))

    def cache_stats(self):
        """(resident experts, evictions so far, resident bytes) -- lru_stats
        (runner.rs:148-158) plus the bytes."""
        a, b, c = C.c_uint64(), C.c_uint64(), C.c_uint64()
        check("cascadia_int4_source_cache_stats", lib().cascadia_int4_source_cache_stats(
            self._h, C.byref(a), C.byref(b), C.byref(c)))
        return a.value, b.value, c.value

    def prefetch(self, layer: int, expert: int) -> None:
        """Queue an expert for the handle's background loader (the runner's
        Prefetcher, runner.rs:282-360): never blocks, drops the request when
        4096 are queued."""
        check("cascadia_int4_prefetch", lib().cascadia_int4_prefetch(self._h, layer, expert))

    def prefetch_wait(self) -> None:
        """Wait until every queued prefetch has been handled."""
        check("cascadia_int4_prefetch_wait", lib().cascadia_int4_prefetch_wait(self._h))

    def prefetch_stats(self):
        """(submitted, dropped, processed, loaded into HBM) -- the runner's
        submits / drops / processed counters (runner.rs:341-350) plus loads."""
        v = [C.c_uint64() for _ in range(4)]
        check("cascadia_int4_prefetch_stats", lib().cascadia_int4_prefetch_stats(
            self._h, *(C.byref(x) for x in v)))
        return tuple(x.value for x in v)

    def close(self) -> None:
        if self._h:
            lib().cascadia_int4_destroy_source(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def stream_read(buf: torch.Tensor, sink: torch.Tensor | None = None) -> torch.Tensor:
    """The benchmark's streaming-read ceiling: read every byte of `buf` the
    way the decode GEMV streams its weights (8 KB per wave, non-temporal) and
    XOR-fold the words into `sink` (int32 [1024], zeroed here when not given;
    the XOR of its words is the XOR of buf's words)."""
    _dev(buf, "buf")
    if sink is None:
        sink = torch.zeros(1024, dtype=torch.int32, device=buf.device)
    _dev(sink, "sink")
    _expect(sink.element_size() * sink.numel() == 4096, "sink must hold 1024 32-bit words")
    check("cascadia_int4_stream_read", lib().cascadia_int4_stream_read(
        buf.data_ptr(), _nbytes(buf), sink.data_ptr(), _stream()))
    return sink


def fill_bytes(out: torch.Tensor, seed: int, stream_id: int):
    _dev(out, "out")
    check("cascadia_int4_fill_synthetic", lib().cascadia_int4_fill_synthetic(
        0, seed, stream_id, _nbytes(out), 0.0, 0.0, 0, out.data_ptr(), _stream()))
    return out


def fill_scales(out: torch.Tensor, seed: int, stream_id: int, scale_dtype=SCALE_F16,
                sigma=0.02, offset=1e-3):
    _dev(out, "out")
    check("cascadia_int4_fill_synthetic", lib().cascadia_int4_fill_synthetic(
        1, seed, stream_id, _nbytes(out) // 2, sigma, offset, scale_dtype, out.data_ptr(),
        _stream()))
    return out


def fill_normal(out: torch.Tensor, seed: int, stream_id: int):
    """f32 or bf16 N(0, 1)."""
    _dev(out, "out")
    kind = 2 if out.dtype == torch.float32 else 3
    n = out.numel()
    check("cascadia_int4_fill_synthetic", lib().cascadia_int4_fill_synthetic(
        kind, seed, stream_id, n, 0.0, 0.0, 0, out.data_ptr(), _stream()))
    return out
