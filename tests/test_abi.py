"""The C-ABI library loads and exports every symbol include/*.h declares; the
host-only entry points (no GPU work) behave as documented."""
import ctypes as C
import glob
import os
import re

import pytest

from conftest import ROOT


def header_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b(cascadia_int4_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def cl():
    import cascadia_amd

    return cascadia_amd


def test_library_exports_every_declared_symbol(cl):
    names = header_functions()
    assert len(names) >= 10
    L = C.CDLL(cl.LIB_PATH)
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # and the ctypes signature table covers exactly the header
    assert set(cl.SIGNATURES) == names


def test_version(cl):
    assert b"gfx950" in cl.lib().cascadia_int4_version()


def test_expert_bytes_matches_oracle(cl, orc):
    for h, i, g in [(7168, 2048, 32), (3072, 1536, 128), (4096, 14336, 128), (64, 32, 32)]:
        assert cl.expert_bytes(h, i, g) == orc.expert_bytes(h, i, g)
    assert cl.expert_bytes(7168, 2048, 32) == 2 * (2048 * 3584 + 2048 * 224 * 2) + 7168 * 1024 + 7168 * 64 * 2


def test_expert_from_flat_offsets(cl, orc):
    e = cl._lib.Expert()
    base = 1 << 20
    rc = cl.lib().cascadia_int4_expert_from_flat(base, 64, 32, 32, C.byref(e))
    assert rc == 0
    offs, _ = orc.expert_offsets(64, 32, 32)
    got = [e.gate_packed, e.gate_scale, e.up_packed, e.up_scale, e.down_packed, e.down_scale]
    assert [g - base for g in got] == offs
    assert cl.lib().cascadia_int4_expert_from_flat(base, 64, 32, 48, C.byref(e)) == cl._lib.ERR_ARG
    assert cl.lib().cascadia_int4_expert_from_flat(None, 64, 32, 32, C.byref(e)) == cl._lib.ERR_NULL


def test_argument_errors_before_device_work(cl):
    L = cl.lib()
    lay = cl._lib.Layout(64, 128, 32, 0)
    # NULL layout / NULL weights
    assert L.cascadia_int4_dequant_gemv(None, 16, 16, 16, 16, None) == cl._lib.ERR_NULL
    assert L.cascadia_int4_dequant_gemv(C.byref(lay), None, 16, 16, 16, None) == cl._lib.ERR_NULL
    # group not a multiple of 32, K not a multiple of G, bad scale dtype, seq 0
    for bad in [cl._lib.Layout(64, 128, 48, 0), cl._lib.Layout(64, 100, 32, 0),
                cl._lib.Layout(64, 128, 32, 7), cl._lib.Layout(0, 128, 32, 0)]:
        assert L.cascadia_int4_dequant_gemv(C.byref(bad), 16, 16, 16, 16, None) == cl._lib.ERR_ARG
    assert L.cascadia_int4_dequant_gemm_multi(C.byref(lay), 16, 16, 16, 0, 16, None) == cl._lib.ERR_ARG
    # misaligned packed pointer
    assert L.cascadia_int4_dequant_gemv(C.byref(lay), 17, 16, 16, 16, None) == cl._lib.ERR_ARG
    assert L.cascadia_int4_fill_synthetic(9, 0, 0, 16, 0.0, 0.0, 0, 16, None) == cl._lib.ERR_ARG
    assert L.cascadia_int4_expert_forward_device(64, 32, 32, 0, None, 16, 1, 16, None, None) == cl._lib.ERR_NULL
    # MoE: null layer / routing / x; bad expert count, top_k, stride, alignment
    R = cl._lib.Routing(mode=cl.ROUTE_SIGMOID_BIAS, top_k=8, logits=256)

    def layer(**kw):
        f = dict(hidden=256, inter=128, group_size=32, scale_dtype=0, tiling=0, n_experts=16,
                 experts=1 << 20, expert_stride=1 << 16)
        f.update(kw)
        return cl._lib.MoeLayer(**f)

    mf = L.cascadia_int4_moe_forward
    assert mf(None, C.byref(R), 256, None, 1, 256, None, None, None, None) == cl._lib.ERR_NULL
    assert mf(C.byref(layer()), None, 256, None, 1, 256, None, None, None, None) == cl._lib.ERR_NULL
    assert mf(C.byref(layer()), C.byref(R), None, None, 1, 256, None, None, None, None) == cl._lib.ERR_NULL
    for bad in [layer(n_experts=0), layer(n_experts=1025), layer(n_experts=4),
                layer(expert_stride=100), layer(expert_stride=256), layer(experts=(1 << 20) + 16),
                layer(group_size=48), layer(inter=100)]:
        assert mf(C.byref(bad), C.byref(R), 256, None, 1, 256, None, None, None, None) == cl._lib.ERR_ARG
    R17 = cl._lib.Routing(mode=cl.ROUTE_SIGMOID_BIAS, top_k=17, logits=256)
    assert mf(C.byref(layer()), C.byref(R17), 256, None, 1, 256, None, None, None, None) == cl._lib.ERR_ARG
    assert mf(C.byref(layer()), C.byref(R), 256, None, 0, 256, None, None, None, None) == cl._lib.ERR_ARG
    assert L.cascadia_int4_moe_workspace_bytes(C.byref(layer(n_experts=0)), 8, 1) == 0


def test_zero_rows_return_ok_before_device_work(cl):
    """Zero token rows read and write nothing: OK with NULL row buffers, no
    HIP call made (this runs without a device).  The weights are still
    validated; the seq-major GEMMs keep the crate's seq >= 1 assert
    (kernel_avx512_multi.rs:80)."""
    L = cl.lib()
    e = cl._lib.Expert()
    assert L.cascadia_int4_expert_from_flat(1 << 20, 64, 32, 32, C.byref(e)) == 0
    OK, NUL = 0, cl._lib.ERR_NULL
    assert L.cascadia_int4_expert_forward_device(64, 32, 32, 0, C.byref(e), None, 0, None, None,
                                                 None) == OK
    assert L.cascadia_int4_expert_forward_noalloc(64, 32, 32, 0, C.byref(e), None, 0, None,
                                                  None) == OK
    assert L.cascadia_int4_gate_up_silu(64, 32, 32, 0, C.byref(e), None, 1, 0, None, None) == OK
    assert L.cascadia_int4_ffn_forward_sparse_f32(64, 32, 32, 0, C.byref(e), None, 0, 0.3, None,
                                                  None, None, None, None) == OK
    assert L.cascadia_int4_expert_forward_sparse(64, 32, 32, 0, C.byref(e), None, 0, 0.3, None,
                                                 None, None, None, None) == OK
    assert L.cascadia_int4_ffn_forward_sparse_axpy_f32(64, 32, 32, 0, C.byref(e), None, 0, 0.3,
                                                       None, None, None, None, None) == OK
    assert L.cascadia_int4_dequant_axpy_active(16, 16, 16, None, 0, 32, 64, 16, None, None) == OK
    assert L.cascadia_int4_ov_to_crate(None, 0, None, None) == OK
    # weights are still checked, and one row needs its buffers
    assert L.cascadia_int4_expert_forward_device(64, 32, 32, 0, None, None, 0, None, None,
                                                 None) == NUL
    assert L.cascadia_int4_expert_forward_device(64, 32, 48, 0, C.byref(e), None, 0, None, None,
                                                 None) == cl._lib.ERR_ARG
    assert L.cascadia_int4_expert_forward_device(64, 32, 32, 0, C.byref(e), None, 1, None, None,
                                                 None) == NUL
    lay = cl._lib.Layout(64, 128, 32, 0)
    assert L.cascadia_int4_dequant_gemm_multi(C.byref(lay), 16, 16, 16, 0, 16,
                                              None) == cl._lib.ERR_ARG


def test_python_mirror_rejects_host_tensors(cl):
    import torch

    p = torch.zeros(64 * 64, dtype=torch.uint8)
    s = torch.zeros(64 * 2 * 2, dtype=torch.uint8)
    with pytest.raises(ValueError):
        cl.dequant_gemv_int4(p, s, torch.zeros(128), 64, 128, torch.zeros(64))


def test_expert_weights_open_errors(cl, tmp_path):
    """format.rs:63-72: a file shorter than one expert is GemmError::Truncated
    (expected / actual), a missing one an I/O GemmError -- both raised on the
    host before any device work."""
    p = tmp_path / "short.bin"
    p.write_bytes(b"\x88" * 100)
    with pytest.raises(cl.GemmTruncated) as ei:
        cl.ExpertWeights.open(str(p), hidden=512, inter=256, group_size=32)
    assert ei.value.expected == cl.expert_bytes(512, 256, 32) and ei.value.actual == 100
    with pytest.raises(cl.GemmError):
        cl.ExpertWeights.open(str(tmp_path / "missing.bin"))
    # the crate's own dims by default: K2.6's 7168 x 2048, G 32
    with pytest.raises(cl.GemmTruncated) as ei:
        cl.ExpertWeights.open(str(p))
    assert ei.value.expected == cl.expert_bytes(cl.HIDDEN, cl.INTERMEDIATE, cl.GROUP_SIZE)


def test_sparsity_mode_is_dense():
    """SparsityMode::is_dense (ffn_sparsity.rs:85-90): Global(t) is dense for
    t <= 0 only, so a NaN tau is sparse; a per-channel vector is dense when
    empty or every entry is <= 0 (a NaN entry is not)."""
    import torch

    import cascadia_amd as cl

    M = cl.SparsityMode
    assert M.Global(0.0).is_dense() and M.Global(-1.0).is_dense()
    assert not M.Global(float("nan")).is_dense() and not M.Global(0.1).is_dense()
    assert M.PerChannel(torch.tensor([0.0, -1.0])).is_dense()
    assert M.PerChannel(torch.empty(0)).is_dense()
    assert not M.PerChannel(torch.tensor([0.0, float("nan")])).is_dense()
    assert M.of(0.3).tau == 0.3 and M.of(torch.zeros(2)).thresholds is not None


def test_cpp_header_compiles():
    """include/cascadia_int4.hpp (the C++ mirror of the crate's API) and the
    program that tests it on the GPU compile as C++17, warnings as errors."""
    import shutil
    import subprocess

    if not shutil.which("g++") or not os.path.isdir("/opt/rocm/include"):
        pytest.skip("no g++ or ROCm headers")
    src = os.path.join(ROOT, "tests", "cpp", "test_cpp_api.cpp")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                        "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                        "-I" + os.path.join(ROOT, "include"), src],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
