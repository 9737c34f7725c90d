"""The C++ host API (include/cascadia_int4.hpp, the crate's public API in
C++ over device slices) on the GPU: tests/cpp/test_cpp_api.cpp calls every
mirrored function and checks it against the CPU oracle at the parity bars,
and the crate's error behaviour (see that file).  Built by
__graft_entry__.build() into tests/cpp/_build/."""
import os
import subprocess

import pytest
import torch

from conftest import GOLDEN, ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_cpp_api")


@pytest.mark.gpu
def test_cpp_host_api():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    assert os.path.exists(BIN), f"{BIN} missing: run __graft_entry__.build()"
    fixture = os.path.join(GOLDEN, "fixture_experts", "dsv4_layer_00", "expert_000.bin")
    r = subprocess.run([BIN, fixture], capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "checks OK" in r.stdout
