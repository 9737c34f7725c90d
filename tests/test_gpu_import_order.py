"""The package imported before torch: one HIP runtime in the process.

The library links against libamdhip64; torch brings its own.  Whichever is
loaded first serves both, so the package imports torch before it loads the
library.  Run in a fresh interpreter (the test process has torch loaded
already): import cascadia_amd first, then torch, then one GEMV checked against
the numpy dequantised product.
"""
import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
sys.path.insert(0, sys.argv[1])
import cascadia_amd as cl   # before torch
import numpy as np
import torch
n, k, g = 64, 256, 32
rng = np.random.default_rng(5)
packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
scales = np.full(n * (k // g), 0x3C00, np.uint16)          # fp16 1.0
x = rng.normal(0, 1, k).astype(np.float32)
y = torch.empty(n, dtype=torch.float32, device="cuda")
cl.dequant_gemv_int4(torch.from_numpy(packed.ravel()).cuda(),
                     torch.from_numpy(scales.view(np.uint8)).cuda(),
                     torch.from_numpy(x).cuda(), n, k, y, group_size=g,
                     scale_dtype=cl.SCALE_F16)
q = np.stack([packed & 15, packed >> 4], -1).reshape(n, k).astype(np.float64) - 8
want = q @ x.astype(np.float64)
got = y.cpu().numpy()
err = np.abs(got - want).max()
print("max_abs", err, flush=True)
sys.exit(0 if err <= 1e-3 * max(1.0, np.abs(want).max()) else 1)
"""


def test_package_before_torch():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("import order: cascadia_amd before torch (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", SCRIPT, ROOT], capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
