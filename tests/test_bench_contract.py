"""bench.py's byte counts and its one-GPU contract, on the CPU.

The headline `value` and `roofline.achieved` divide algorithmic bytes by
time.  Both counts must equal the figures the workload definition fixes:
- the decode FFN chain reads gate, up and down (codes + scales) once, plus
  M·H bf16 in and M·H bf16 out: 90,832,896 + 16,384·M bytes at config 1;
- the fused gate/up kernel reads two matrices, x, and writes M·I f32:
  60,620,800 bytes at M = 1.
The rotation of weight copies must push every matrix past twice the
Infinity Cache, so that no timed step reads its weights from it.  A run
asking for more than one GPU must stop with an error line, not measure.
"""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402  (module scope imports only the standard library)

H, I, G = 4096, 14336, 128


@pytest.mark.parametrize("m", [1, 4, 16])
def test_chain_bytes(m):
    # 3 matrices x (14336 x 4096 / 2 codes + 14336 x 32 x 2 scale bytes)
    assert 3 * (I * H // 2 + I * (H // G) * 2) == 90_832_896
    assert bench.ffn_bytes(H, I, G, m) == 90_832_896 + 16_384 * m


def test_gate_up_bytes():
    assert bench.gate_up_bytes(H, I, G, 1) == 60_620_800
    # each extra token adds its bf16 row in and its f32 SwiGLU row out
    assert bench.gate_up_bytes(H, I, G, 2) - bench.gate_up_bytes(H, I, G, 1) == H * 2 + I * 4


@pytest.mark.parametrize("h,i,g", [(4096, 14336, 128), (7168, 2048, 32), (3072, 1536, 128)])
def test_copies_rotate_past_the_infinity_cache(h, i, g):
    n = bench.chain_copies(None, h, i, g)
    smallest = h * i // 2 + h * (i // g) * 2  # one matrix: the down (or any of the three)
    # the n - 1 copies read between two uses of one copy exceed 2x the cache
    assert (n - 1) * smallest > 2 * bench.MALL_BYTES


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
