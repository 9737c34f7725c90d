import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture
def tuning(monkeypatch):
    """Set a CASCADIA_INT4_* tuning variable for one test: tuning(name, value).
    The library reads those variables once per process, so every change is
    followed by cascadia_int4_reload_tuning(); teardown restores the
    environment and reloads again, so no setting leaks into later tests."""
    import cascadia_amd

    L = cascadia_amd.lib()

    def setenv(name, value):
        monkeypatch.setenv(name, str(value))
        L.cascadia_int4_reload_tuning()

    yield setenv
    monkeypatch.undo()
    L.cascadia_int4_reload_tuning()


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    den = np.sqrt(np.sum(want * want))
    num = np.sqrt(np.sum((got - want) ** 2))
    return float(num / den) if den > 0 else float(num)


def max_abs(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.max(np.abs(got - want))) if got.size else 0.0


# Parity bar from the north star: rel-L2 <= 1e-3 and max-abs <= 2e-2 against
# the fp32-accumulated CPU result; dequantised weights bit-exact.
REL_L2_TOL = 1e-3
MAX_ABS_TOL = 2e-2
