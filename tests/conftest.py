import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library")


@pytest.fixture(scope="session")
def ctx():
    import vlrf_amd as V
    if V.Context.device_count() == 0:
        pytest.fail("no HIP device visible: the gpu tests need an MI355X")
    c = V.Context(0)
    print("\n[device]", c.device_info(), flush=True)
    yield c


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


def rel_err(a, b):
    """max |a-b| / max |b| (the tolerance measure used across the parity tests)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / den) if den > 0 else float(np.max(np.abs(a - b)))
