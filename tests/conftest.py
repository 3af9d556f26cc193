import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def norm_err(got, ref) -> float:
    """max |got - ref| / max |ref| over the tensor (the parity metric)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(np.max(np.abs(ref)), 1e-30)
    return float(np.max(np.abs(got - ref)) / scale)


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o
