"""The short fp64 division, square root and Jacobi rotation of
slime_amd/csrc/fp64.hpp against the IEEE `/` and `sqrt` of the same device, bit for
bit (slime_probe_fp64_core in libslime_probe.so). The fitness solve uses the short
forms on its serial rotation chain; equal bits keep its rotations those of the
IEEE formulas that the oracle (oracle/ca_oracle.cpp, oracle_jacobi_eigs) states.
"""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _probe():
    path = os.path.join(ROOT, "slime_amd", "libslime_probe.so")
    if not os.path.exists(path):
        raise RuntimeError("libslime_probe.so is not built")
    lib = ctypes.CDLL(path)
    lib.slime_probe_fp64_core.restype = ctypes.c_longlong
    lib.slime_probe_fp64_core.argtypes = [ctypes.c_longlong, ctypes.c_ulonglong]
    return lib


@pytest.mark.parametrize("seed", [1, 0x5EED])
def test_short_fp64_forms_equal_ieee(seed):
    print(f"[case] fp64 core check seed={seed}", flush=True)
    bad = _probe().slime_probe_fp64_core(1 << 22, seed)
    assert bad == 0, f"{bad} mismatches in {4 << 22} comparisons"
