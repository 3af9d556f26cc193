"""CPU checks of the C ABI: the library loads, exports exactly what
include/slime_ca.h declares, and rejects bad arguments with status codes before
touching a device (no compute calls: this container has no GPU)."""
import ctypes
import os
import re

import pytest

from slime_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    with open(os.path.join(ROOT, "include", "slime_ca.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(slime_(?:ca|neural_ca|pool|snapshot)_\w+)\s*\(", text)))


def test_header_declares_the_exported_set():
    assert _header_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _header_functions():
        assert hasattr(lib, name), name


def _cfg(**kw):
    base = dict(B=1, G=32, H=8, D=8, dtype=_lib.SLIME_F32, dt=0.1, growth_per_cell=0, pods=1,
                pvi_chain=0)
    base.update(kw)
    return _lib.Config(**base)


@pytest.mark.parametrize("bad", [dict(B=0), dict(G=12), dict(G=4), dict(H=4), dict(D=48),
                                 dict(dtype=7), dict(pods=3), dict(dt=float("nan")),
                                 dict(growth_per_cell=2), dict(pvi_chain=5), dict(pvi_chain=3),
                                 dict(growth_fn=3), dict(growth_fn=-1), dict(conservation=2)])
def test_create_rejects_invalid_config(bad):
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.slime_ca_create(ctypes.byref(_cfg(**bad)), ctypes.byref(h))
    assert rc == _lib.SLIME_EINVAL
    assert not h.value
    assert lib.slime_ca_last_error()


@pytest.mark.parametrize("bad", [
    # bf16: G*G*C = 2056^2 * 512 > 2^31, past the stencil's int element offsets
    dict(B=1, G=2056, D=64, dtype=_lib.SLIME_BF16),
    # fp32: G*G*C*4 = 1456^2 * 512 * 4 > 2^32, past its unsigned byte offsets
    dict(B=1, G=1456, D=64, dtype=_lib.SLIME_F32),
    # bf16 state whose last step is written in fp32: 1456^2 * 512 * 4 > 2^32 too
    dict(B=1, G=1456, D=64, dtype=_lib.SLIME_BF16),
])
def test_create_rejects_batch_entries_past_32bit_offsets(bad):
    """validate() runs before any device call, so this needs no GPU."""
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.slime_ca_create(ctypes.byref(_cfg(**bad)), ctypes.byref(h))
    assert rc == _lib.SLIME_EINVAL
    assert not h.value
    assert b"32-bit" in lib.slime_ca_last_error()


def test_largest_batch_entry_within_32bit_offsets_is_not_rejected_as_too_large():
    """G = 1448 fp32 (1448^2 * 512 * 4 < 2^32) passes validation: without a GPU the
    call fails later, at the device check, not with the offset message."""
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.slime_ca_create(ctypes.byref(_cfg(B=1, G=1448, D=64)), ctypes.byref(h))
    if rc == _lib.SLIME_OK:  # a GPU is visible and had the memory
        lib.slime_ca_destroy(h)
        return
    assert b"32-bit" not in lib.slime_ca_last_error()


def test_null_arguments_are_errors_not_crashes():
    lib = _lib.load()
    assert lib.slime_ca_create(None, None) == _lib.SLIME_EINVAL
    h = ctypes.c_void_p()
    assert lib.slime_ca_create(None, ctypes.byref(h)) == _lib.SLIME_EINVAL
    assert lib.slime_ca_step(None, None, None, 1, None) == _lib.SLIME_EINVAL
    assert lib.slime_ca_set_params(None, None) == _lib.SLIME_EINVAL
    assert lib.slime_ca_destroy(None) == _lib.SLIME_OK
    assert lib.slime_ca_uses_mfma(None) == 0
    assert lib.slime_neural_ca_update(None, None, None, None, 0, None) == _lib.SLIME_EINVAL
    assert lib.slime_ca_get_state(None, None, None, 16) == _lib.SLIME_EINVAL
    assert b"NULL" in lib.slime_ca_last_error()


def test_valid_config_without_gpu_reports_no_device():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is visible; covered by the gpu tests")
    lib = _lib.load()
    h = ctypes.c_void_p()
    rc = lib.slime_ca_create(ctypes.byref(_cfg()), ctypes.byref(h))
    assert rc in (_lib.SLIME_ENODEV, _lib.SLIME_EHIP)
    assert not h.value


def test_probe_library_exports_the_ceiling_probes():
    """libslime_probe.so (measured MFMA/HBM ceilings) is separate from the CA library."""
    path = os.path.join(ROOT, "slime_amd", "libslime_probe.so")
    if not os.path.exists(path):
        pytest.skip("probe library not built")
    lib = ctypes.CDLL(path)
    assert hasattr(lib, "slime_probe_mfma_tflops")
    assert hasattr(lib, "slime_probe_hbm_gbs")
    assert hasattr(lib, "slime_probe_fp64_core")
    ca = _lib.load()
    assert not hasattr(ca, "slime_probe_mfma_tflops")


# ---- the header and a compiled host, as a C or C++ caller uses them ---------------------

@pytest.mark.parametrize("lang", ["c", "c++"])
def test_header_compiles_alone(lang):
    """include/slime_ca.h alone, as C99 and as C++17, with -Wall -Wextra -Werror
    -pedantic: it includes what it uses (size_t) and nothing else is assumed."""
    from tests import binding
    binding.compile_header(lang)


def test_compiled_cpp_host_checks_without_a_gpu():
    """tests/ca_binding.cpp built with g++ against the header and linked to the
    library: its status-code checks (EINVAL for bad configurations and non-finite
    parameters, ENODEV or EHIP for a valid one here) all pass."""
    import subprocess
    from tests import binding
    exe = binding.build_binding()
    r = subprocess.run([exe, "checks"], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("checks ok")


def _param_arrays(cfg, fill=0.01):
    import numpy as np
    C = cfg.H * cfg.D
    g = (cfg.pods, cfg.G, cfg.G, cfg.H) if cfg.growth_per_cell else (cfg.pods, cfg.H)
    return {"WP": np.full((cfg.pods, C, C), fill, np.float32),
            "WI": np.full((cfg.pods, C, C), fill, np.float32),
            "WV": np.full((cfg.pods, C, C), fill, np.float32),
            "K": np.full((cfg.pods, cfg.H, 9), 0.1, np.float32),
            "mu": np.full(g, 0.2, np.float32), "sigma": np.full(g, 0.03, np.float32),
            "M": np.tile(np.eye(cfg.H, dtype=np.float32), (cfg.pods, 1, 1))}


@pytest.mark.parametrize("name,index", [("WP", 0), ("WI", -1), ("WV", 77), ("K", 5), ("M", 3),
                                        ("mu", 1), ("sigma", -1)])
@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -float("inf")])
def test_check_params_rejects_non_finite_entries(name, index, bad):
    """slime_ca_check_params, the checks slime_ca_set_params makes before any upload:
    every array of every pod, per-cell growth included, must be finite."""
    lib = _lib.load()
    cfg = _cfg(B=2, pods=2, growth_per_cell=int(name in ("mu", "sigma")))
    arrs = _param_arrays(cfg)
    p = _lib.Params(*[arrs[k].ctypes.data for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")])
    assert lib.slime_ca_check_params(ctypes.byref(cfg), ctypes.byref(p)) == _lib.SLIME_OK
    arrs[name].reshape(-1)[index] = bad
    rc = lib.slime_ca_check_params(ctypes.byref(cfg), ctypes.byref(p))
    assert rc == _lib.SLIME_EINVAL
    assert name.encode() in lib.slime_ca_last_error() and b"finite" in lib.slime_ca_last_error()


def test_check_params_rejects_zero_sigma_for_the_gaussian_growth_only():
    lib = _lib.load()
    for fn, ok in ((0, True), (1, False), (2, True)):
        cfg = _cfg(growth_fn=fn)
        arrs = _param_arrays(cfg)
        arrs["sigma"][0, 3] = 0.0
        p = _lib.Params(*[arrs[k].ctypes.data for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")])
        rc = lib.slime_ca_check_params(ctypes.byref(cfg), ctypes.byref(p))
        assert rc == (_lib.SLIME_OK if ok else _lib.SLIME_EINVAL), fn


def test_check_params_rejects_null_and_invalid_config():
    lib = _lib.load()
    cfg = _cfg()
    arrs = _param_arrays(cfg)
    p = _lib.Params(*[arrs[k].ctypes.data for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")])
    assert lib.slime_ca_check_params(None, ctypes.byref(p)) == _lib.SLIME_EINVAL
    assert lib.slime_ca_check_params(ctypes.byref(cfg), None) == _lib.SLIME_EINVAL
    p.K = None
    assert lib.slime_ca_check_params(ctypes.byref(cfg), ctypes.byref(p)) == _lib.SLIME_EINVAL
    assert lib.slime_ca_check_params(ctypes.byref(_cfg(G=12)), ctypes.byref(p)) == _lib.SLIME_EINVAL
