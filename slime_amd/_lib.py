"""ctypes binding of ``libslime_ca.so`` (declared in ``include/slime_ca.h``).

Loading fails loudly: there is no Python or CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libslime_ca.so")

SLIME_OK = 0
SLIME_EINVAL = -1
SLIME_ENOMEM = -2
SLIME_EHIP = -3
SLIME_ENODEV = -4
SLIME_ESTATE = -5
SLIME_ENONFINITE = -6
SLIME_F32 = 0
SLIME_BF16 = 1

# Every symbol include/slime_ca.h declares.
EXPORTS = (
    "slime_ca_create", "slime_ca_destroy", "slime_ca_set_params", "slime_ca_project",
    "slime_ca_flow_lenia", "slime_ca_step", "slime_ca_mass", "slime_ca_fitness",
    "slime_ca_fitness_sweeps", "slime_ca_init_from_field", "slime_ca_field_from_state",
    "slime_ca_get_state",
    "slime_ca_uses_mfma", "slime_ca_set_timing", "slime_ca_timings", "slime_ca_last_error",
    "slime_neural_ca_update", "slime_ca_backward", "slime_pool_init", "slime_pool_set_fitness",
    "slime_ca_hunger", "slime_pool_age", "slime_pool_cull", "slime_pool_spawn", "slime_pool_spawn_wave",
    "slime_pool_evolve", "slime_snapshot_json", "slime_ca_fitness_static", "slime_ca_rollout",
    "slime_ca_fitness_scaled", "slime_ca_check_params",
)


class Config(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("G", ctypes.c_int), ("H", ctypes.c_int),
                ("D", ctypes.c_int), ("dtype", ctypes.c_int), ("dt", ctypes.c_float),
                ("growth_per_cell", ctypes.c_int), ("pods", ctypes.c_int),
                ("pvi_chain", ctypes.c_int), ("growth_fn", ctypes.c_int),
                ("conservation", ctypes.c_int)]


class Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("WP", "WI", "WV", "K", "mu", "sigma", "M")]


class MultiHeadCAState(ctypes.Structure):
    """slime_multihead_ca_state: the per-generation buffers of MultiHeadCAState."""
    _fields_ = [("mass_buffer", ctypes.c_void_p), ("ca_input", ctypes.c_void_p),
                ("ca_output", ctypes.c_void_p)]


class Grads(ctypes.Structure):
    """slime_ca_grads: device fp32 parameter-gradient pointers (NULL allowed)."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("WP", "WI", "WV", "K", "mu", "sigma", "M")]


class Pool(ctypes.Structure):
    """slime_pool: device arrays of the component pool."""
    _fields_ = [("capacity", ctypes.c_int), ("genome_size", ctypes.c_int)] + [
        (n, ctypes.c_void_p) for n in ("id", "fitness", "coherence", "hunger", "age", "alive",
                                       "genome", "gradients", "counters")]


class SlimeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"slime_ca error {code}: {msg}")
        self.code = code


_lib = None


def load() -> ctypes.CDLL:
    """Loads the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python -m slime_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, ip, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float
    sig = {
        "slime_ca_create": [ctypes.POINTER(Config), ctypes.POINTER(ctypes.c_void_p)],
        "slime_ca_destroy": [vp],
        "slime_ca_set_params": [vp, ctypes.POINTER(Params)],
        "slime_ca_check_params": [ctypes.POINTER(Config), ctypes.POINTER(Params)],
        "slime_ca_project": [vp, vp, vp, vp, vp, vp],
        "slime_ca_flow_lenia": [vp, vp, vp, vp, vp, vp, vp],
        "slime_ca_step": [vp, vp, vp, i, vp],
        "slime_ca_mass": [vp, vp, vp],
        "slime_ca_fitness": [vp, vp, i, vp, vp, vp, vp],
        "slime_ca_fitness_sweeps": [vp, vp],
        "slime_ca_init_from_field": [vp, vp, vp, vp],
        "slime_ca_field_from_state": [vp, vp, vp, vp],
        "slime_ca_get_state": [vp, vp, vp, i],
        "slime_ca_uses_mfma": [vp],
        "slime_ca_set_timing": [vp, i],
        "slime_ca_timings": [vp, vp, vp, vp, vp],
        "slime_ca_last_error": [],
        "slime_neural_ca_update": [vp, ctypes.POINTER(MultiHeadCAState), vp, vp, i, vp],
        "slime_ca_backward": [vp, vp, vp, vp, ctypes.POINTER(Grads), ctypes.POINTER(ctypes.c_double),
                              vp],
        "slime_pool_init": [ctypes.POINTER(Pool), vp],
        "slime_pool_set_fitness": [ctypes.POINTER(Pool), vp, vp, i, i, i, vp, vp, vp],
        "slime_ca_hunger": [vp, vp, i, vp],
        "slime_pool_age": [ctypes.POINTER(Pool), vp],
        "slime_pool_cull": [ctypes.POINTER(Pool), f, f, vp],
        "slime_pool_spawn": [ctypes.POINTER(Pool), i, f, vp],
        "slime_pool_spawn_wave": [ctypes.POINTER(Pool), f, i, vp],
        "slime_pool_evolve": [ctypes.POINTER(Pool), vp, vp, i, i, i, vp, vp, vp],
        "slime_snapshot_json": [vp, vp, ctypes.POINTER(Pool), i, ctypes.c_double, ctypes.c_char_p,
                                ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_char_p if name == "slime_ca_last_error" else ip
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != SLIME_OK:
        msg = load().slime_ca_last_error().decode(errors="replace")
        raise SlimeError(rc, msg)
