"""ctypes wrapper for the CPU oracle (``oracle/build/libca_oracle.so``).

TEST INFRASTRUCTURE: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only to check
or time the HIP library against it. The product package ``slime_amd`` never
imports it.

Every function takes numpy arrays in the layouts documented in
``oracle/ca_oracle.h`` and returns new numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libca_oracle.so")
_lib = None


class _Cfg(ctypes.Structure):
    _fields_ = [
        ("B", ctypes.c_int),
        ("G", ctypes.c_int),
        ("H", ctypes.c_int),
        ("D", ctypes.c_int),
        ("pods", ctypes.c_int),
        ("growth_per_cell", ctypes.c_int),
        ("pvi_chain", ctypes.c_int),
        ("dt", ctypes.c_float),
        ("growth_fn", ctypes.c_int),
        ("conservation", ctypes.c_int),
    ]


@dataclass
class OracleConfig:
    B: int
    G: int
    H: int
    D: int
    pods: int = 1
    growth_per_cell: bool = False
    pvi_chain: int = 0  # 0 parallel, 1 chained, 2 chained with the 3x3 perception sum
    dt: float = 0.1
    growth_fn: int = 0  # 0 bell, 1 Gaussian, 2 shipped U exp(-U^2)
    conservation: int = 0  # 0 per (b, head); 1 per (cell, head) first

    @property
    def C(self) -> int:
        return self.H * self.D

    def c(self) -> _Cfg:
        return _Cfg(self.B, self.G, self.H, self.D, self.pods, int(self.growth_per_cell),
                    int(self.pvi_chain), self.dt, int(self.growth_fn), int(self.conservation))


def build() -> str:
    """Compile the oracle with its Makefile (g++ only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for name in ("oracle_project", "oracle_potential", "oracle_growth", "oracle_attention",
                     "oracle_propagate", "oracle_mix", "oracle_conserve", "oracle_step",
                     "oracle_gram", "oracle_coherence", "oracle_fitness", "oracle_step_backward"):
            getattr(_lib, name).restype = ctypes.c_int
        _lib.oracle_jacobi_eigs.restype = ctypes.c_int
        _lib.oracle_effective_rank.restype = ctypes.c_double
        _lib.oracle_init_from_field.restype = ctypes.c_int
        _lib.oracle_field_from_state.restype = ctypes.c_int
        _lib.oracle_num_threads.restype = ctypes.c_int
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its configuration")


def _state(cfg: OracleConfig) -> tuple:
    return (cfg.B, cfg.G, cfg.G, cfg.C)


def project(cfg, X, WP, WI, WV):
    X, WP, WI, WV = map(_f32, (X, WP, WI, WV))
    P, I, V = (np.empty(_state(cfg), np.float32) for _ in range(3))
    _check(lib().oracle_project(ctypes.byref(cfg.c()), _p(X), _p(WP), _p(WI), _p(WV), _p(P),
                                _p(I), _p(V)), "project")
    return P, I, V


def potential(cfg, X, K):
    X, K = _f32(X), _f32(K)
    U = np.empty(_state(cfg), np.float32)
    _check(lib().oracle_potential(ctypes.byref(cfg.c()), _p(X), _p(K), _p(U)), "potential")
    return U


def growth(cfg, U, mu, sigma):
    U, mu, sigma = map(_f32, (U, mu, sigma))
    g = np.empty(_state(cfg), np.float32)
    _check(lib().oracle_growth(ctypes.byref(cfg.c()), _p(U), _p(mu), _p(sigma), _p(g)), "growth")
    return g


def attention(cfg, P, I):
    P, I = _f32(P), _f32(I)
    A = np.empty((cfg.B, cfg.G, cfg.G, cfg.H, 9), np.float32)
    _check(lib().oracle_attention(ctypes.byref(cfg.c()), _p(P), _p(I), _p(A)), "attention")
    return A


def propagate(cfg, A, V):
    A, V = _f32(A), _f32(V)
    Vt = np.empty(_state(cfg), np.float32)
    _check(lib().oracle_propagate(ctypes.byref(cfg.c()), _p(A), _p(V), _p(Vt)), "propagate")
    return Vt


def mix(cfg, X, g, Vt, M):
    X, g, Vt, M = map(_f32, (X, g, Vt, M))
    Y = np.empty(_state(cfg), np.float32)
    _check(lib().oracle_mix(ctypes.byref(cfg.c()), _p(X), _p(g), _p(Vt), _p(M), _p(Y)), "mix")
    return Y


def conserve(cfg, X, Y):
    X = _f32(X)
    Y = np.array(Y, dtype=np.float32, copy=True)
    mi = np.empty((cfg.B, cfg.H), np.float64)
    mo = np.empty((cfg.B, cfg.H), np.float64)
    _check(lib().oracle_conserve(ctypes.byref(cfg.c()), _p(X), _p(Y), _p(mi), _p(mo)),
           "conserve")
    return Y, mi, mo


def step(cfg, X, params, n_steps=1):
    """Full S1-S7 step(s). ``params`` holds WP, WI, WV, K, mu, sigma, M."""
    X = _f32(X)
    arrs = [_f32(params[k]) for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")]
    out = np.empty(_state(cfg), np.float32)
    mi = np.zeros((cfg.B, cfg.H), np.float64)
    mo = np.zeros((cfg.B, cfg.H), np.float64)
    _check(lib().oracle_step(ctypes.byref(cfg.c()), _p(X), *[_p(a) for a in arrs], _p(out),
                             ctypes.c_int(n_steps), _p(mi), _p(mo)), "step")
    return out, mi, mo


def step_loss(cfg, X, params, T):
    """Loss mean((step(X) - T)^2) of one step (parallel projections)."""
    X, T = _f32(X), _f32(T)
    arrs = [_f32(params[k]) for k in ("WP", "WI", "WV", "K", "mu", "sigma", "M")]
    loss = ctypes.c_double()
    null = ctypes.c_void_p()
    _check(lib().oracle_step_backward(ctypes.byref(cfg.c()), _p(X), *[_p(a) for a in arrs], _p(T),
                                      ctypes.byref(loss), *([null] * 8)), "step_backward")
    return loss.value


def step_backward(cfg, X, params, T):
    """Loss of one step and its gradients: returns (loss, grads) with grads keyed
    X, WP, WI, WV, K, mu, sigma, M (shapes as the inputs)."""
    X, T = _f32(X), _f32(T)
    names = ("WP", "WI", "WV", "K", "mu", "sigma", "M")
    arrs = [_f32(params[k]) for k in names]
    grads = {"X": np.empty_like(X)}
    for k, a in zip(names, arrs):
        grads[k] = np.empty_like(a)
    loss = ctypes.c_double()
    _check(lib().oracle_step_backward(ctypes.byref(cfg.c()), _p(X), *[_p(a) for a in arrs], _p(T),
                                      ctypes.byref(loss), _p(grads["X"]),
                                      *[_p(grads[k]) for k in names]), "step_backward")
    return loss.value, grads


def gram(cfg, X):
    X = _f32(X)
    A = np.empty((cfg.B, cfg.H, cfg.D, cfg.D), np.float64)
    _check(lib().oracle_gram(ctypes.byref(cfg.c()), _p(X), _p(A)), "gram")
    return A


def jacobi_eigs(A, max_sweeps=30, tol=1e-6):
    A = np.ascontiguousarray(A, dtype=np.float64)
    n = A.shape[0]
    eig = np.empty(n, np.float64)
    sweeps = lib().oracle_jacobi_eigs(_p(A), ctypes.c_int(n), _p(eig), ctypes.c_int(max_sweeps),
                                      ctypes.c_double(tol))
    if sweeps < 0:
        raise ValueError("oracle jacobi rejected its input")
    return eig, sweeps


def effective_rank(sv):
    sv = np.ascontiguousarray(sv, dtype=np.float64)
    return lib().oracle_effective_rank(_p(sv), ctypes.c_int(sv.shape[0]))


def coherence(cfg, hist):
    hist = _f32(hist)
    coh = np.empty((cfg.B, cfg.H), np.float64)
    _check(lib().oracle_coherence(ctypes.byref(cfg.c()), _p(hist), ctypes.c_int(hist.shape[0]),
                                  _p(coh)), "coherence")
    return coh


def fitness(cfg, hist):
    hist = _f32(hist)
    er, coh, fit = (np.empty((cfg.B, cfg.H), np.float64) for _ in range(3))
    _check(lib().oracle_fitness(ctypes.byref(cfg.c()), _p(hist), ctypes.c_int(hist.shape[0]),
                                _p(er), _p(coh), _p(fit)), "fitness")
    return er, coh, fit


def init_from_field(conc, C):
    conc = _f32(conc)
    G = conc.shape[0]
    X = np.empty((G, G, C), np.float32)
    _check(lib().oracle_init_from_field(G, C, _p(conc), _p(X)), "init_from_field")
    return X


def field_from_state(X):
    X = _f32(X)
    G, C = X.shape[0], X.shape[-1]
    conc = np.empty((G, G), np.float32)
    _check(lib().oracle_field_from_state(G, C, _p(X), _p(conc)), "field_from_state")
    return conc


def num_threads() -> int:
    return lib().oracle_num_threads()


# ---- component pool (pool_oracle.cpp) -------------------------------------------------
class _PoolC(ctypes.Structure):
    _fields_ = [("capacity", ctypes.c_int), ("genome_size", ctypes.c_int)] + [
        (n, ctypes.c_void_p) for n in ("id", "fitness", "coherence", "hunger", "age", "alive",
                                       "genome", "gradients", "counters")]


class Pool:
    """Host component pool in the layout of ``slime_pool`` (numpy arrays); the
    methods run the oracle's restatement of the reference's pool kernels."""

    FIELDS = ("id", "fitness", "coherence", "hunger", "age", "alive", "genome", "gradients", "counters")

    def __init__(self, capacity: int = 256, genome_size: int = 512):
        self.capacity, self.genome_size = capacity, genome_size
        self.id = np.full(capacity, -1, np.int32)
        self.fitness = np.zeros(capacity, np.float32)
        self.coherence = np.zeros(capacity, np.float32)
        self.hunger = np.full(capacity, 0.5, np.float32)
        self.age = np.zeros(capacity, np.int32)
        self.alive = np.zeros(capacity, np.int32)
        self.genome = np.zeros((capacity, genome_size), np.float32)
        self.gradients = np.zeros((capacity, genome_size), np.float32)
        self.counters = np.zeros(3, np.int32)

    def _c(self) -> _PoolC:
        return _PoolC(self.capacity, self.genome_size, *[getattr(self, n).ctypes.data for n in self.FIELDS])

    def copy(self) -> "Pool":
        q = Pool(self.capacity, self.genome_size)
        for n in self.FIELDS:
            setattr(q, n, getattr(self, n).copy())
        return q

    def init(self) -> None:
        lib().oracle_pool_init(ctypes.byref(self._c()))

    def set_fitness(self, fitness, coherence, n: int, heads: int, generation: int,
                    fitness_history=None, coherence_history=None) -> None:
        f, c = _f32(fitness), _f32(coherence)
        fh = fitness_history.ctypes.data if fitness_history is not None else None
        ch = coherence_history.ctypes.data if coherence_history is not None else None
        lib().oracle_pool_set_fitness(ctypes.byref(self._c()), _p(f), _p(c), n, heads, generation,
                                      ctypes.c_void_p(fh), ctypes.c_void_p(ch))

    def age_up(self) -> None:
        lib().oracle_pool_age(ctypes.byref(self._c()))

    def cull(self, fitness_threshold: float, hunger_threshold: float) -> None:
        lib().oracle_pool_cull(ctypes.byref(self._c()), ctypes.c_float(fitness_threshold),
                               ctypes.c_float(hunger_threshold))

    def spawn(self, parent: int, rate: float) -> None:
        lib().oracle_pool_spawn(ctypes.byref(self._c()), parent, ctypes.c_float(rate))

    def spawn_wave(self, probability: float, generation: int) -> float:
        fn = lib().oracle_pool_spawn_wave
        fn.restype = ctypes.c_float
        return fn(ctypes.byref(self._c()), ctypes.c_float(probability), generation)

    def evolve(self, fitness, coherence, n: int, heads: int, generation: int,
               fitness_history=None, coherence_history=None) -> None:
        f, c = _f32(fitness), _f32(coherence)
        fh = fitness_history.ctypes.data if fitness_history is not None else None
        ch = coherence_history.ctypes.data if coherence_history is not None else None
        lib().oracle_pool_evolve(ctypes.byref(self._c()), _p(f), _p(c), n, heads, generation,
                                 ctypes.c_void_p(fh), ctypes.c_void_p(ch))


def hunger(coherence) -> np.ndarray:
    c = _f32(coherence)
    out = np.empty_like(c)
    lib().oracle_hunger(_p(c), _p(out), c.size)
    return out


class Xorshift128p:
    """The oracle's xorshift128+ stream (float mapping and Box-Muller of the reference)."""

    def __init__(self, s0: int, s1: int):
        self.s = (ctypes.c_ulonglong * 2)(s0 & (2**64 - 1), s1 & (2**64 - 1))

    def next(self) -> float:
        fn = lib().oracle_xorshift_next
        fn.restype = ctypes.c_float
        return fn(ctypes.byref(self.s, 0), ctypes.byref(self.s, 8))

    def gaussian(self) -> float:
        fn = lib().oracle_xorshift_gaussian
        fn.restype = ctypes.c_float
        return fn(ctypes.byref(self.s, 0), ctypes.byref(self.s, 8))

    @property
    def state(self) -> tuple:
        return int(self.s[0]), int(self.s[1])
