"""Component pool on the device: the consumers of the CA fitness.

Mirrors the reference's ComponentPool / PoolEntry (slime/memory/pool.cu:12-30)
as a structure of CUDA tensors and runs its lifecycle operations through
``libslime_ca.so`` (include/slime_ca.h, ``slime_pool_*``): ``init``
(init_pool_kernel, pool.cu:300-320), ``set_fitness`` (the writes of
fitness_computation_kernel, slime/core/organism.cu:204-289, fed by the fused CA
fitness), ``hunger`` (slime/kernels/warp_ca.cu:229-240), ``age``
(pool.cu:162-168), ``cull`` (culling_kernel, organism.cu:590-614), ``spawn``
(spawn_component_kernel, pool.cu:57-121), ``spawn_wave`` (organism.cu:557-587)
and ``evolve`` (component_evolution_kernel without selection, organism.cu:144-201).
"""
from __future__ import annotations

import ctypes

from . import _lib
from .ca import _ptr, _stream, _torch

# The lifecycle's constants (slime/core/organism.cu:19-21; slime/memory/pool.cu:7-9).
FITNESS_THRESHOLD = 0.8
HUNGER_DEATH_THRESHOLD = 0.95
SPAWN_RATE = 0.1
MAX_POOL_SIZE = 256
GENOME_SIZE = 512

FIELDS = ("id", "fitness", "coherence", "hunger", "age", "alive", "genome", "gradients", "counters")


class ComponentPool:
    """``capacity`` entries with ``genome_size`` floats of genome and gradients each,
    as CUDA tensors; ``counters`` holds (active, spawned, culled)."""

    def __init__(self, capacity: int = MAX_POOL_SIZE, genome_size: int = GENOME_SIZE,
                 stream=None):
        torch = _torch()
        self.lib = _lib.load()
        self.capacity, self.genome_size = capacity, genome_size
        dev = "cuda"
        self.id = torch.empty(capacity, dtype=torch.int32, device=dev)
        self.fitness = torch.empty(capacity, dtype=torch.float32, device=dev)
        self.coherence = torch.empty(capacity, dtype=torch.float32, device=dev)
        self.hunger = torch.empty(capacity, dtype=torch.float32, device=dev)
        self.age = torch.empty(capacity, dtype=torch.int32, device=dev)
        self.alive = torch.empty(capacity, dtype=torch.int32, device=dev)
        self.genome = torch.empty((capacity, genome_size), dtype=torch.float32, device=dev)
        self.gradients = torch.empty((capacity, genome_size), dtype=torch.float32, device=dev)
        self.counters = torch.empty(3, dtype=torch.int32, device=dev)
        self._c = _lib.Pool(capacity, genome_size, *[getattr(self, n).data_ptr() for n in FIELDS])
        self.init(stream)

    def _call(self, name: str, *args) -> None:
        _lib.check(getattr(self.lib, name)(ctypes.byref(self._c), *args))

    def init(self, stream=None) -> None:
        self._call("slime_pool_init", _stream(stream))

    def set_fitness(self, fitness, coherence, generation: int, fitness_history=None,
                    coherence_history=None, stream=None) -> None:
        """``fitness``, ``coherence``: [n, heads] (or [n]) float32 CUDA tensors, e.g. the
        per-(batch, head) outputs of ``Pseudopod.fitness`` with batch entry = component."""
        f, c = _as2d(fitness), _as2d(coherence)
        if f.shape != c.shape:
            raise ValueError("fitness and coherence must have the same shape")
        self._call("slime_pool_set_fitness", _ptr(f), _ptr(c), int(f.shape[0]), int(f.shape[1]),
                   generation, _opt(fitness_history), _opt(coherence_history), _stream(stream))

    def age_up(self, stream=None) -> None:
        self._call("slime_pool_age", _stream(stream))

    def cull(self, fitness_threshold: float = FITNESS_THRESHOLD,
             hunger_threshold: float = HUNGER_DEATH_THRESHOLD, stream=None) -> None:
        self._call("slime_pool_cull", ctypes.c_float(fitness_threshold),
                   ctypes.c_float(hunger_threshold), _stream(stream))

    def spawn(self, parent: int, mutation_rate: float = 0.01, stream=None) -> None:
        self._call("slime_pool_spawn", int(parent), ctypes.c_float(mutation_rate), _stream(stream))

    def spawn_wave(self, probability: float, generation: int, stream=None) -> None:
        """``probability`` < 0: the lifecycle's 0.1 exp(-active / 256), computed on the device."""
        self._call("slime_pool_spawn_wave", ctypes.c_float(probability), int(generation),
                   _stream(stream))

    def evolve(self, fitness, coherence, generation: int, fitness_history=None,
               coherence_history=None, stream=None) -> None:
        f, c = _as2d(fitness), _as2d(coherence)
        self._call("slime_pool_evolve", _ptr(f), _ptr(c), int(f.shape[0]), int(f.shape[1]),
                   generation, _opt(fitness_history), _opt(coherence_history), _stream(stream))

    def host(self) -> dict:
        """Host copies of every field (synchronises)."""
        return {n: getattr(self, n).cpu().numpy() for n in FIELDS}

    @property
    def stats(self) -> dict:
        a, s, c = (int(v) for v in self.counters.cpu().tolist())
        return {"active": a, "capacity": self.capacity, "spawned": s, "culled": c}


def hunger(coherence, out=None, stream=None):
    """hunger = 1 - coherence over a float32 CUDA tensor (hunger_kernel)."""
    torch = _torch()
    c = coherence.contiguous()
    if c.dtype != torch.float32 or not c.is_cuda:
        raise ValueError("coherence must be a float32 CUDA tensor")
    out = torch.empty_like(c) if out is None else out
    _lib.check(_lib.load().slime_ca_hunger(_ptr(c), _ptr(out), c.numel(), _stream(stream)))
    return out


def _as2d(t):
    torch = _torch()
    if t.dtype != torch.float32 or not t.is_cuda:
        raise ValueError("fitness inputs must be float32 CUDA tensors")
    t = t.contiguous()
    return t.reshape(t.shape[0], -1) if t.dim() != 1 else t.reshape(-1, 1)


def _opt(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p()


__all__ = ["ComponentPool", "hunger", "FIELDS", "FITNESS_THRESHOLD", "HUNGER_DEATH_THRESHOLD",
           "SPAWN_RATE", "MAX_POOL_SIZE", "GENOME_SIZE"]
