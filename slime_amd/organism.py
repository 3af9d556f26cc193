"""The organism's host generation loop over the CA, with evolution.json snapshots.

Replaces the device-side orchestration of the CA path: ``run_organism``
(slime/runtime.cu:386-411) launches ``organism_lifecycle_kernel`` per generation,
which launches ``neural_ca_update_kernel`` (slime/core/organism.cu:113-120) by
dynamic parallelism, and every 100 generations appends ``extract_system_state``
(slime/extract_state.cu:64-184) to ``evolution.json``. Here the host calls
``slime_neural_ca_update`` once per generation on one stream and
``slime_snapshot_json`` for the records; the chemical field, the CA buffers of
``MultiHeadCAState`` and the effective-rank history stay on the device.
"""
from __future__ import annotations

import ctypes
import time

from . import _lib
from .ca import Pseudopod, _ptr, _torch

SNAPSHOT_EVERY = 100  # slime/runtime.cu:401
MAX_GENERATIONS = 10000


class Organism:
    """One organism's CA (a B = 1 ``Pseudopod``), its chemical field and histories.

    ``params``: CA parameters as for ``Pseudopod.set_params``; ``concentration``:
    the initial [G, G] chemical field (host or device); ``pool``: an optional
    ``ComponentPool`` whose counters the snapshots report."""

    def __init__(self, params: dict, concentration, G: int = 128, H: int = 8, D: int = 64,
                 dtype: str = "fp32", pool=None, max_generations: int = MAX_GENERATIONS):
        torch = _torch()
        self.ca = Pseudopod(1, G, H, D, dtype=dtype)
        self.ca.set_params(params)
        self.G, self.H, self.C = G, H, H * D
        self.conc = torch.as_tensor(concentration, dtype=torch.float32).to("cuda").contiguous()
        if tuple(self.conc.shape) != (G, G):
            raise ValueError(f"concentration must be [{G}, {G}]")
        self.ca_input = torch.empty((G, G, self.C), dtype=self.ca.torch_dtype, device="cuda")
        self.ca_output = torch.empty_like(self.ca_input)
        self.mass_buffer = torch.zeros(H, dtype=torch.float32, device="cuda")
        self.effective_rank_history = torch.zeros(max_generations, dtype=torch.float32,
                                                  device="cuda")
        self.pool = pool

    def close(self) -> None:
        self.ca.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def generation(self, gen: int, stream=None) -> None:
        """One generation of the CA (neural_ca_update_kernel's sequence)."""
        self.ca.neural_ca_update(self.conc, self.ca_input, self.ca_output,
                                 self.effective_rank_history, gen, mass_buffer=self.mass_buffer,
                                 stream=stream)

    def snapshot(self, gen: int, elapsed: float) -> str:
        """One evolution.json record of the current state (synchronous)."""
        torch = _torch()
        torch.cuda.synchronize()
        lib = self.ca.lib
        pool = ctypes.byref(self.pool._c) if self.pool is not None else None
        n = ctypes.c_size_t(0)
        cap = 8192
        while True:
            buf = ctypes.create_string_buffer(cap)
            rc = lib.slime_snapshot_json(self.ca._h, _ptr(self.conc), pool, int(gen),
                                         float(elapsed), buf, cap, ctypes.byref(n))
            if rc == _lib.SLIME_EINVAL and n.value + 1 > cap:
                cap = n.value + 1
                continue
            _lib.check(rc)
            return buf.value.decode()

    def run(self, n_generations: int, json_path: str | None = None,
            snapshot_every: int = SNAPSHOT_EVERY, start: int = 0) -> list:
        """Generations start .. start + n - 1; every ``snapshot_every``-th generation
        (gen % snapshot_every == 0) is recorded. Returns the records and, with
        ``json_path``, writes them as a JSON array (run_organism's file)."""
        if start + n_generations > self.effective_rank_history.numel():
            raise ValueError("more generations than the effective-rank history holds")
        records = []
        t0 = time.perf_counter()
        for gen in range(start, start + n_generations):
            self.generation(gen)
            if gen % snapshot_every == 0:
                records.append(self.snapshot(gen, time.perf_counter() - t0))
        if json_path is not None:
            with open(json_path, "w") as f:
                f.write("[\n" + ",\n".join(records) + "\n]\n")
        return records


__all__ = ["Organism", "SNAPSHOT_EVERY", "MAX_GENERATIONS"]
