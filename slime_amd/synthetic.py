"""Seeded synthetic inputs for the CA step, one recipe per benchmark configuration.

All draws use ``numpy.random.default_rng(seed)`` (PCG64), so the same seed gives
the same arrays on every machine. Distributions follow the configurations the
benchmark is quoted on:

  c1  B1, G32, H8, D8, fp32: X ~ U[0,1); K, W ~ N(0, 0.1); mu ~ U[0.1, 0.3],
      sigma ~ U[0.01, 0.05] per head
  c2  B1, G128, H8, D64, fp32: X ~ U[0,1) with 5 % sparse blobs; W, K ~ N(0, 0.05);
      mu, sigma per cell and head
  c3  B64, G128, H8, D64, bf16: as c2 but mu, sigma per head
  c4  16 pods (batch entry = pod), G128, D64, bf16, independent weights per pod
  c5  B4, G512, D64, bf16

Head mixing M is the identity plus N(0, 0.01) noise, as init_multihead_ca_kernel
sets it (slime/core/pseudopod.cu:419-426).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class CAConfig:
    name: str
    B: int
    G: int
    H: int
    D: int
    dtype: str
    steps: int
    w_std: float
    growth_per_cell: bool = False
    pods: int = 1
    blobs: bool = False
    dt: float = 0.1

    @property
    def C(self) -> int:
        return self.H * self.D

    @property
    def cell_updates_per_step(self) -> int:
        return self.B * self.G * self.G


CONFIGS = {
    "c1": CAConfig("c1", B=1, G=32, H=8, D=8, dtype="fp32", steps=1, w_std=0.1),
    "c2": CAConfig("c2", B=1, G=128, H=8, D=64, dtype="fp32", steps=100, w_std=0.05,
                   growth_per_cell=True, blobs=True),
    "c3": CAConfig("c3", B=64, G=128, H=8, D=64, dtype="bf16", steps=10, w_std=0.05, blobs=True),
    "c4": CAConfig("c4", B=16, G=128, H=8, D=64, dtype="bf16", steps=8, w_std=0.05, pods=16,
                   blobs=True),
    "c5": CAConfig("c5", B=4, G=512, H=8, D=64, dtype="bf16", steps=1, w_std=0.05, blobs=True),
}


def make_params(cfg: CAConfig, seed: int = 1) -> dict:
    rng = np.random.default_rng(seed)
    C, H, P = cfg.C, cfg.H, cfg.pods
    f32 = np.float32
    p = {
        "WP": rng.normal(0.0, cfg.w_std, (P, C, C)).astype(f32),
        "WI": rng.normal(0.0, cfg.w_std, (P, C, C)).astype(f32),
        "WV": rng.normal(0.0, cfg.w_std, (P, C, C)).astype(f32),
        "K": rng.normal(0.0, cfg.w_std, (P, H, 9)).astype(f32),
        "M": (np.eye(H, dtype=f32)[None] + rng.normal(0.0, 0.01, (P, H, H))).astype(f32),
    }
    g = (P, cfg.G, cfg.G, H) if cfg.growth_per_cell else (P, H)
    p["mu"] = rng.uniform(0.1, 0.3, g).astype(f32)
    p["sigma"] = rng.uniform(0.01, 0.05, g).astype(f32)
    return p


def make_state(cfg: CAConfig, seed: int = 2, B: int | None = None) -> np.ndarray:
    """[B, G, G, C] fp32: U[0,1) plus, when ``cfg.blobs``, discs of radius 4 set to
    1.0 at random centres, enough of them to cover about 5 % of the cells."""
    B = cfg.B if B is None else B
    rng = np.random.default_rng(seed)
    X = rng.random((B, cfg.G, cfg.G, cfg.C), dtype=np.float32)
    if cfg.blobs:
        r = 4
        n_blobs = max(1, int(round(0.05 * cfg.G * cfg.G / (np.pi * r * r))))
        dy, dx = np.mgrid[-r:r + 1, -r:r + 1]
        disc = (dy * dy + dx * dx) <= r * r
        oy, ox = dy[disc], dx[disc]
        for b in range(B):
            cy = rng.integers(0, cfg.G, n_blobs)
            cx = rng.integers(0, cfg.G, n_blobs)
            for y0, x0 in zip(cy, cx):
                X[b, (y0 + oy) % cfg.G, (x0 + ox) % cfg.G, :] = 1.0
    return X


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)
