"""Writes and checks the committed fixtures under tests/golden/.

  jacobi_eigs.npz  symmetric matrices with eigenvalues fixed by construction
                   (A = Q diag(lam) Q^T, Q orthogonal from a QR factorisation)
                   and LAPACK's eigvalsh of the same A. These pin the oracle's
                   Jacobi solver independently of it.
  c1_step.json     the oracle's one-step output on configuration c1 (B1, G32, H8,
                   D8, fp32, seeds 1/2) at 512 sampled elements, plus checksums
                   and per-head masses. Written by the oracle itself, so it is a
                   regression anchor for the oracle and a fixture for the GPU
                   parity test, not an independent pin.

The reference ships no golden vectors for this path, so nothing here comes from
it. Run ``python -m tests.golden.make_golden`` to regenerate (the repo root must
be on sys.path).
"""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
JACOBI = os.path.join(HERE, "jacobi_eigs.npz")
C1 = os.path.join(HERE, "c1_step.json")


def _jacobi_cases():
    cases = []
    rng = np.random.default_rng(20240601)
    for n, kind in ((8, "spread"), (16, "spread"), (64, "gram"), (64, "lowrank"), (64, "cluster")):
        Q, _ = np.linalg.qr(rng.normal(size=(n, n)))
        if kind == "spread":
            lam = np.sort(rng.uniform(0.01, 3.0, n))[::-1]
        elif kind == "gram":   # like a Gram matrix of U[0,1) data: one large, many ~1/12
            lam = np.concatenate([[n * 0.25 + 1 / 12], np.full(n - 1, 1 / 12) * rng.uniform(0.5, 1.5, n - 1)])
            lam = np.sort(lam)[::-1]
        elif kind == "lowrank":
            lam = np.concatenate([np.sort(rng.uniform(0.5, 2.0, 4))[::-1], np.zeros(n - 4)])
        else:                  # clustered eigenvalues
            lam = np.sort(1.0 + 1e-3 * rng.normal(size=n))[::-1]
        A = (Q * lam) @ Q.T
        A = 0.5 * (A + A.T)
        cases.append((A, lam, np.sort(np.linalg.eigvalsh(A))[::-1]))
    return cases


def write_jacobi():
    cases = _jacobi_cases()
    arrs = {}
    for i, (A, lam, eig) in enumerate(cases):
        arrs[f"A{i}"] = A
        arrs[f"lam{i}"] = lam
        arrs[f"eig{i}"] = eig
    np.savez_compressed(JACOBI, **arrs)


def load_jacobi():
    with np.load(JACOBI, allow_pickle=False) as z:
        n = len([k for k in z.files if k.startswith("A")])
        return [(z[f"A{i}"], z[f"lam{i}"], z[f"eig{i}"]) for i in range(n)]


def _c1_inputs():
    from slime_amd.synthetic import CONFIGS, make_params, make_state
    cfg = CONFIGS["c1"]
    return cfg, make_params(cfg, seed=1), make_state(cfg, seed=2)


def _oracle_cfg(cfg):
    from oracle import OracleConfig
    return OracleConfig(B=cfg.B, G=cfg.G, H=cfg.H, D=cfg.D, pods=cfg.pods,
                        growth_per_cell=cfg.growth_per_cell, dt=cfg.dt)


def _summary(Y: np.ndarray, mi, mo) -> dict:
    flat = Y.astype(np.float64).ravel()
    idx = np.random.default_rng(99).choice(flat.size, 512, replace=False)
    w = np.cos(np.arange(flat.size) * 0.001)
    return {
        "idx": idx.tolist(), "values": flat[idx].tolist(),
        "sum": float(flat.sum()), "sumsq": float((flat * flat).sum()), "wsum": float((w * flat).sum()),
        "mass_in": np.asarray(mi).tolist(), "mass_out": np.asarray(mo).tolist(),
    }


def write_c1(oracle):
    cfg, p, X = _c1_inputs()
    Y, mi, mo = oracle.step(_oracle_cfg(cfg), X, p, 1)
    out = {"config": "c1", "param_seed": 1, "state_seed": 2, "n_steps": 1, **_summary(Y, mi, mo)}
    with open(C1, "w") as f:
        json.dump(out, f)


def load_c1() -> dict:
    with open(C1) as f:
        return json.load(f)


def check_c1(Y: np.ndarray, mi=None, mo=None, tol: float = 1e-5) -> None:
    g = load_c1()
    flat = np.asarray(Y, dtype=np.float64).ravel()
    vals = np.array(g["values"])
    scale = np.max(np.abs(vals))
    err = np.max(np.abs(flat[np.array(g["idx"])] - vals)) / scale
    assert err <= tol, f"c1 sampled values differ: normalised error {err:.3e} > {tol}"
    n = flat.size
    assert abs(flat.sum() - g["sum"]) <= tol * np.abs(flat).sum()
    assert abs((flat * flat).sum() - g["sumsq"]) <= 2 * tol * g["sumsq"]
    w = np.cos(np.arange(n) * 0.001)
    assert abs((w * flat).sum() - g["wsum"]) <= tol * np.abs(flat).sum()
    if mi is not None:
        np.testing.assert_allclose(mi, np.array(g["mass_in"]), rtol=1e-6)
    if mo is not None:
        np.testing.assert_allclose(mo, np.array(g["mass_out"]), rtol=1e-6)


def check_golden(oracle) -> None:
    cfg, p, X = _c1_inputs()
    Y, mi, mo = oracle.step(_oracle_cfg(cfg), X, p, 1)
    check_c1(Y, mi, mo, tol=1e-7)
    for A, lam, eig in load_jacobi():
        got, sweeps = oracle.jacobi_eigs(A)
        assert sweeps <= 30
        # Rotations are skipped for |a_pq| <= 1e-6 and the sweep loop stops once
        # sum |a_pq| < 1e-6 n, so each diagonal entry is within 1e-6 n of an
        # eigenvalue (Gershgorin); a wrong rotation would be off by O(1).
        bound = 1e-6 * A.shape[0]
        np.testing.assert_allclose(got, eig, rtol=0, atol=bound)
        np.testing.assert_allclose(got, lam, rtol=0, atol=bound)


if __name__ == "__main__":
    import oracle as o
    o.build()
    write_jacobi()
    write_c1(o)
    check_golden(o)
    print("wrote", JACOBI, C1)
