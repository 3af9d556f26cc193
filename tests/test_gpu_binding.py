"""The compiled C++ host of the library (tests/ca_binding.cpp, built by
tests/binding.py): the binding a reference maintainer would add, run as its own
process on the GPU. Its weights are the reference's per-head tensors
(MultiHeadCAState, slime/core/pseudopod.cu:29-38) embedded in C++, and its engine
runs the reference's own S1 (pvi_chain 2: the 3x3 neighbourhood sum before the
perception product, then the chain, pseudopod.cu:62-119). The result is checked
against the oracle's init -> step -> field sequence with the same tensors embedded
by slime_amd.refweights."""
import json
import os
import subprocess

import numpy as np
import pytest

from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H, D, CHANNELS, HIDDEN = 8, 64, 512, 256


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _binary():
    from tests import binding
    if not os.path.exists(binding.BINDING):
        pytest.fail("tests/_build/ca_binding is not built (run __graft_entry__.build())")
    return binding.BINDING


def test_binding_checks_on_the_gpu():
    print("[case] ca_binding checks", flush=True)
    r = subprocess.run([_binary(), "checks"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stderr
    assert "create(valid) is OK on a GPU" in r.stdout
    assert "set_params rejects the Inf weight" in r.stdout
    assert r.stdout.strip().endswith("checks ok")


def test_binding_generations_match_the_oracle(oracle, tmp_path):
    from slime_amd.refweights import from_reference_weights
    G, gens, chain = 32, 3, 2
    r = np.random.default_rng(17)
    f32 = np.float32
    perception = r.normal(0, 0.05, (H, CHANNELS, HIDDEN)).astype(f32)
    interaction = r.normal(0, 0.05, (H, CHANNELS, HIDDEN)).astype(f32)
    value = r.normal(0, 0.05, (H, HIDDEN, CHANNELS)).astype(f32)
    mixing = (np.eye(H) + r.normal(0, 0.01, (H, H))).astype(f32)
    flow = r.normal(0, 0.1, (H, 3, 3)).astype(f32)
    mu = r.uniform(0.1, 0.3, H).astype(f32)
    sigma = r.uniform(0.01, 0.05, H).astype(f32)
    conc0 = r.random((G, G), dtype=f32)
    src = tmp_path / "in.bin"
    with open(src, "wb") as f:
        np.array([G, gens, chain], np.int32).tofile(f)
        for a in (perception, interaction, value, mixing, flow, mu, sigma, conc0):
            a.tofile(f)
    out, js = tmp_path / "out.bin", tmp_path / "snapshot.json"
    print(f"[case] ca_binding generation G={G} gens={gens} pvi_chain={chain}", flush=True)
    res = subprocess.run([_binary(), "generation", str(src), str(out), str(js)], capture_output=True,
                         text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stderr
    assert "generation ok" in res.stdout
    C = H * D
    o = np.fromfile(out, dtype=f32)
    sizes = [G * G, H, gens, G * G * C, G * G * C]
    parts = np.split(o, np.cumsum(sizes)[:-1])
    assert o.size == sum(sizes)
    conc, mass, erank, xin, xout = parts
    xin, xout = xin.reshape(G, G, C), xout.reshape(G, G, C)

    p = from_reference_weights(perception, interaction, value, mixing, flow)
    p["mu"], p["sigma"] = mu[None], sigma[None]
    ocfg = oracle.OracleConfig(B=1, G=G, H=H, D=D, pvi_chain=chain)
    # the oracle's generations from the same starting field
    c = conc0
    for _ in range(gens):
        X = oracle.init_from_field(c, C)
        Y, _, mo = oracle.step(ocfg, X[None], p, 1)
        c = oracle.field_from_state(Y[0])
    # The field is a channel mean that cancels heavily (conc * sin(0.1 c)), so the
    # fp32 differences of each generation grow through the chain: the chained input
    # and field are held to 1e-4, each generation on its own input to 1e-5.
    assert norm_err(xin, X) <= 1e-4
    # last generation: the device's own input, stepped by the oracle
    Yd, _, mo_d = oracle.step(ocfg, xin[None], p, 1)
    err = norm_err(xout, Yd[0])
    print(f"  last generation: ca_output normalised error {err:.3e}")
    assert err <= 1e-5
    scale = np.abs(Yd[0]).mean(axis=-1)
    assert np.max(np.abs(conc.reshape(G, G) - oracle.field_from_state(Yd[0])) / scale) <= 1e-5
    assert np.max(np.abs(conc.reshape(G, G) - c) / np.abs(Y[0]).mean(axis=-1)) <= 1e-4
    absmass = np.abs(xin.astype(np.float64)).reshape(-1, H, D).sum(axis=(0, 2))
    assert np.all(np.abs(mass - mo_d[0]) <= 1e-6 * absmass)
    rer, _, _ = oracle.fitness(ocfg, np.stack([xin[None], xout[None]]))
    assert abs(erank[-1] - rer.mean()) <= 1e-5
    assert np.all(erank > 0)
    rec = json.loads(js.read_text())
    assert list(rec.keys()) == ["gen", "elapsed", "chemical", "ca", "agents", "voronoi", "archive", "pool"]
    assert rec["gen"] == gens - 1
    np.testing.assert_allclose(np.array(rec["ca"]["flow_kernels"]), flow.reshape(H, 9), atol=5e-5)
