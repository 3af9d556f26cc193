"""GPU organism loop and evolution.json records (slime_snapshot_json, the host
generation loop over slime_neural_ca_update): the records carry the reference's
keys in its order (slime/extract_state.cu:64-184) with the device state's values
in its formatting, and the loop reproduces the oracle's init -> step -> field ->
rank sequence generation after generation.
"""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from slime_amd import ComponentPool  # noqa: E402
from slime_amd.organism import Organism  # noqa: E402
from slime_amd.synthetic import CAConfig, make_params  # noqa: E402

KEYS = ["gen", "elapsed", "chemical", "ca", "agents", "voronoi", "archive", "pool"]


def _cfg(G=32, D=8):
    return CAConfig(name="org", B=1, G=G, H=8, D=D, dtype="fp32", steps=1, w_std=0.1)


def _expected(conc, K, gen, elapsed, counters, capacity):
    G = conc.shape[0]
    n = min(16, G)
    off = (G - n) // 2
    s = conc[off:off + n, off:off + n].reshape(-1)
    rec = '{"gen":%d,"elapsed":%.2f,' % (gen, elapsed)
    rec += '"chemical":{"concentration":[' + ",".join("%.4f" % float(v) for v in s) + '],"size":%d},' % n
    rec += '"ca":{"flow_kernels":[' + ",".join(
        "[" + ",".join("%.4f" % float(v) for v in K[h]) + "]" for h in range(K.shape[0])) + "]},"
    rec += '"agents":[],"voronoi":[],"archive":{"size":0,"elites":[]},'
    rec += '"pool":{"active":%d,"capacity":%d,"spawned":%d,"culled":%d}}' % (
        counters[0], capacity, counters[1], counters[2])
    return rec


@pytest.mark.parametrize("G", [32, 64])
def test_snapshot_record_matches_device_state(G):
    cfg = _cfg(G)
    p = make_params(cfg, seed=3)
    conc0 = np.random.default_rng(4).random((G, G), dtype=np.float32) * 2 - 0.5
    pool = ComponentPool(16, 32)
    for _ in range(5):
        pool.spawn(-1, 0.0)
    pool.fitness[:] = 0.01
    pool.cull()
    print(f"[case] snapshot G={G}", flush=True)
    with Organism(p, conc0, G=G, H=8, D=8, pool=pool, max_generations=8) as org:
        rec = org.snapshot(7, 12.345)
        counters = pool.counters.cpu().numpy()
        assert rec == _expected(conc0, p["K"][0], 7, 12.345, counters, 16)
        d = json.loads(rec)
        assert list(d.keys()) == KEYS
        assert d["pool"] == {"active": 0, "capacity": 16, "spawned": 5, "culled": 5}
        assert len(d["ca"]["flow_kernels"]) == 8 and len(d["chemical"]["concentration"]) == min(16, G) ** 2
        org.pool = None
        d = json.loads(org.snapshot(0, 0.0))
        assert d["pool"] == {"active": 0, "capacity": 0, "spawned": 0, "culled": 0}


def test_generation_loop_tracks_the_oracle(oracle, tmp_path):
    cfg = _cfg(32, 8)
    p = make_params(cfg, seed=1)
    conc0 = np.random.default_rng(5).random((32, 32), dtype=np.float32)
    ocfg = oracle.OracleConfig(B=1, G=32, H=8, D=8)
    print("[case] organism generations 0..3 against the oracle", flush=True)
    with Organism(p, conc0, G=32, H=8, D=8, max_generations=16) as org:
        for gen in range(4):
            before = org.conc.cpu().numpy()
            org.generation(gen)
            torch.cuda.synchronize()
            after = org.conc.cpu().numpy()
            xin, xout = org.ca_input.cpu().numpy(), org.ca_output.cpu().numpy()
            # each generation against the oracle's init -> step -> field from the same field
            Y, _, _ = oracle.step(ocfg, oracle.init_from_field(before, cfg.C)[None], p, 1)
            ref = oracle.field_from_state(Y[0])
            scale = np.abs(Y[0]).mean(axis=-1)  # the field shrinks by orders each generation
            assert np.max(np.abs(after - ref) / scale) <= 1e-5, gen
            rer, _, _ = oracle.fitness(ocfg, np.stack([xin[None], xout[None]]))
            assert abs(org.effective_rank_history[gen].item() - rer.mean()) <= 1e-5, gen
        erank = org.effective_rank_history.cpu().numpy()
        assert np.all(erank[4:] == 0.0) and np.all(erank[:4] > 0)


def test_run_writes_the_evolution_file(tmp_path):
    cfg = _cfg(32, 8)
    p = make_params(cfg, seed=1)
    conc0 = np.random.default_rng(5).random((32, 32), dtype=np.float32)
    path = tmp_path / "evolution.json"
    with Organism(p, conc0, G=32, H=8, D=8, max_generations=16) as org:
        recs = org.run(5, json_path=str(path), snapshot_every=2)
    data = json.loads(path.read_text())
    assert [r["gen"] for r in data] == [0, 2, 4] and len(recs) == 3
    assert all(list(r.keys()) == KEYS for r in data)
    assert all(r["chemical"]["size"] == 16 and len(r["ca"]["flow_kernels"]) == 8 for r in data)
