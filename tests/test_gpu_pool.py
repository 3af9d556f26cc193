"""GPU component pool (slime_pool_* through the C ABI) against the pool oracle:
the fitness consumers of the reference (hunger, age, cull, spawn, spawn wave and
the lifecycle's evolve step; slime/memory/pool.cu, slime/core/organism.cu:144-201,
557-614, slime/kernels/warp_ca.cu:229-240).

Integer state (ids, alive flags, ages, counters) and the fitness fields must agree
exactly; genomes agree to 1e-6 (the Gaussian mutation calls the device's and the
host's own log, cos and sqrt).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from slime_amd import ComponentPool, Pseudopod  # noqa: E402
from slime_amd import pool as poolmod  # noqa: E402
from slime_amd.synthetic import CAConfig, make_params, make_state  # noqa: E402


def _compare(dev: ComponentPool, ref: oracle.Pool, what: str):
    h = dev.host()
    for n in ("id", "alive", "age", "counters", "fitness", "coherence", "hunger"):
        assert np.array_equal(h[n], getattr(ref, n)), f"{what}: {n}"
    for n in ("genome", "gradients"):
        np.testing.assert_allclose(h[n], getattr(ref, n), rtol=0, atol=1e-6, err_msg=f"{what}: {n}")


def _fit(rng, n, heads):
    return (rng.random((n, heads), dtype=np.float32), rng.random((n, heads), dtype=np.float32))


def test_pool_init_matches_oracle():
    dev = ComponentPool(256, 512)
    ref = oracle.Pool(256, 512)
    ref.init()
    _compare(dev, ref, "init")


def test_pool_sequence_matches_oracle():
    rng = np.random.default_rng(11)
    dev = ComponentPool(64, 512)
    ref = oracle.Pool(64, 512)
    ref.init()
    print("[case] pool 64 x 512: spawns, fitness, cull, age, waves", flush=True)
    for _ in range(6):
        dev.spawn(-1, 0.0)
        ref.spawn(-1, 0.0)
    _compare(dev, ref, "random spawns")
    for parent, rate in ((0, 0.0), (1, 0.01), (2, 0.5), (3, 2.0), (70, 0.01)):
        dev.spawn(parent, rate)
        ref.spawn(parent, rate)
    _compare(dev, ref, "inherited spawns")
    fh = torch.full((5, 64), -1.0, device="cuda")
    ch = torch.full((5, 64), -1.0, device="cuda")
    fh_ref = np.full((5, 64), -1.0, np.float32)
    ch_ref = np.full((5, 64), -1.0, np.float32)
    for gen in range(5):
        f, c = _fit(rng, 20, 8)
        f[:4] += 0.5  # some fit parents
        dev.set_fitness(torch.from_numpy(f).cuda(), torch.from_numpy(c).cuda(), gen, fh, ch)
        ref.set_fitness(f, c, 20, 8, gen, fh_ref, ch_ref)
        _compare(dev, ref, f"set_fitness gen {gen}")
        dev.spawn_wave(0.3, gen + 1)
        ref.spawn_wave(0.3, gen + 1)
        _compare(dev, ref, f"spawn wave gen {gen}")
        dev.age_up()
        ref.age_up()
        dev.cull(0.8, 0.6)
        ref.cull(0.8, 0.6)
        _compare(dev, ref, f"cull gen {gen}")
    assert np.array_equal(fh.cpu().numpy(), fh_ref) and np.array_equal(ch.cpu().numpy(), ch_ref)
    h = dev.host()
    assert h["counters"][0] == int(h["alive"].sum())


def test_spawn_wave_lifecycle_probability_and_full_pool():
    dev = ComponentPool(16, 32)
    ref = oracle.Pool(16, 32)
    ref.init()
    dev.spawn(-1, 0.0)
    ref.spawn(-1, 0.0)
    f = np.full((1, 1), 0.9, np.float32)
    c = np.full((1, 1), 0.5, np.float32)
    dev.set_fitness(torch.from_numpy(f).cuda(), torch.from_numpy(c).cuda(), 0)
    ref.set_fitness(f, c, 1, 1, 0)
    for gen in range(1, 40):
        dev.spawn_wave(-1.0, gen)  # 0.1 exp(-active / 256) on the device
        ref.spawn_wave(-1.0, gen)
    _compare(dev, ref, "lifecycle waves")
    dev.spawn_wave(1.0, 7)
    ref.spawn_wave(1.0, 7)
    _compare(dev, ref, "wave into a full pool")
    assert dev.stats["active"] == 16


def test_hunger_matches():
    c = torch.rand(1000, device="cuda")
    h = poolmod.hunger(c)
    assert torch.equal(h, 1.0 - c)
    assert np.array_equal(oracle.hunger(c.cpu().numpy()), h.cpu().numpy())


def test_evolve_on_the_ca_ensemble_fitness():
    """c4-shaped path: 8 pods, batch entry = pod = component; the fused fitness of a
    short rollout feeds the pool's lifecycle step."""
    cfg = CAConfig(name="pool", B=8, G=32, H=8, D=8, dtype="fp32", steps=1, w_std=0.1, pods=8)
    params = make_params(cfg, seed=5)
    x = make_state(cfg, seed=6)
    print("[case] evolve on an 8-pod fp32 rollout, G=32 D=8", flush=True)
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, dtype="fp32", pods=cfg.pods) as pp:
        pp.set_params(params)
        xs = [torch.from_numpy(x).cuda()]
        for _ in range(3):
            xs.append(pp.forward(xs[-1]))
        hist = torch.stack(xs).contiguous()
        erank, coh, fit = pp.fitness(hist)
    dev = ComponentPool(32, 64)
    ref = oracle.Pool(32, 64)
    ref.init()
    for _ in range(8):
        dev.spawn(-1, 0.0)
        ref.spawn(-1, 0.0)
    f, c = fit.cpu().numpy(), coh.cpu().numpy()
    # scale the fitness into the lifecycle's range so that both branches occur
    f = (f / f.max()).astype(np.float32)
    fh = torch.zeros((4, 32), device="cuda")
    fh_ref = np.zeros((4, 32), np.float32)
    for gen in range(4):
        dev.evolve(torch.from_numpy(f).cuda(), torch.from_numpy(c).cuda(), gen, fh)
        ref.evolve(f, c, 8, 8, gen, fh_ref)
        _compare(dev, ref, f"evolve gen {gen}")
    assert np.array_equal(fh.cpu().numpy(), fh_ref)
