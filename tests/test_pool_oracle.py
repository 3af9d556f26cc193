"""CPU checks of the pool oracle (oracle/pool_oracle.cpp): the restatement of the
reference's component pool (slime/memory/pool.cu, slime/core/organism.cu:144-201,
557-614; slime/kernels/warp_ca.cu:229-240) that the GPU pool is compared with.

The checks pin it by properties, not by retyping its formulas: the PRNG's state
transition is a full-period linear map over GF(2)^128, its output is the sum of
the two state words, Box-Muller matches its textbook closed form and moments, and
the pool operations keep their invariants (counters, slot choice, thresholds,
inheritance).
"""
import numpy as np
import pytest

import oracle

MASK = (1 << 64) - 1


# ---- xorshift128+ ---------------------------------------------------------------------
def _transition(state: int) -> int:
    """One oracle step on a 128-bit state (s0 in the low word)."""
    g = oracle.Xorshift128p(state & MASK, state >> 64)
    g.next()
    s0, s1 = g.state
    return s0 | (s1 << 64)


def _gf2_matrix() -> np.ndarray:
    """The transition as a 128 x 128 matrix over GF(2), probed with unit states."""
    m = np.zeros((128, 128), np.uint8)
    for j in range(128):
        out = _transition(1 << j)
        m[:, j] = [(out >> i) & 1 for i in range(128)]
    return m


def _matmul2(a, b):
    return (a.astype(np.int64) @ b.astype(np.int64) % 2).astype(np.uint8)


def _matpow2(m, e: int):
    r = np.eye(128, dtype=np.uint8)
    while e:
        if e & 1:
            r = _matmul2(r, m)
        m = _matmul2(m, m)
        e >>= 1
    return r


def test_xorshift_transition_is_linear_and_shifts_s1_into_s0():
    rng = np.random.default_rng(1)
    for _ in range(20):
        a = int(rng.integers(0, 2**63)) | (int(rng.integers(0, 2**63)) << 64)
        b = int(rng.integers(0, 2**63)) | (int(rng.integers(0, 2**63)) << 64)
        assert _transition(a ^ b) == _transition(a) ^ _transition(b)
        assert _transition(a) & MASK == a >> 64  # new s0 = old s1


def test_xorshift_has_full_period():
    # A maximal-period xorshift generator: M^(2^128 - 1) = I and M^((2^128 - 1)/p) != I
    # for every prime p dividing 2^128 - 1. A wrong shift amount or direction breaks this.
    m = _gf2_matrix()
    order = (1 << 128) - 1
    primes = [3, 5, 17, 257, 641, 65537, 274177, 6700417, 67280421310721]
    prod = 1
    for p in primes:
        prod *= p
    assert prod == order
    eye = np.eye(128, dtype=np.uint8)
    assert np.array_equal(_matpow2(m, order), eye)
    for p in primes:
        assert not np.array_equal(_matpow2(m, order // p), eye), p


def test_xorshift_output_is_the_sum_of_the_new_state_words():
    g = oracle.Xorshift128p(0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9)
    for _ in range(100):
        u = g.next()
        s0, s1 = g.state
        assert u == np.float32(float(np.float32((s0 + s1) & MASK)) / 2.0**64)
        assert 0.0 <= u <= 1.0


def test_xorshift_uniform_moments():
    g = oracle.Xorshift128p(12345, 67890)
    u = np.array([g.next() for _ in range(20000)])
    assert abs(u.mean() - 0.5) < 0.01
    assert abs(u.var() - 1.0 / 12.0) < 0.005


def test_box_muller_closed_form_and_moments():
    g = oracle.Xorshift128p(0xDEADBEEF, 0x12345678)
    ref = oracle.Xorshift128p(*g.state)
    for _ in range(50):
        z = g.gaussian()
        u1, u2 = ref.next(), ref.next()
        expect = np.sqrt(-2.0 * np.log(u1 + 1e-10)) * np.cos(2.0 * np.pi * u2)
        assert z == pytest.approx(expect, rel=1e-5, abs=1e-5)
    zs = np.array([g.gaussian() for _ in range(20000)])
    assert abs(zs.mean()) < 0.03
    assert abs(zs.var() - 1.0) < 0.05


# ---- pool operations ------------------------------------------------------------------
def _pool(capacity=16, genome=64):
    p = oracle.Pool(capacity, genome)
    p.init()
    return p


def _check_counters(p):
    assert p.counters[0] == int(p.alive.sum())


def test_init_state():
    p = oracle.Pool(8, 16)
    p.genome[:] = 3.0
    p.alive[:] = 1
    p.counters[:] = 7
    p.init()
    assert (p.id == -1).all() and (p.alive == 0).all() and (p.age == 0).all()
    assert (p.fitness == 0).all() and (p.coherence == 0).all() and (p.hunger == 0.5).all()
    assert (p.genome == 0).all() and (p.gradients == 0).all() and (p.counters == 0).all()


def test_spawn_without_parent_fills_first_slot_uniformly():
    p = _pool(8, 512)
    p.spawn(-1, 0.01)
    assert p.alive.tolist() == [1, 0, 0, 0, 0, 0, 0, 0]
    assert p.id[0] == 0 and p.counters.tolist() == [1, 1, 0]
    g = p.genome[0]
    # new_id 0 seeds both words with 0: the all-zero state stays zero, every draw is 0
    assert (g == -1.0).all()
    p.spawn(-1, 0.01)
    g = p.genome[1]
    assert p.id[1] == 1 and ((g >= -1.0) & (g < 1.0)).all() and abs(g.mean()) < 0.1
    assert (p.gradients[:2] == 0).all()
    _check_counters(p)


def test_spawn_inherits_with_mutation():
    p = _pool(8, 512)
    p.spawn(-1, 0.0)
    p.spawn(-1, 0.0)  # entry 1: uniform genome
    p.gradients[1] = np.linspace(-1, 1, 512, dtype=np.float32)
    p.spawn(1, 0.0)  # rate 0: exact copy, gradients decayed by 0.9
    assert np.array_equal(p.genome[2], p.genome[1])
    assert np.allclose(p.gradients[2], p.gradients[1] * np.float32(0.9), rtol=0, atol=0)
    p.spawn(1, 2.0)  # rate > 1: every element draws a Gaussian step, clamped
    d = p.genome[3] - p.genome[1]
    assert (d != 0).sum() > 500
    assert ((p.genome[3] >= -1) & (p.genome[3] <= 1)).all()
    assert abs(d).max() < 0.9  # 0.1 * |z| with |z| < sqrt(-2 ln 1e-10) ~ 6.8
    p.spawn(1, 0.05)  # ~5 % of the elements
    n = int((p.genome[4] != p.genome[1]).sum())
    assert 8 < n < 50
    assert p.id[2:5].tolist() == [2, 3, 4]
    _check_counters(p)


def test_spawn_into_full_pool_does_nothing():
    p = _pool(4, 8)
    for _ in range(4):
        p.spawn(-1, 0.0)
    before = p.copy()
    p.spawn(0, 0.5)
    for n in oracle.Pool.FIELDS:
        assert np.array_equal(getattr(p, n), getattr(before, n)), n


def test_spawn_reuses_the_first_dead_slot():
    p = _pool(6, 8)
    for _ in range(5):
        p.spawn(-1, 0.0)
    p.fitness[:] = 1.0
    p.fitness[1] = 0.0  # culled below 0.8 * 0.1
    p.hunger[:] = 0.0
    p.cull(0.8, 0.95)
    assert p.alive.tolist() == [1, 0, 1, 1, 1, 0]
    p.spawn(0, 0.0)
    assert p.alive.tolist() == [1, 1, 1, 1, 1, 0] and p.id[1] == 5
    _check_counters(p)


def test_set_fitness_averages_heads_and_sets_hunger_and_history():
    p = _pool(8, 8)
    for _ in range(3):
        p.spawn(-1, 0.0)
    heads = 4
    rng = np.random.default_rng(3)
    fit = rng.random((5, heads), dtype=np.float32)
    coh = rng.random((5, heads), dtype=np.float32)
    fh = np.full((3, 8), -7.0, np.float32)
    ch = np.full((3, 8), -7.0, np.float32)
    p.set_fitness(fit, coh, 5, heads, 2, fh, ch)
    # entries 0..2 alive: head means in order; 3, 4 dead: untouched
    for i in range(3):
        f = np.float32(0)
        c = np.float32(0)
        for h in range(heads):
            f = np.float32(f + fit[i, h])
            c = np.float32(c + coh[i, h])
        assert p.fitness[i] == np.float32(f / np.float32(heads))
        assert p.coherence[i] == np.float32(c / np.float32(heads))
        assert p.hunger[i] == np.float32(1) - p.coherence[i]
        assert fh[2, i] == p.fitness[i] and ch[2, i] == p.coherence[i]
    assert (p.fitness[3:] == 0).all() and (fh[:2] == -7).all() and (fh[2, 3:] == -7).all()
    assert np.allclose(oracle.hunger(coh), 1.0 - coh)


def test_cull_thresholds_are_strict():
    p = _pool(6, 8)
    for _ in range(6):
        p.spawn(-1, 0.0)
    p.fitness[:] = [0.08, np.nextafter(np.float32(0.08), np.float32(0)), 0.5, 0.5, 0.5, 0.5]
    p.hunger[:] = [0.0, 0.0, 0.95, np.nextafter(np.float32(0.95), np.float32(1)), 0.2, 0.9]
    p.cull(0.8, 0.95)
    # fitness < 0.8 * 0.1 (in fp32) or hunger > 0.95 dies
    assert p.alive.tolist() == [1 if np.float32(0.08) >= np.float32(0.8) * np.float32(0.1) else 0, 0, 1, 0, 1, 1]
    assert p.counters[2] == 6 - int(p.alive.sum())
    _check_counters(p)


def test_age_counts_alive_entries_only():
    p = _pool(4, 8)
    p.spawn(-1, 0.0)
    p.spawn(-1, 0.0)
    p.age_up()
    p.age_up()
    assert p.age.tolist() == [2, 2, 0, 0]


def test_spawn_wave_generation_zero_is_all_or_nothing():
    # At generation 0 every lane's seed is 0, so all 32 draws equal u0.
    u0 = float(np.float32((1013904223 & 0xFFFFFF) / 16777216.0))
    for prob, expect in ((np.nextafter(np.float32(u0), np.float32(1)), 32), (u0, 0)):
        p = _pool(64, 8)
        p.spawn(-1, 0.0)
        p.fitness[0] = 0.9  # the parent
        used = p.spawn_wave(float(prob), 0)
        assert used == np.float32(prob)
        assert int(p.alive.sum()) == 1 + expect and p.counters[1] == 1 + expect


def test_spawn_wave_needs_a_fit_parent_and_respects_capacity():
    p = _pool(8, 8)
    p.spawn(-1, 0.0)
    p.fitness[0] = 0.5  # not > 0.5
    p.spawn_wave(1.0, 3)
    assert int(p.alive.sum()) == 1
    p.fitness[0] = 0.6
    p.spawn_wave(1.0, 3)  # every draw < 1: spawns until the pool is full
    assert int(p.alive.sum()) == 8 and p.counters[1] == 8
    _check_counters(p)


def test_spawn_wave_lifecycle_probability():
    p = _pool(8, 8)
    assert p.spawn_wave(-1.0, 5) == np.float32(0.1)  # 0.1 * exp(0)
    for _ in range(8):
        p.spawn(-1, 0.0)
    used = p.spawn_wave(-1.0, 5)
    assert used == pytest.approx(0.1 * np.exp(-8 / 256.0), rel=1e-6)


def test_evolve_is_set_fitness_spawn_wave_cull():
    rng = np.random.default_rng(7)
    a = _pool(32, 16)
    for _ in range(10):
        a.spawn(-1, 0.0)
    b = a.copy()
    fit = rng.random((10, 2), dtype=np.float32)
    coh = rng.random((10, 2), dtype=np.float32)
    a.evolve(fit, coh, 10, 2, 4)
    b.set_fitness(fit, coh, 10, 2, 4)
    b.spawn_wave(-1.0, 4)
    b.cull(0.8, 0.95)
    for n in oracle.Pool.FIELDS:
        assert np.array_equal(getattr(a, n), getattr(b, n)), n
