"""GPU parity: the HIP library (through its C ABI) against the CPU oracle on the
same seeded inputs.

Tolerances (the parity metric is max|gpu - ref| / max|ref| per tensor):
  fp32 state and weights: 1e-5;  bf16 state and weights: 2e-2.
  Mass: |sum_out - sum_in| <= 1e-6 |sum_in| per (batch, head), asserted on the
  conserved fp32 result (for bf16 on the value before the final rounding, with
  the rounding drift of the stored tensor bounded separately).
"""
import numpy as np
import pytest

from slime_amd import Pseudopod, make_params, make_state, round_bf16
from slime_amd.synthetic import CAConfig
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = {"fp32": 1e-5, "bf16": 2e-2}


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _ocfg(cfg, **kw):
    from oracle import OracleConfig
    base = dict(B=cfg.B, G=cfg.G, H=cfg.H, D=cfg.D, pods=cfg.pods,
                growth_per_cell=cfg.growth_per_cell, dt=cfg.dt)
    base.update(kw)
    return OracleConfig(**base)


def _prep(cfg, pseed=1, sseed=2):
    """Params and state as the device sees them (bf16-rounded when bf16)."""
    p = make_params(cfg, seed=pseed)
    X = make_state(cfg, seed=sseed)
    if cfg.dtype == "bf16":
        p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
        X = round_bf16(X)
    return p, X


def _dev(a, dtype):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
    return t.to(torch.bfloat16 if dtype == "bf16" else torch.float32).contiguous()


def _host(t):
    return t.float().cpu().numpy()


def _engine(cfg, pvi_chain=False, **kw):
    print(f"[case] {cfg.name} B={cfg.B} G={cfg.G} D={cfg.D} {cfg.dtype} pods={cfg.pods} "
          f"per_cell={cfg.growth_per_cell} chain={pvi_chain}", flush=True)
    e = Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, cfg.growth_per_cell, cfg.pods,
                  pvi_chain, **kw)
    return e


def _cfg(name, B, G, D, dtype, **kw):
    return CAConfig(name, B=B, G=G, H=8, D=D, dtype=dtype, steps=1, w_std=0.05, **kw)


def _oracle_flow(oracle, ocfg, X, P, I, V, p):
    U = oracle.potential(ocfg, X, p["K"])
    g = oracle.growth(ocfg, U, p["mu"], p["sigma"])
    A = oracle.attention(ocfg, P, I)
    Vt = oracle.propagate(ocfg, A, V)
    Y = oracle.mix(ocfg, X, g, Vt, p["M"])
    return oracle.conserve(ocfg, X, Y)


# ---- configuration c1 against the committed golden fixture and the oracle ----------------

def test_c1_step_matches_golden_and_oracle(oracle):
    from slime_amd import CONFIGS
    from tests.golden.make_golden import check_c1
    cfg = CONFIGS["c1"]
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, cfg.dtype))
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    check_c1(Y, tol=TOL["fp32"])
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 1)
    assert norm_err(Y, ref) <= TOL["fp32"]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    ys = Y.astype(np.float64).reshape(cfg.B, -1, cfg.H, cfg.D).sum(axis=(1, 3))
    np.testing.assert_allclose(ys, rmi, rtol=1e-6)


# ---- stage by stage, MFMA projection path ----------------------------------------------------

@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_project_mfma_matches_oracle(oracle, dtype):
    cfg = _cfg("proj", B=2, G=16, D=64, dtype=dtype)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        assert e.uses_mfma
        e.set_params(p)
        P, I, V = e.project(_dev(X, dtype))
        torch.cuda.synchronize()
        got = [_host(t) for t in (P, I, V)]
    ref = oracle.project(_ocfg(cfg), X, p["WP"], p["WI"], p["WV"])
    for name, g, r in zip("PIV", got, ref):
        err = norm_err(g, r)
        print(f"  {name}: normalised error {err:.3e}")
        assert err <= TOL[dtype], name


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_flow_lenia_matches_oracle_on_same_projections(oracle, dtype):
    cfg = _cfg("flow", B=2, G=16, D=64, dtype=dtype)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, dtype)
        P, I, V = e.project(x)
        y = e.flow_lenia(x, P, I, V)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        hp, hi, hv, Y = (_host(t) for t in (P, I, V, y))
    ref, rmi, rmo = _oracle_flow(oracle, _ocfg(cfg), X, hp, hi, hv, p)
    err = norm_err(Y, ref)
    print(f"  Y: normalised error {err:.3e}")
    assert err <= TOL[dtype]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    drift = np.abs(Y.astype(np.float64).reshape(cfg.B, -1, cfg.H, cfg.D).sum(axis=(1, 3)) - rmi)
    # bf16: one rounding of each stored element; the sum over 16 K elements of
    # ~U[0,1) values carries ~1e-5 relative noise (4 sigma ~ 4e-5). A second,
    # biased rounding (rescaling already-rounded values) would show up as ~1e-4.
    bound = 1e-6 if dtype == "fp32" else 5e-5
    assert np.all(drift <= bound * np.abs(rmi)), drift / np.abs(rmi)


# ---- peaked attention: the bf16 matrix-core stencil's S4 and S5 ------------------------------
#
# At the configurations' own weights the attention is nearly uniform and the tests
# above cannot see S4/S5 (a uniform, mirrored or query/key-swapped attention moves Y
# by less than the bf16 bar). These cases use the peaked weights of
# tests.conftest.peaked_params, where tests/test_oracle.py shows on the same inputs
# that each of those mistakes moves Y by more than 5x the bar.

def _prep_peaked(cfg, pseed=1, sseed=2):
    from tests.conftest import peaked_params
    p = peaked_params(cfg, seed=pseed)
    p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
    return p, round_bf16(make_state(cfg, seed=sseed))


@pytest.mark.parametrize("G", [16, 32])
def test_flow_lenia_peaked_attention_matches_oracle_on_same_projections(oracle, G):
    cfg = _cfg("peak", B=2, G=G, D=64, dtype="bf16", pods=2)
    p, X = _prep_peaked(cfg)
    with _engine(cfg) as e:
        assert e.uses_mfma
        e.set_params(p)
        x = _dev(X, "bf16")
        P, I, V = e.project(x)
        y = e.flow_lenia(x, P, I, V)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        hp, hi, hv, Y = (_host(t) for t in (P, I, V, y))
    ocfg = _ocfg(cfg)
    A = oracle.attention(ocfg, hp, hi)
    peak = float(A.max(axis=-1).mean())
    ref, rmi, _ = _oracle_flow(oracle, ocfg, X, hp, hi, hv, p)
    err = norm_err(Y, ref)
    print(f"  G={G}: mean largest attention weight {peak:.3f}; Y normalised error {err:.3e}")
    assert peak > 0.5  # the case is peaked, or it pins nothing
    assert err <= TOL["bf16"]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


@pytest.mark.parametrize("per_cell", [False, True])
def test_step_peaked_attention_matches_oracle(oracle, per_cell):
    # The whole step against the oracle's own projections: the device's bf16-rounded
    # P and I move the scores by ~0.4 % of their size, which flips no neighbour
    # choice at these seeds (a flip would show as an error of ~0.1).
    cfg = _cfg("peakstep", B=2, G=16, D=64, dtype="bf16", pods=2, growth_per_cell=per_cell)
    p, X = _prep_peaked(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, "bf16"))
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 1)
    err = norm_err(Y, ref)
    print(f"  Y: normalised error {err:.3e}")
    assert err <= TOL["bf16"]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


# ---- the growth functions and the per-cell conservation of the shipped kernel ----------------

@pytest.mark.parametrize("dtype,D,fn,cons,per_cell", [
    ("fp32", 64, 1, 0, False),
    ("fp32", 64, 2, 1, True),
    ("fp32", 16, 0, 1, False),
    ("bf16", 64, 1, 0, False),   # matrix-core stencil with the general growth
    ("bf16", 64, 2, 0, True),
    ("bf16", 64, 0, 1, False),   # matrix-core stencil, per-cell conservation
    ("bf16", 32, 1, 1, True),
])
def test_step_growth_and_conservation_variants_match_oracle(oracle, dtype, D, fn, cons, per_cell):
    from tests.conftest import growth_variant_params
    cfg = _cfg("variant", B=2, G=16, D=D, dtype=dtype, growth_per_cell=per_cell, pods=2)
    X = make_state(cfg, seed=2)
    if dtype == "bf16":
        X = round_bf16(X)
    p = growth_variant_params(cfg, oracle, X)
    if dtype == "bf16":
        p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
    with _engine(cfg, growth_fn=fn, conservation=cons) as e:
        e.set_params(p)
        x = _dev(X, dtype)
        y1 = e.forward(x)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        y2 = e.forward(x, n_steps=2)
        torch.cuda.synchronize()
        mi2, mo2 = e.mass()
        Y1, Y2 = _host(y1), _host(y2)
    ocfg = _ocfg(cfg, growth_fn=fn, conservation=cons)
    ref1, rmi, _ = oracle.step(ocfg, X, p, 1)
    ref2, _, _ = oracle.step(ocfg, X, p, 2)
    e1, e2 = norm_err(Y1, ref1), norm_err(Y2, ref2)
    print(f"  growth_fn {fn}, conservation {cons}: 1 step {e1:.3e}, 2 steps {e2:.3e}")
    assert e1 <= TOL[dtype] and e2 <= TOL[dtype]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    np.testing.assert_allclose(mo2, mi2, rtol=1e-6)
    if cons == 1 and dtype == "fp32":
        # every cell keeps its head sums (no cell of these states takes the guard)
        cx = X.astype(np.float64).reshape(cfg.B, cfg.G, cfg.G, cfg.H, D).sum(-1)
        cy = Y1.astype(np.float64).reshape(cfg.B, cfg.G, cfg.G, cfg.H, D).sum(-1)
        np.testing.assert_allclose(cy, cx, rtol=1e-5, atol=1e-6 * np.abs(cx).max())


# ---- full steps ------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,per_cell,pods,chain,D", [
    ("fp32", False, 1, False, 64),
    ("fp32", True, 1, False, 64),
    ("bf16", False, 1, False, 64),
    ("bf16", False, 2, False, 64),
    ("bf16", True, 1, False, 64),
    ("bf16", False, 1, True, 64),
    ("fp32", False, 1, True, 32),
    ("bf16", True, 2, False, 16),
    # pvi_chain 2: the reference's perception (3x3 neighbourhood sum) and chain
    ("fp32", False, 1, 2, 64),
    ("bf16", False, 2, 2, 64),
    ("fp32", True, 1, 2, 8),
])
def test_step_matches_oracle(oracle, dtype, per_cell, pods, chain, D):
    cfg = _cfg("step", B=2, G=16, D=D, dtype=dtype, growth_per_cell=per_cell, pods=pods)
    p, X = _prep(cfg)
    with _engine(cfg, pvi_chain=chain) as e:
        e.set_params(p)
        y = e.forward(_dev(X, dtype))
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    ref, rmi, _ = oracle.step(_ocfg(cfg, pvi_chain=chain), X, p, 1)
    err = norm_err(Y, ref)
    print(f"  Y: normalised error {err:.3e}")
    assert err <= TOL[dtype]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_multi_step_fp32_matches_oracle(oracle):
    cfg = _cfg("multi", B=1, G=16, D=64, dtype="fp32", growth_per_cell=True)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "fp32")
        y3 = e.forward(x, n_steps=3)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y3)
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 3)
    err = norm_err(Y, ref)
    print(f"  Y after 3 steps: normalised error {err:.3e}")
    assert err <= TOL["fp32"]
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


# fp32 only: in bf16 the chain through the 3x3 sum amplifies the storage rounding of
# P, I and V past the 2e-2 bar within two steps (one step of it is held to the bar
# in test_step_matches_oracle); the scale folding checked here is the same code for
# both storage types.
@pytest.mark.parametrize("dtype", ["fp32"])
def test_multi_step_perception_sum_chain_matches_oracle(oracle, dtype):
    # pvi_chain 2 over two steps in one call: step 2 reads step 1's unscaled output,
    # whose mass scale is folded into W_P (the neighbourhood sum is per channel, so
    # the per-head scale commutes with it). The chain through the 3x3 sum amplifies
    # rounding quickly: one fp32 rounding of X and W moves the oracle's own result by
    # 6e-7, 1.9e-6 and 9e-6 after 1, 2 and 3 steps (3e-7, 4.7e-7, 9.4e-7 for parallel
    # projections), so two steps is where the 1e-5 bar still measures the device.
    cfg = _cfg("multichain", B=2, G=16, D=64, dtype=dtype)
    p, X = _prep(cfg)
    with _engine(cfg, pvi_chain=2) as e:
        e.set_params(p)
        x = _dev(X, dtype)
        P, I, V = e.project(x)
        y2 = e.forward(x, n_steps=2)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        hp, hi, hv, Y = (_host(t) for t in (P, I, V, y2))
    ocfg = _ocfg(cfg, pvi_chain=2)
    rp, ri, rv = oracle.project(ocfg, X, p["WP"], p["WI"], p["WV"])
    for name, g, r in zip("PIV", (hp, hi, hv), (rp, ri, rv)):
        err = norm_err(g, r)
        print(f"  {name}: normalised error {err:.3e}")
        assert err <= TOL[dtype], name
    ref, rmi, _ = oracle.step(ocfg, X, p, 2)
    err = norm_err(Y, ref)
    print(f"  Y after 2 steps: normalised error {err:.3e}")
    assert err <= TOL[dtype]
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_persistent_tiles_across_batches_and_pods(oracle):
    # 24 x 32 x 32 cells = 768 stencil tiles: more than the persistent grid holds at
    # once, so workgroups carry their staging pipeline across tile, batch and pod
    # boundaries. Every batch entry is checked against the oracle.
    cfg = _cfg("persist", B=24, G=32, D=64, dtype="bf16", pods=3)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, "bf16"))
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 1)
    for b in range(cfg.B):
        err = norm_err(Y[b], ref[b])
        assert err <= TOL["bf16"], (b, err)
    print(f"  max normalised error over batches {max(norm_err(Y[b], ref[b]) for b in range(cfg.B)):.3e}")
    np.testing.assert_allclose(mi, rmi, rtol=1e-6)
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_tile_tickets_cover_every_tile_on_each_launch(oracle):
    # After its fixed first tiles a workgroup draws its tiles from a per-XCD ticket
    # counter that the launch leaves at zero for the next one. Three launches on one
    # handle with three different states: a launch that skipped tiles would leave the
    # previous launch's values in the handle's output buffer, so each result is
    # checked in full against the oracle for its own state.
    cfg = _cfg("tickets", B=24, G=32, D=64, dtype="bf16", pods=3)
    p = _prep(cfg)[0]
    ocfg = _ocfg(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        for seed in (2, 3, 4):
            X = round_bf16(make_state(cfg, seed=seed))
            x = _dev(X, "bf16")
            P, I, V = e.project(x)
            y = e.flow_lenia(x, P, I, V)
            torch.cuda.synchronize()
            mi, mo = e.mass()
            hp, hi, hv, Y = (_host(t) for t in (P, I, V, y))
            ref, rmi, _ = _oracle_flow(oracle, ocfg, X, hp, hi, hv, p)
            errs = [norm_err(Y[b], ref[b]) for b in range(cfg.B)]
            print(f"  launch with state seed {seed}: max normalised error over batches {max(errs):.3e}")
            assert max(errs) <= TOL["bf16"], (seed, int(np.argmax(errs)), max(errs))
            np.testing.assert_allclose(mi, rmi, rtol=1e-6)
            np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_fixed_stride_tile_walk_when_the_tile_count_is_not_a_multiple_of_eight(oracle):
    # 37 x (24 / 4) x (24 / 8) = 666 tiles: not a multiple of 8, so the stencil takes
    # the fixed-stride walk instead of the per-XCD tickets, and with more tiles than
    # the persistent grid some workgroups take a second tile. The 24 x 24 grid's
    # 21,312 cells are not a multiple of 256, so the projections take the plain GEMM.
    cfg = _cfg("stride", B=37, G=24, D=64, dtype="bf16")
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, "bf16"), n_steps=2)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 2)
    errs = [norm_err(Y[b], ref[b]) for b in range(cfg.B)]
    print(f"  2 steps: max normalised error over batches {max(errs):.3e}")
    assert max(errs) <= TOL["bf16"], (int(np.argmax(errs)), max(errs))
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_multi_step_bf16_conserves_mass_and_tracks_oracle(oracle):
    # Two steps in one call: the second folds the first step's mass scale into its
    # weights and X loads; mass is conserved against the caller's input.
    cfg = _cfg("multi16", B=24, G=32, D=64, dtype="bf16", pods=2)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        y = e.forward(x, n_steps=2)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Y = _host(y)
    ref, rmi, _ = oracle.step(_ocfg(cfg), X, p, 2)
    err = norm_err(Y, ref)
    print(f"  Y after 2 bf16 steps: normalised error {err:.3e}")
    assert err <= TOL["bf16"]
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    # the stored bf16 state keeps the input mass up to its own rounding
    sums = Y.reshape(cfg.B, -1, cfg.H, cfg.D).sum(axis=(1, 3), dtype=np.float64)
    x_sums = X.reshape(cfg.B, -1, cfg.H, cfg.D).sum(axis=(1, 3), dtype=np.float64)
    assert np.all(np.abs(sums - x_sums) <= 5e-5 * np.abs(x_sums))


def test_in_place_and_zero_steps():
    cfg = _cfg("inplace", B=1, G=16, D=16, dtype="bf16")
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        y_ref = e.forward(x.clone(), n_steps=2)
        x2 = x.clone()
        e.forward(x2, out=x2, n_steps=2)
        x0 = e.forward(x, n_steps=0)
        torch.cuda.synchronize()
        assert torch.equal(x2, y_ref)
        assert torch.equal(x0, x)


def test_step_is_deterministic():
    cfg = _cfg("det", B=2, G=16, D=64, dtype="bf16")
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        a = e.forward(x, n_steps=2)
        b = e.forward(x, n_steps=2)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_non_finite_state_is_reported_by_mass(dtype):
    # One NaN in one channel of batch entry 1's head 3: the step runs, and the mass
    # read-back reports SLIME_ENONFINITE (the sums are copied out all the same). A
    # finite state on the same handle reads back cleanly afterwards.
    from slime_amd import SlimeError
    from slime_amd._lib import SLIME_ENONFINITE
    cfg = _cfg("nan", B=2, G=16, D=64, dtype=dtype)
    p, X = _prep(cfg)
    bad = X.copy()
    bad[1, 5, 7, 3 * 64 + 10] = np.nan
    with _engine(cfg) as e:
        e.set_params(p)
        e.forward(_dev(bad, dtype))
        torch.cuda.synchronize()
        with pytest.raises(SlimeError) as info:
            e.mass()
        assert info.value.code == SLIME_ENONFINITE
        assert "batch 1" in str(info.value)
        e.forward(_dev(X, dtype))
        torch.cuda.synchronize()
        mi, mo = e.mass()
        np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_set_params_rejects_non_finite_weights_and_keeps_the_old_ones():
    from slime_amd import SlimeError
    cfg = _cfg("nanp", B=1, G=16, D=64, dtype="bf16")
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        y0 = e.forward(x)
        for k in ("WP", "K", "M", "mu"):
            q = {n: v.copy() for n, v in p.items()}
            q[k].reshape(-1)[3] = np.inf if k == "M" else np.nan
            with pytest.raises(SlimeError, match=k):
                e.set_params(q)
        y1 = e.forward(x)  # the old parameters are still in place
        torch.cuda.synchronize()
        assert torch.equal(y0, y1)


def test_errors_surface_as_exceptions():
    from slime_amd import SlimeError
    cfg = _cfg("err", B=1, G=16, D=8, dtype="fp32")
    with _engine(cfg) as e:
        with pytest.raises(SlimeError):
            e.forward(_dev(make_state(cfg), "fp32"))  # parameters not set yet
        p, X = _prep(cfg)
        e.set_params(p)
        x = _dev(X, "fp32")
        with pytest.raises(SlimeError):
            e.flow_lenia(x, x, x, x, out=x)  # output aliases an input


# ---- fitness -----------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,D", [("bf16", 64), ("fp32", 8), ("fp32", 16), ("bf16", 32)])
def test_fitness_matches_oracle(oracle, dtype, D):
    cfg = _cfg("fit", B=2, G=16, D=D, dtype=dtype)
    p, X = _prep(cfg)
    T = 4
    with _engine(cfg) as e:
        e.set_params(p)
        hist = torch.empty((T,) + e.state_shape, dtype=e.torch_dtype, device="cuda")
        hist[0] = _dev(X, dtype)
        for t in range(1, T):
            e.forward(hist[t - 1], out=hist[t])
        er, coh, fit = e.fitness(hist)
        torch.cuda.synchronize()
        sweeps = e.jacobi_sweeps()
        H_ = _host(hist)
        er, coh, fit = _host(er), _host(coh), _host(fit)
    rer, rcoh, rfit = oracle.fitness(_ocfg(cfg), H_)
    print(f"  erank max abs diff {np.max(np.abs(er - rer)):.3e}, coh {np.max(np.abs(coh - rcoh)):.3e}")
    # Same history, same fp64 Gram up to summation order, same cyclic Jacobi order:
    # the results agree to fp32 output rounding, far inside the 0.01 erank criterion
    # of buildplan.md:289, and the sweep counts are equal.
    gram = oracle.gram(_ocfg(cfg), H_[-1])
    rsweeps = np.array([[oracle.jacobi_eigs(gram[b, h])[1] for h in range(cfg.H)]
                        for b in range(cfg.B)])
    np.testing.assert_array_equal(sweeps, rsweeps)
    np.testing.assert_allclose(er, rer, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(coh, rcoh, atol=1e-6)
    np.testing.assert_allclose(fit, rfit, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("T", [9, 11, 17])
def test_fitness_long_history_matches_oracle(oracle, T):
    """Histories longer than the 8 states one pass of the partial kernel reads: the
    later passes start from the previous pass's last state."""
    cfg = _cfg("fitT", B=1, G=16, D=32, dtype="fp32")
    rng = np.random.default_rng(T)
    X = make_state(cfg, seed=3)
    hist_h = np.stack([X + 0.05 * t * rng.standard_normal(X.shape).astype(np.float32)
                       for t in range(T)]).astype(np.float32)
    with _engine(cfg) as e:
        er, coh, fit = e.fitness(torch.from_numpy(hist_h).cuda().contiguous())
        torch.cuda.synchronize()
        er, coh, fit = _host(er), _host(coh), _host(fit)
    rer, rcoh, rfit = oracle.fitness(_ocfg(cfg), hist_h)
    print(f"  T={T}: coh {coh.ravel()[:3]} oracle {rcoh.ravel()[:3]}")
    np.testing.assert_allclose(er, rer, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(coh, rcoh, atol=1e-6)
    np.testing.assert_allclose(fit, rfit, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("kind", ["diagonal", "rank1", "rank1_plus_noise"])
def test_fitness_sweep_paths(oracle, kind):
    """The three ways the solve ends, against the oracle's sweep counts and ranks: a
    diagonal Gram (no rotation, the first sweep converges), a rank-1 Gram (rotations,
    then the off-diagonal sum falls below 1e-6 D before the limit) and a rank-1 Gram
    plus small noise (sub-threshold pairs keep the sum up: the 30-sweep limit, reached
    by the stop at the first sweep that rotates nothing)."""
    cfg = _cfg("fitsw", B=1, G=16, D=64, dtype="fp32")
    rng = np.random.default_rng(11)
    cells, C = cfg.G * cfg.G, cfg.H * cfg.D
    if kind == "diagonal":
        X = np.zeros((cells, C), np.float32)
        X[np.arange(cells), np.arange(cells) % C] = 1.0  # channel (cell mod C) only
    else:
        v = rng.standard_normal(C).astype(np.float32)
        X = np.outer(rng.random(cells, dtype=np.float32) + 0.5, v).astype(np.float32)
        if kind == "rank1_plus_noise":
            X += 1e-3 * rng.standard_normal(X.shape).astype(np.float32)
    X = X.reshape(1, cfg.G, cfg.G, C)
    hist_h = np.stack([X * 0.5, X])
    with _engine(cfg) as e:
        er, coh, fit = e.fitness(torch.from_numpy(hist_h).cuda().contiguous())
        torch.cuda.synchronize()
        sweeps = e.jacobi_sweeps()
        er = _host(er)
    gram = oracle.gram(_ocfg(cfg), hist_h[-1])
    rsweeps = np.array([[oracle.jacobi_eigs(gram[0, h])[1] for h in range(cfg.H)]])
    rer, _, _ = oracle.fitness(_ocfg(cfg), hist_h)
    print(f"  {kind}: sweeps {sweeps.ravel().tolist()} oracle {rsweeps.ravel().tolist()}")
    np.testing.assert_array_equal(sweeps, rsweeps)
    # A rank-1 Gram's other 63 eigenvalues sit at the fp64 rounding floor of its sums
    # (whose order differs between the two), and enter the rank through their square
    # roots: agreement to 1e-5 there, still far inside the 0.01 of buildplan.md:289.
    tol = 1e-5 if kind == "rank1" else 1e-6
    np.testing.assert_allclose(er, rer, rtol=tol, atol=tol)
    if kind == "diagonal":
        assert (sweeps == 1).all()
    elif kind == "rank1_plus_noise":
        assert (sweeps == 30).all()


def test_fitness_closed_forms():
    cfg = _cfg("fitcf", B=1, G=16, D=64, dtype="fp32")
    X = make_state(cfg, seed=5)
    with _engine(cfg) as e:
        hist = torch.from_numpy(np.stack([X, X, X])).cuda().contiguous()
        er, coh, fit = e.fitness(hist)
        np.testing.assert_allclose(_host(coh), 1.0, atol=1e-5)
        hist2 = torch.from_numpy(np.stack([X - 0.5, 0.5 - X])).cuda().contiguous()
        _, coh2, _ = e.fitness(hist2)
        np.testing.assert_allclose(_host(coh2), 0.0, atol=1e-5)


# ---- organism adapters ----------------------------------------------------------------------------

def test_field_adapters_match_oracle(oracle):
    cfg = _cfg("field", B=1, G=32, D=64, dtype="fp32")
    conc = np.random.default_rng(3).random((32, 32), dtype=np.float32)
    with _engine(cfg) as e:
        x = e.init_from_field(torch.from_numpy(conc))
        c2 = e.field_from_state(x)
        torch.cuda.synchronize()
        X, C2 = _host(x), _host(c2)
    ref = oracle.init_from_field(conc, cfg.C)
    assert norm_err(X, ref) <= 1e-6
    # The channel mean of conc*sin(0.1c) cancels heavily (|mean| << mean |X|): bound
    # the error by fp32 summation noise relative to the magnitudes summed.
    scale = np.abs(ref).mean(axis=-1)
    assert np.max(np.abs(C2 - oracle.field_from_state(ref)) / scale) <= 1e-6


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_get_state_reads_back_the_field_of_a_state(oracle, dtype):
    # get_ca_state (slime/runtime.cu:479-504) copies the organism's concentration,
    # which after a generation is mean_c of the CA output (organism.cu:723-743).
    cfg = _cfg("view", B=1, G=32, D=64, dtype=dtype)
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, dtype))  # on torch's stream; get_state waits for the device
        full = e.get_state(y)
        part = e.get_state(y, size=100)
        none = e.get_state(y, size=0)
        conc = _host(e.field_from_state(y))
        Y = _host(y)
        with pytest.raises(Exception):
            e.get_state(y, size=cfg.G * cfg.G + 1)
        with pytest.raises(Exception):
            e.get_state(y, size=-1)
    assert full.shape == (cfg.G * cfg.G,) and part.shape == (100,) and none.shape == (0,)
    np.testing.assert_array_equal(full, conc.reshape(-1))
    np.testing.assert_array_equal(part, full[:100])
    ref = oracle.field_from_state(Y[0]).reshape(-1)
    assert np.max(np.abs(full - ref)) <= 1e-6 * np.max(np.abs(ref))


@pytest.mark.parametrize("D", [8, 64])
def test_neural_ca_update_matches_oracle_organism_sequence(oracle, D):
    """slime_neural_ca_update = init-from-field -> one step -> field update -> mean
    per-head effective rank (slime/core/organism.cu:617-688), against the same
    sequence composed from the oracle."""
    cfg = _cfg("organism", B=1, G=32, D=D, dtype="fp32")
    p = make_params(cfg, seed=1)
    conc0 = np.random.default_rng(5).random((32, 32), dtype=np.float32)
    gen = 2
    with _engine(cfg) as e:
        e.set_params(p)
        conc = torch.from_numpy(conc0).cuda()
        xin = torch.empty((32, 32, cfg.C), dtype=torch.float32, device="cuda")
        xout = torch.empty_like(xin)
        hist = torch.full((4,), -1.0, dtype=torch.float32, device="cuda")
        mass = torch.empty(8, dtype=torch.float32, device="cuda")
        e.neural_ca_update(conc, xin, xout, hist, gen, mass_buffer=mass)
        torch.cuda.synchronize()
        Xin, Xout, C1, Hs, Ms = _host(xin), _host(xout), _host(conc), _host(hist), _host(mass)
        from slime_amd._lib import SlimeError
        with pytest.raises(SlimeError, match="distinct"):
            e.neural_ca_update(conc, xin, xin, hist, 0)
    ocfg = _ocfg(cfg)
    Xref = oracle.init_from_field(conc0, cfg.C)[None]
    Yref, _, rmo = oracle.step(ocfg, Xref, p, 1)
    # The Gram of this field-initialised state is nearly singular per head, where the
    # reference's absolute 1e-6 Jacobi threshold makes the rank sensitive to the last
    # bits of the state: score the GPU's own states with the oracle.
    rer, _, _ = oracle.fitness(ocfg, np.stack([Xin[None], Xout[None]]))
    assert norm_err(Xin, Xref[0]) <= 1e-6
    assert norm_err(Xout, Yref[0]) <= TOL["fp32"]
    scale = np.abs(Yref[0]).mean(axis=-1)
    assert np.max(np.abs(C1 - oracle.field_from_state(Yref[0])) / scale) <= 1e-5
    # Head masses of conc*sin(0.1c) cancel (head 0: 4.9 against sum|X| ~ 1e4): bound
    # the error relative to the magnitudes summed.
    absmass = np.abs(Xref[0].astype(np.float64)).reshape(-1, cfg.H, cfg.D).sum(axis=(0, 2))
    assert np.all(np.abs(Ms - rmo[0]) <= 1e-6 * absmass), (Ms, rmo[0])
    print(f"  erank history entry {Hs[gen]:.6f} vs oracle {rer.mean():.6f}")
    assert abs(Hs[gen] - rer.mean()) <= 1e-5
    assert np.all(Hs[[0, 1, 3]] == -1.0)


# ---- full-size throughput shape: size-independent properties --------------------------------------

C3_ENTRIES = [0, 21, 42, 63]  # batch entries of c3 compared with the oracle


def _rms_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.sqrt(np.mean((got - ref) ** 2)) / np.sqrt(np.mean(ref ** 2)))


def test_c3_shape_conserves_mass_and_matches_oracle_on_four_batches(oracle):
    # One step of the full c3 shape (64 x 128 x 128, bf16): four batch entries spread
    # over the batch (and so over the stencil's tile tickets) against the oracle.
    from slime_amd import CONFIGS
    cfg = CONFIGS["c3"]
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        y = e.forward(x)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        assert bool(torch.isfinite(y.float()).all())
        Ys = _host(y[C3_ENTRIES])
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    sub = _ocfg(cfg, B=len(C3_ENTRIES))
    ref, rmi, _ = oracle.step(sub, X[C3_ENTRIES], p, 1)
    for j, b in enumerate(C3_ENTRIES):
        err = norm_err(Ys[j], ref[j])
        print(f"  batch {b} of c3: normalised error {err:.3e}")
        assert err <= TOL["bf16"], b
    np.testing.assert_allclose(mi[C3_ENTRIES], rmi, rtol=1e-6)


def test_c3_two_step_call_matches_oracle_on_four_batches(oracle):
    # The benched call's code path over two steps: step 2 reads step 1's unscaled
    # bf16 output with its mass scale folded into the weights and the stencil's loads,
    # the last step is written in fp32 and rescaled once into the bf16 state. Over
    # two steps the oracle's own trajectory with bf16-rounded states stays within
    # 1.0e-2 of its fp32 one, so the bf16 bar still measures the device there.
    from slime_amd import CONFIGS
    cfg = CONFIGS["c3"]
    p, X = _prep(cfg)
    with _engine(cfg) as e:
        e.set_params(p)
        y = e.forward(_dev(X, "bf16"), n_steps=2)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        Ys = _host(y[C3_ENTRIES])
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    ref, _, _ = oracle.step(_ocfg(cfg, B=len(C3_ENTRIES)), X[C3_ENTRIES], p, 2)
    for j, b in enumerate(C3_ENTRIES):
        err = norm_err(Ys[j], ref[j])
        print(f"  batch {b} of c3 after 2 steps: normalised error {err:.3e}")
        assert err <= TOL["bf16"], b


def test_c3_bench_call_conserves_mass_repeats_bitwise_and_tracks_oracle(oracle):
    """The benched call: 10 chained c3 steps in one slime_ca_step (each step's mass
    scale folded into the next step's weights and loads, the last step written in
    fp32 and rescaled once), run twice on one handle.

    * every value finite; the stored state's per-(batch, head) sums equal the
      input's up to one bf16 rounding of each element; the second call repeats the
      first bit for bit (the stencil's tile tickets decide which workgroup runs a
      tile, never what it computes);
    * batch entry 0 against the oracle's 10 steps. The map is chaotic at bf16
      resolution: the oracle's own trajectory with every state rounded to bf16 ends
      2.9e-1 (max-normalised) from its fp32 trajectory after 10 steps, so a
      max-norm bar there tests nothing. The RMS difference grows slowly (1.6e-3
      after one step, 9.4e-3 after ten), and the device is held to 3x the RMS
      difference of that bf16-state oracle trajectory, computed here."""
    from slime_amd import CONFIGS
    cfg = CONFIGS["c3"]
    p, X = _prep(cfg)

    def head_sums(t):
        return t.to(torch.float64).reshape(cfg.B, -1, cfg.H, cfg.D).sum(dim=(1, 3)).cpu().numpy()

    with _engine(cfg) as e:
        e.set_params(p)
        x = _dev(X, "bf16")
        y1 = e.forward(x, n_steps=10)
        y2 = e.forward(x, n_steps=10)
        torch.cuda.synchronize()
        mi, mo = e.mass()
        assert bool(torch.isfinite(y1.float()).all())
        assert torch.equal(y1, y2)
        s_in, s_out = head_sums(x), head_sums(y1)
        Y0 = _host(y1[0:1])
    np.testing.assert_allclose(mo, mi, rtol=1e-6)
    drift = np.abs(s_out - s_in) / np.abs(s_in)
    print(f"  10 chained c3 steps: max relative drift of the stored head sums {drift.max():.2e}")
    assert drift.max() <= 5e-5
    one = _ocfg(cfg, B=1)
    ref, cur = X[0:1], X[0:1]
    for _ in range(10):
        ref = oracle.step(one, ref, p, 1)[0]
        cur = round_bf16(oracle.step(one, cur, p, 1)[0])
    spread = _rms_err(cur, ref)
    err = _rms_err(Y0, ref)
    print(f"  batch 0 after 10 steps: RMS-normalised error {err:.3e} (max-normalised "
          f"{norm_err(Y0, ref):.3e}); bf16-state oracle trajectory {spread:.3e} "
          f"(max-normalised {norm_err(cur, ref):.3e})")
    assert err <= 3.0 * spread
