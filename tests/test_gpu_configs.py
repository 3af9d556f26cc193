"""GPU parity on the BASELINE workloads at their real sizes: c2 (the README
configuration: 128x128, fp32, per-cell growth parameters, 100 steps) and c4 (the
ensemble: 16 pods with their own weights on one shared 128x128 grid, bf16, an
8-state history scored by the fused fitness). Everything goes through the C ABI
and is compared with the CPU oracle on the same seeded inputs.

Chained steps and the oracle. The flow-Lenia map is sensitive to its input: the
bell growth's slope reaches 1/sigma (sigma as small as 0.01), so a relative input
perturbation at fp32 rounding grows about tenfold per step (measured on the
oracle itself below). After n chained steps an fp32 device and the fp64 oracle can
therefore differ by the oracle's own amplification of rounding noise, not by a
fixed 1e-5. Each step is therefore checked one at a time, the oracle starting
from the device's previous state (tolerance 1e-5 fp32, 2e-2 bf16), and a chained
n-step result is held to a bound scaled by the oracle's measured sensitivity to
a unit-roundoff perturbation of the input.
"""
import numpy as np
import pytest

from slime_amd import CONFIGS, Pseudopod, make_params, make_state, round_bf16
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = {"fp32": 1e-5, "bf16": 2e-2}


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _engine(cfg):
    print(f"[case] {cfg.name} B={cfg.B} G={cfg.G} D={cfg.D} {cfg.dtype} pods={cfg.pods} "
          f"per_cell={cfg.growth_per_cell}", flush=True)
    return Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, cfg.growth_per_cell,
                     cfg.pods)


def _ocfg(cfg, **kw):
    from oracle import OracleConfig
    base = dict(B=cfg.B, G=cfg.G, H=cfg.H, D=cfg.D, pods=cfg.pods,
                growth_per_cell=cfg.growth_per_cell, dt=cfg.dt)
    base.update(kw)
    return OracleConfig(**base)


def _head_sums(t, H):
    """Per-(batch, head) sums of a [B, G, G, C] device state, in fp64."""
    B = t.shape[0]
    return t.double().reshape(B, -1, H, t.shape[-1] // H).sum(dim=(1, 3)).cpu().numpy()


def _pod_params(p, pod):
    return {k: v[pod:pod + 1] for k, v in p.items()}


# ---- c2: README configuration ---------------------------------------------------------------

def test_c2_readme_workload(oracle):
    """c2: B 1, 128x128, H 8, D 64, fp32, per-cell mu and sigma, blobs.

    * one step and ten single steps, each against the oracle from the device's
      previous state (1e-5);
    * one call of 10 steps (the device folds each step's mass scale into the next)
      against the oracle's 10 steps, within the oracle's own sensitivity;
    * 100 single-step calls with the per-head mass checked after every step;
    * the 100-step difference from the oracle's 100 steps is printed.

    Mass. This configuration's state grows from step to step (in the oracle too:
    max|x| ~ 6 after 10 steps, ~3e5 after 70, with sum|x| / |sum x| ~ 6e4 per
    head), while the head sums stay fixed. Every stored element is one fp32
    rounding of the conserved value, so the stored sum scatters around the
    conserved one with a standard deviation of at most u sqrt(sum x^2 / 3)
    (u = 2^-24), which exceeds 1e-6 |sum x| once the values are ~1e4 times their
    mean. Each step is therefore held to max(1e-6 |sum|, 10 such deviations): the
    device's input sums against the host's fp64 sums of the stored input, and the
    stored output against the input, and the drift from the initial state to
    the same bound accumulated over the steps."""
    cfg = CONFIGS["c2"]
    p = make_params(cfg, seed=1)
    X = make_state(cfg, seed=2)
    ocfg = _ocfg(cfg)
    states = [X]
    u = 2.0 ** -24
    with _engine(cfg) as e:
        e.set_params(p)
        x0 = torch.from_numpy(X).cuda()
        m0 = _head_sums(x0, cfg.H)
        cur, nxt = x0.clone(), torch.empty_like(x0)
        m_prev = m0
        sd_prev = u * np.sqrt(_head_sums(x0.double() ** 2, cfg.H) / 3.0)
        worst_step, worst_total, var_total = 0.0, 0.0, np.zeros((1, cfg.H))
        for i in range(100):
            e.forward(cur, out=nxt)
            mi, mo = e.mass()
            ms = _head_sums(nxt, cfg.H)
            sd = u * np.sqrt(_head_sums(nxt.double() ** 2, cfg.H) / 3.0)  # rounding scatter
            var_total += sd ** 2
            bound_in = np.maximum(1e-6 * np.abs(m_prev), 10.0 * sd_prev)
            bound = np.maximum(1e-6 * np.abs(m_prev), 10.0 * sd)
            np.testing.assert_allclose(mo, mi, rtol=1e-12)
            assert np.all(np.abs(mi - m_prev) <= bound_in), (i, np.abs(mi - m_prev) / bound_in)
            assert np.all(np.abs(ms - mi) <= bound), (i, np.abs(ms - mi) / bound)
            assert np.all(np.abs(ms - m0) <= np.maximum(1e-6 * np.abs(m0), 10.0 * np.sqrt(var_total))), i
            worst_step = max(worst_step, float(np.max(np.abs(ms - mi) / np.abs(mi))))
            worst_total = max(worst_total, float(np.max(np.abs(ms - m0) / np.abs(m0))))
            if i < 10:
                states.append(nxt.cpu().numpy())
            m_prev, sd_prev = ms, sd
            cur, nxt = nxt, cur
        Y100 = cur.cpu().numpy()
        y10 = e.forward(x0, n_steps=10)
        torch.cuda.synchronize()
        mi10, mo10 = e.mass()
        Y10 = y10.cpu().numpy()
    print(f"  mass over 100 single steps: worst per-step relative drift {worst_step:.2e}, "
          f"worst drift from the initial state {worst_total:.2e}")
    # 10 steps in one call: the state is still small there (max|x| ~ 6)
    np.testing.assert_allclose(mo10, mi10, rtol=1e-12)
    np.testing.assert_allclose(_head_sums(torch.from_numpy(Y10), cfg.H), m0, rtol=1e-6)

    # one step at a time along the device's trajectory
    errs = []
    for i in range(10):
        ref, rmi, _ = oracle.step(ocfg, states[i], p, 1)
        errs.append(norm_err(states[i + 1], ref))
        np.testing.assert_allclose(_head_sums(torch.from_numpy(states[i]), cfg.H), rmi, rtol=1e-9)
    print(f"  single steps vs oracle from the device's previous state: "
          f"{', '.join(f'{v:.1e}' for v in errs)}")
    assert max(errs) <= TOL["fp32"], errs

    # chained: 10 steps in one call, against the oracle's 10 steps and the oracle's
    # own spread under a unit-roundoff perturbation of the input
    ref10, _, _ = oracle.step(ocfg, X, p, 10)
    rng = np.random.default_rng(7)
    Xp = (X * (1.0 + 2.0 ** -24 * rng.standard_normal(X.shape))).astype(np.float32)
    pert10, _, _ = oracle.step(ocfg, Xp, p, 10)
    sens10 = norm_err(pert10, ref10)
    err10_call = norm_err(Y10, ref10)
    err10_chain = norm_err(states[10], ref10)
    print(f"  10 steps: one call {err10_call:.2e}, ten calls {err10_chain:.2e}; oracle under a "
          f"unit-roundoff input perturbation {sens10:.2e}")
    assert err10_call <= max(TOL["fp32"], 20.0 * sens10)
    assert err10_chain <= max(TOL["fp32"], 20.0 * sens10)

    ref100, _, _ = oracle.step(ocfg, X, p, 100)
    print(f"  100 single steps vs the oracle's 100 steps: normalised error "
          f"{norm_err(Y100, ref100):.2e} (printed, not asserted: chaotic amplification)")


# ---- c4: the ensemble ---------------------------------------------------------------------

def test_c4_ensemble_workload(oracle):
    """c4: 16 pods (batch entry = pod) with independent weights on one shared
    128x128 grid, D 64, bf16. Seven single steps build an 8-state history; after
    each, three pods are checked against the oracle from the device's previous
    state (2e-2) and every (pod, head) mass to 1e-6; then the fused fitness of
    the device's own history against the oracle for all 128 (pod, head), with
    equal Jacobi sweep counts. At G = 128 every fitness chunk spans 16 stages of
    64 cells, so the Gram and moment sums accumulate across stages."""
    cfg = CONFIGS["c4"]
    p = make_params(cfg, seed=1)
    p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
    X1 = round_bf16(make_state(cfg, seed=2, B=1))
    T = cfg.steps
    with _engine(cfg) as e:
        e.set_params(p)
        hist = torch.empty((T, cfg.B, cfg.G, cfg.G, cfg.C), dtype=torch.bfloat16, device="cuda")
        hist[0] = torch.from_numpy(X1).cuda().to(torch.bfloat16).expand(cfg.B, -1, -1, -1)
        for t in range(1, T):
            e.forward(hist[t - 1], out=hist[t])
            mi, mo = e.mass()
            np.testing.assert_allclose(mo, mi, rtol=1e-6)
            np.testing.assert_allclose(mi, _head_sums(hist[t - 1], cfg.H), rtol=1e-6)
            drift = np.abs(_head_sums(hist[t], cfg.H) - mi) / np.abs(mi)
            assert np.all(drift <= 5e-5), (t, drift.max())
        er, coh, fit = e.fitness(hist)
        torch.cuda.synchronize()
        sweeps = e.jacobi_sweeps()
        Hh = hist.float().cpu().numpy()
        er, coh, fit = (v.cpu().numpy() for v in (er, coh, fit))

    one = _ocfg(cfg, B=1, pods=1)
    worst = 0.0
    for t in range(1, T):
        for pod in sorted({(3 * t) % cfg.pods, (3 * t + 7) % cfg.pods, (5 * t + 2) % cfg.pods}):
            ref, rmi, _ = oracle.step(one, Hh[t - 1][pod:pod + 1], _pod_params(p, pod), 1)
            err = norm_err(Hh[t][pod:pod + 1], ref)
            worst = max(worst, err)
            assert err <= TOL["bf16"], (t, pod, err)
    print(f"  worst single-step error over the checked pods {worst:.2e}")

    ocfg = _ocfg(cfg)
    rer, rcoh, rfit = oracle.fitness(ocfg, Hh)
    gram = oracle.gram(ocfg, Hh[-1])
    rsweeps = np.array([[oracle.jacobi_eigs(gram[b, h])[1] for h in range(cfg.H)]
                        for b in range(cfg.B)])
    print(f"  fitness: erank {er.mean():.4f} (oracle {rer.mean():.4f}), coherence "
          f"{coh.mean():.6f} (oracle {rcoh.mean():.6f}); max |d erank| "
          f"{np.max(np.abs(er - rer)):.2e}, max |d coh| {np.max(np.abs(coh - rcoh)):.2e}")
    np.testing.assert_array_equal(sweeps, rsweeps)
    np.testing.assert_allclose(er, rer, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(coh, rcoh, atol=1e-6)
    np.testing.assert_allclose(fit, rfit, rtol=1e-6, atol=1e-6)


# ---- fitness with several 64-cell stages per chunk ----------------------------------------------

@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_fitness_multi_stage_chunks(oracle, dtype, G):
    """G = 64 gives 4 stages of 64 cells per fitness chunk, G = 128 gives 16: the
    per-thread Gram blocks and fp64 moment sums carry across stages (and across
    the LDS staging barriers of each stage)."""
    from slime_amd.synthetic import CAConfig
    cfg = CAConfig("fitms", B=2, G=G, H=8, D=64, dtype=dtype, steps=1, w_std=0.05, blobs=True)
    p = make_params(cfg, seed=4)
    X = make_state(cfg, seed=5)
    if dtype == "bf16":
        p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
        X = round_bf16(X)
    T = 4
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    with _engine(cfg) as e:
        e.set_params(p)
        hist = torch.empty((T, cfg.B, G, G, cfg.C), dtype=tdt, device="cuda")
        hist[0] = torch.from_numpy(X).cuda().to(tdt)
        for t in range(1, T):
            e.forward(hist[t - 1], out=hist[t])
        er, coh, fit = e.fitness(hist)
        torch.cuda.synchronize()
        sweeps = e.jacobi_sweeps()
        Hh = hist.float().cpu().numpy()
        er, coh, fit = (v.cpu().numpy() for v in (er, coh, fit))
    ocfg = _ocfg(cfg)
    rer, rcoh, rfit = oracle.fitness(ocfg, Hh)
    gram = oracle.gram(ocfg, Hh[-1])
    rsweeps = np.array([[oracle.jacobi_eigs(gram[b, h])[1] for h in range(cfg.H)]
                        for b in range(cfg.B)])
    print(f"  G={G} {dtype}: max |d erank| {np.max(np.abs(er - rer)):.2e}, "
          f"max |d coh| {np.max(np.abs(coh - rcoh)):.2e}, sweeps {sweeps.ravel()[:4]}")
    np.testing.assert_array_equal(sweeps, rsweeps)
    np.testing.assert_allclose(er, rer, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(coh, rcoh, atol=1e-6)
    np.testing.assert_allclose(fit, rfit, rtol=1e-6, atol=1e-6)


def test_c4_rollout_matches_oracle_and_single_steps(oracle):
    """slime_ca_rollout on the c4 workload: 7 steps into an 8-state history, each state
    stored before its mass rescale with its factor in `scales`. The completed states
    (factor x stored values) are checked step by step against the oracle from the
    previous completed state (2e-2), their head sums against the input's (1e-6: the
    factor is applied in fp64 here, so the bf16 storage rounding does not enter the
    sums), the first state against the single-step path (the two differ only in where
    the bf16 rounding falls: before or after the factor, at most one bf16 unit), and
    the scaled fitness against the oracle's fitness of the completed states (1e-6,
    equal Jacobi sweep counts)."""
    cfg = CONFIGS["c4"]
    p = make_params(cfg, seed=1)
    p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
    X1 = round_bf16(make_state(cfg, seed=2, B=1))
    T = cfg.steps
    with _engine(cfg) as e:
        e.set_params(p)
        x0 = torch.from_numpy(X1).cuda().to(torch.bfloat16).expand(cfg.B, -1, -1, -1).contiguous()
        hist = torch.empty((T,) + tuple(x0.shape), dtype=torch.bfloat16, device="cuda")
        hist[0] = x0
        scales = e.rollout(hist)
        er, coh, fit = e.fitness_scaled(hist, scales)
        torch.cuda.synchronize()
        sweeps = e.jacobi_sweeps()
        y1 = e.forward(x0)  # the single-step path's first state
        torch.cuda.synchronize()
        S = scales.cpu().numpy()
        true = hist.double().view(T, cfg.B, cfg.G * cfg.G, cfg.H, cfg.D) * scales.view(T, cfg.B, 1, cfg.H, 1)
        sums = true.sum(dim=(2, 4)).cpu().numpy()
        truef = true.float().view(T, cfg.B, cfg.G, cfg.G, cfg.C).cpu().numpy()
        del true
        Y1 = y1.float().cpu().numpy()
        er, coh, fit = (v.cpu().numpy() for v in (er, coh, fit))
    assert np.all(S[0] == 1.0) and np.all(S > 0)
    drift = np.max(np.abs(sums[1:] - sums[0]) / np.abs(sums[0]))
    print(f"  rollout: factors in [{S[1:].min():.6f}, {S[1:].max():.6f}], head-mass drift over 7 steps {drift:.2e}")
    assert drift <= 1e-6
    e1 = norm_err(truef[1], Y1)
    print(f"  first state against the single-step path: normalised difference {e1:.2e}")
    assert e1 <= 2.0 ** -7
    one = _ocfg(cfg, B=1, pods=1)
    worst = 0.0
    for t in range(1, T):
        for pod in sorted({(3 * t) % cfg.pods, (5 * t + 2) % cfg.pods}):
            ref, _, _ = oracle.step(one, truef[t - 1][pod:pod + 1], _pod_params(p, pod), 1)
            err = norm_err(truef[t][pod:pod + 1], ref)
            worst = max(worst, err)
            assert err <= TOL["bf16"], (t, pod, err)
    print(f"  worst single-step error over the checked pods {worst:.2e}")
    ocfg = _ocfg(cfg)
    rer, rcoh, rfit = oracle.fitness(ocfg, truef)
    gram = oracle.gram(ocfg, truef[-1])
    rsweeps = np.array([[oracle.jacobi_eigs(gram[b, h])[1] for h in range(cfg.H)]
                        for b in range(cfg.B)])
    print(f"  fitness: max |d erank| {np.max(np.abs(er - rer)):.2e}, max |d coh| {np.max(np.abs(coh - rcoh)):.2e}")
    np.testing.assert_array_equal(sweeps, rsweeps)
    np.testing.assert_allclose(er, rer, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(coh, rcoh, atol=1e-6)
    np.testing.assert_allclose(fit, rfit, rtol=1e-6, atol=1e-6)
