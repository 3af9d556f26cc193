"""CPU tests that pin the oracle (oracle/ca_oracle.cpp) before it is trusted.

Each stage is checked against a library routine that computes the same thing
independently (numpy matmul, scipy.ndimage.correlate in wrap mode, LAPACK
eigvalsh, numpy corrcoef) and against closed forms chosen so that a dropped term,
a wrong sign, a transposed operand or a wrong neighbour index fails.
"""
import math

import numpy as np
import pytest
from scipy import ndimage

from tests.conftest import norm_err

from oracle import OracleConfig

H = 8


def _rng(seed):
    return np.random.default_rng(seed)


def _params(cfg, seed=3, w_std=0.1):
    r = _rng(seed)
    C = cfg.C
    g = (cfg.pods, cfg.G, cfg.G, H) if cfg.growth_per_cell else (cfg.pods, H)
    return {
        "WP": r.normal(0, w_std, (cfg.pods, C, C)).astype(np.float32),
        "WI": r.normal(0, w_std, (cfg.pods, C, C)).astype(np.float32),
        "WV": r.normal(0, w_std, (cfg.pods, C, C)).astype(np.float32),
        "K": r.normal(0, w_std, (cfg.pods, H, 9)).astype(np.float32),
        "mu": r.uniform(0.1, 0.3, g).astype(np.float32),
        "sigma": r.uniform(0.01, 0.05, g).astype(np.float32),
        "M": (np.eye(H)[None] + r.normal(0, 0.01, (cfg.pods, H, H))).astype(np.float32),
    }


def _state(cfg, seed=4):
    return _rng(seed).random((cfg.B, cfg.G, cfg.G, cfg.C), dtype=np.float32)


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


# ---- S1 projections ------------------------------------------------------------------

@pytest.mark.parametrize("D,pods,chain", [(8, 1, False), (16, 2, False), (8, 1, True)])
def test_project_matches_numpy_matmul(oracle, D, pods, chain):
    cfg = OracleConfig(B=2, G=8, H=H, D=D, pods=pods, pvi_chain=chain)
    p, X = _params(cfg), _state(cfg)
    P, I, V = oracle.project(cfg, X, p["WP"], p["WI"], p["WV"])
    Xd = X.astype(np.float64).reshape(cfg.B, -1, cfg.C)
    for b in range(cfg.B):
        q = b // (cfg.B // pods)
        x = Xd[b]
        rp = np.maximum(x @ p["WP"][q].astype(np.float64), 0)
        ri = _gelu((rp if chain else x) @ p["WI"][q].astype(np.float64))
        rv = (ri if chain else x) @ p["WV"][q].astype(np.float64)
        assert norm_err(P[b].reshape(-1, cfg.C), rp) < 1e-6
        assert norm_err(I[b].reshape(-1, cfg.C), ri) < 1e-6
        assert norm_err(V[b].reshape(-1, cfg.C), rv) < 1e-6


@pytest.mark.parametrize("pods", [1, 2])
def test_project_perception_sum_matches_scipy_wrap_filter(oracle, pods):
    """pvi_chain 2: P = ReLU(S W_P) with S = 9 x the 3 x 3 wrap-mode box mean of X
    (scipy.ndimage.uniform_filter), then the chain I = GELU(P W_I), V = I W_V."""
    cfg = OracleConfig(B=2, G=8, H=H, D=8, pods=pods, pvi_chain=2)
    p, X = _params(cfg), _state(cfg)
    P, I, V = oracle.project(cfg, X, p["WP"], p["WI"], p["WV"])
    for b in range(cfg.B):
        q = b // (cfg.B // pods)
        S = 9.0 * ndimage.uniform_filter(X[b].astype(np.float64), size=(3, 3, 1), mode="wrap")
        S = S.reshape(-1, cfg.C)
        rp = np.maximum(S @ p["WP"][q].astype(np.float64), 0)
        ri = _gelu(rp @ p["WI"][q].astype(np.float64))
        rv = ri @ p["WV"][q].astype(np.float64)
        for got, ref in ((P, rp), (I, ri), (V, rv)):
            np.testing.assert_allclose(got[b].reshape(-1, cfg.C), ref, rtol=1e-5, atol=1e-6)


def test_project_identity_weights(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=8)
    X = _state(cfg) - 0.5
    eye = np.eye(cfg.C, dtype=np.float32)[None]
    P, I, V = oracle.project(cfg, X, eye, eye, eye)
    np.testing.assert_allclose(P, np.maximum(X, 0), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(V, X, rtol=1e-6, atol=1e-7)
    # tanh-GELU against an independent implementation (torch's), not a retyped formula
    import torch
    ref = torch.nn.functional.gelu(torch.from_numpy(X.astype(np.float64)), approximate="tanh").numpy()
    np.testing.assert_allclose(I, ref, rtol=1e-6, atol=1e-7)


def test_project_block_diagonal_is_per_head_form(oracle):
    """Block-diagonal dense W equals per-head D x D projections (the reference's
    per-head 64-wide loops, slime/core/pseudopod.cu:84,101)."""
    cfg = OracleConfig(B=1, G=8, H=H, D=8)
    r = _rng(7)
    blocks = r.normal(0, 0.1, (H, cfg.D, cfg.D)).astype(np.float32)
    W = np.zeros((1, cfg.C, cfg.C), np.float32)
    for h in range(H):
        W[0, h * cfg.D:(h + 1) * cfg.D, h * cfg.D:(h + 1) * cfg.D] = blocks[h]
    X = _state(cfg)
    P, _, V = oracle.project(cfg, X, W, W, W)
    for h in range(H):
        xh = X[..., h * cfg.D:(h + 1) * cfg.D].astype(np.float64)
        np.testing.assert_allclose(V[..., h * cfg.D:(h + 1) * cfg.D], xh @ blocks[h], rtol=1e-5,
                                   atol=1e-6)
        np.testing.assert_allclose(P[..., h * cfg.D:(h + 1) * cfg.D],
                                   np.maximum(xh @ blocks[h], 0), rtol=1e-5, atol=1e-6)


# ---- S2 potential ----------------------------------------------------------------------

def test_potential_matches_scipy_wrap_correlate(oracle):
    cfg = OracleConfig(B=2, G=8, H=H, D=4, pods=2)
    p, X = _params(cfg), _state(cfg)
    U = oracle.potential(cfg, X, p["K"])
    for b in range(cfg.B):
        for h in range(H):
            k = p["K"][b, h].reshape(3, 3).astype(np.float64)  # pod = b (per_pod = 1)
            for c in range(cfg.D):
                ref = ndimage.correlate(X[b, :, :, h * cfg.D + c].astype(np.float64), k,
                                        mode="wrap")
                np.testing.assert_allclose(U[b, :, :, h * cfg.D + c], ref, rtol=1e-5, atol=1e-6)


def test_potential_centre_tap_and_shift_equivariance(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=4)
    X = _state(cfg)
    K = np.zeros((1, H, 9), np.float32)
    K[..., 4] = 1.0
    np.testing.assert_array_equal(oracle.potential(cfg, X, K), X)
    K = _params(cfg)["K"]
    U = oracle.potential(cfg, X, K)
    Xs = np.roll(X, (2, -3), axis=(1, 2))
    np.testing.assert_allclose(oracle.potential(cfg, Xs, K), np.roll(U, (2, -3), axis=(1, 2)),
                               rtol=1e-6, atol=1e-7)
    # tap (dy=-1, dx=+1) alone reads the cell above-right
    K = np.zeros((1, H, 9), np.float32)
    K[..., 2] = 1.0
    np.testing.assert_array_equal(oracle.potential(cfg, X, K), np.roll(X, (1, -1), axis=(1, 2)))


# ---- S3 growth -------------------------------------------------------------------------

def test_growth_closed_forms(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=2)
    mu = np.full((1, H), 0.2, np.float32)
    sigma = np.full((1, H), 0.03, np.float32)
    U = np.full((1, 8, 8, cfg.C), 0.2, np.float32)
    np.testing.assert_allclose(oracle.growth(cfg, U, mu, sigma), 1.0, atol=1e-6)
    U = np.full((1, 8, 8, cfg.C), 5.0, np.float32)
    np.testing.assert_allclose(oracle.growth(cfg, U, mu, sigma), -1.0, atol=1e-6)
    d = 0.017
    g1 = oracle.growth(cfg, np.full((1, 8, 8, cfg.C), 0.2 + d, np.float32), mu, sigma)
    g2 = oracle.growth(cfg, np.full((1, 8, 8, cfg.C), 0.2 - d, np.float32), mu, sigma)
    np.testing.assert_allclose(g1, g2, atol=1e-5)
    z = d / (0.03 + 1e-7)
    np.testing.assert_allclose(g1, 2 * math.exp(-z * z) - 1, atol=1e-5)


def test_growth_gaussian_closed_forms(oracle):
    """growth_fn 1, exp(-(U - mu)^2 / (2 sigma^2)) (failed_attempts/pseudopod.cu:46-48):
    1 at mu, exp(-1/2) one sigma away on either side, exp(-2) at two sigma, and no
    offset (the bell's 2 g - 1 would give 1, 0.213, -0.73 there)."""
    cfg = OracleConfig(B=1, G=8, H=H, D=2, growth_fn=1)
    mu = np.full((1, H), 0.2, np.float32)
    sigma = np.full((1, H), 0.03, np.float32)

    def g_at(u):
        return oracle.growth(cfg, np.full((1, 8, 8, cfg.C), u, np.float32), mu, sigma)

    np.testing.assert_allclose(g_at(0.2), 1.0, atol=1e-6)
    np.testing.assert_allclose(g_at(0.23), math.exp(-0.5), rtol=1e-5)
    np.testing.assert_allclose(g_at(0.17), math.exp(-0.5), rtol=1e-5)
    np.testing.assert_allclose(g_at(0.26), math.exp(-2.0), rtol=1e-5)
    np.testing.assert_allclose(g_at(5.0), 0.0, atol=1e-30)


def test_growth_shipped_closed_forms(oracle):
    """growth_fn 2, the shipped kernel's U exp(-U^2) (slime/core/pseudopod.cu:183):
    odd, zero at 0, +-1/e at +-1, its maximum exp(-1/2)/sqrt(2) at 1/sqrt(2); mu and
    sigma play no part."""
    cfg = OracleConfig(B=1, G=8, H=H, D=2, growth_fn=2)
    r = _rng(13)
    mu = r.uniform(0.1, 0.3, (1, H)).astype(np.float32)
    sigma = r.uniform(0.01, 0.05, (1, H)).astype(np.float32)

    def g_at(u):
        return oracle.growth(cfg, np.full((1, 8, 8, cfg.C), u, np.float32), mu, sigma)

    np.testing.assert_allclose(g_at(0.0), 0.0, atol=1e-30)
    np.testing.assert_allclose(g_at(1.0), math.exp(-1.0), rtol=1e-6)
    np.testing.assert_allclose(g_at(-1.0), -math.exp(-1.0), rtol=1e-6)
    np.testing.assert_allclose(g_at(2 ** -0.5), math.exp(-0.5) * 2 ** -0.5, rtol=1e-6)
    U = r.normal(0, 1, (1, 8, 8, cfg.C)).astype(np.float32)
    np.testing.assert_allclose(oracle.growth(cfg, -U, mu, sigma), -oracle.growth(cfg, U, mu, sigma),
                               rtol=1e-6)
    for u in (0.6, 0.7, 0.75, 0.9):  # 1/sqrt(2) = 0.7071 is the maximum
        assert g_at(u).max() <= math.exp(-0.5) * 2 ** -0.5 + 1e-7


@pytest.mark.parametrize("D,per_cell", [(64, False), (16, True)])
def test_growth_variant_case_tells_the_functions_apart(oracle, D, per_cell):
    """On the inputs of the GPU growth-variant cases (tests.conftest.
    growth_variant_params), one step with each growth function differs from the
    others by more than 5x the bf16 bar, and a Gaussian with sigma^2 in place of
    2 sigma^2 by more than 3x, so a device computing the wrong function fails those
    cases."""
    from slime_amd import make_state
    from slime_amd.synthetic import CAConfig
    from tests.conftest import growth_variant_params
    scfg = CAConfig("variant", B=2, G=16, H=H, D=D, dtype="fp32", steps=1, w_std=0.05, pods=2,
                    growth_per_cell=per_cell)
    X = make_state(scfg, seed=2)
    p = growth_variant_params(scfg, oracle, X)
    Ys = {fn: oracle.step(OracleConfig(B=2, G=16, H=H, D=D, pods=2, growth_per_cell=per_cell,
                                       growth_fn=fn), X, p, 1)[0] for fn in (0, 1, 2)}
    for a, b in ((0, 1), (0, 2), (1, 2)):
        moved = norm_err(Ys[a], Ys[b])
        print(f"  growth {a} vs {b}: {moved:.3f}")
        assert moved > 5 * 2e-2, (a, b)
    q = dict(p, sigma=(p["sigma"] / np.sqrt(2.0)).astype(np.float32))  # exp(-(U-mu)^2 / sigma^2)
    wrong = oracle.step(OracleConfig(B=2, G=16, H=H, D=D, pods=2, growth_per_cell=per_cell,
                                     growth_fn=1), X, q, 1)[0]
    assert norm_err(wrong, Ys[1]) > 3 * 2e-2


def test_growth_per_cell_parameters(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=2, growth_per_cell=True)
    r = _rng(11)
    mu = r.uniform(0.1, 0.3, (1, 8, 8, H)).astype(np.float32)
    sigma = r.uniform(0.01, 0.05, (1, 8, 8, H)).astype(np.float32)
    U = np.repeat(mu[0][None, :, :, :, None], cfg.D, axis=-1).reshape(1, 8, 8, cfg.C)
    np.testing.assert_allclose(oracle.growth(cfg, U, mu, sigma), 1.0, atol=1e-5)


# ---- S4/S5 activation and propagation ------------------------------------------------------

def test_attention_uniform_when_perception_is_zero(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=4)
    I = _state(cfg)
    A = oracle.attention(cfg, np.zeros_like(I), I)
    np.testing.assert_allclose(A, 1.0 / 9.0, rtol=1e-6)
    V = _state(cfg, seed=9)
    Vt = oracle.propagate(cfg, A, V)
    box = np.stack([ndimage.uniform_filter(V[0, :, :, c].astype(np.float64), 3, mode="wrap")
                    for c in range(cfg.C)], axis=-1)
    np.testing.assert_allclose(Vt[0], box, rtol=1e-5, atol=1e-6)


def test_attention_one_hot_and_normalised(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=4)
    P = np.zeros((1, 8, 8, cfg.C), np.float32)
    I = np.zeros_like(P)
    P[0, 3, 5, :] = 1.0
    I[0, 2, 6, :] = 100.0  # neighbour (dy=-1, dx=+1) of cell (3, 5): tap k = 2
    A = oracle.attention(cfg, P, I)
    assert A[0, 3, 5, 0, 2] > 0.999999
    np.testing.assert_allclose(A.sum(-1), 1.0, rtol=1e-6)
    r = _rng(5)
    A = oracle.attention(cfg, r.normal(size=P.shape).astype(np.float32),
                         r.normal(size=P.shape).astype(np.float32))
    np.testing.assert_allclose(A.sum(-1), 1.0, rtol=1e-6)
    # a tap-k one-hot attention propagates exactly that neighbour's value
    V = _state(cfg, seed=12)
    A1 = np.zeros((1, 8, 8, H, 9), np.float32)
    A1[..., 6] = 1.0  # (dy=+1, dx=-1)
    np.testing.assert_array_equal(oracle.propagate(cfg, A1, V), np.roll(V, (-1, 1), axis=(1, 2)))


def test_attention_matches_vectorised_numpy(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=4)
    r = _rng(21)
    P = r.normal(size=(1, 8, 8, cfg.C)).astype(np.float32)
    I = r.normal(size=(1, 8, 8, cfg.C)).astype(np.float64)
    A = oracle.attention(cfg, P, I)
    Ph = P.astype(np.float64).reshape(1, 8, 8, H, cfg.D)
    s = np.empty((1, 8, 8, H, 9))
    for k in range(9):
        dy, dx = k // 3 - 1, k % 3 - 1
        In = np.roll(I, (-dy, -dx), axis=(1, 2)).reshape(1, 8, 8, H, cfg.D)
        s[..., k] = (Ph * In).sum(-1) / math.sqrt(cfg.D)
    e = np.exp(s - s.max(-1, keepdims=True))
    np.testing.assert_allclose(A, e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("G", [16, 32])
def test_peaked_attention_case_sees_planted_s4_s5_mistakes(oracle, G):
    """The inputs of the GPU peaked-attention parity cases (bf16 D=64, 2 pods,
    tests.conftest.peaked_params), run through the oracle with one stage mistake
    planted at a time. Each moves Y by more than 5x the bf16 bar of 2e-2, while the
    rounding the device applies (bf16 P, I, V, attention weights and Y) moves it
    by less than a quarter of the bar: a device with any of these mistakes fails
    the GPU cases, and a correct one passes them."""
    from slime_amd import make_state, round_bf16
    from slime_amd.synthetic import CAConfig
    from tests.conftest import peaked_params
    bar = 2e-2
    scfg = CAConfig("peak", B=2, G=G, H=H, D=64, dtype="bf16", steps=1, w_std=0.05, pods=2)
    p = peaked_params(scfg)
    p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
    X = round_bf16(make_state(scfg, seed=2))
    cfg = OracleConfig(B=2, G=G, H=H, D=64, pods=2)
    P, I, V = map(round_bf16, oracle.project(cfg, X, p["WP"], p["WI"], p["WV"]))
    g = oracle.growth(cfg, oracle.potential(cfg, X, p["K"]), p["mu"], p["sigma"])

    def y_of(A):
        Y = oracle.mix(cfg, X, g, oracle.propagate(cfg, A, V), p["M"])
        return oracle.conserve(cfg, X, Y)[0]

    A = oracle.attention(cfg, P, I)
    assert A.max(axis=-1).mean() > 0.5
    Y = y_of(A)
    centre = np.zeros_like(A)
    centre[..., 4] = 1.0
    planted = {
        "uniform attention": np.full_like(A, 1.0 / 9.0),
        "neighbours mirrored (k -> 8-k)": A[..., ::-1].copy(),
        "query and key swapped": oracle.attention(cfg, I, P),
        "scores from P.P": oracle.attention(cfg, P, P),
        "scores without 1/sqrt(d)": oracle.attention(cfg, np.sqrt(64.0) * P, I),
        "value of the centre cell only": centre,
        "attention map transposed (y <-> x)": A.transpose(0, 2, 1, 3, 4).copy(),
    }
    for name, Aw in planted.items():
        moved = norm_err(y_of(Aw), Y)
        print(f"  G={G} {name}: Y moves by {moved:.3f}")
        assert moved > 5 * bar, name
    rounding = norm_err(round_bf16(y_of(round_bf16(A))), Y)
    print(f"  G={G} device rounding: {rounding:.2e}")
    assert rounding < bar / 4
    # the whole step from unrounded projections stays inside the bar as well
    assert norm_err(oracle.step(cfg, X, p, 1)[0], Y) < bar / 4


# ---- S6 update and mixing ----------------------------------------------------------------

def test_mix_closed_forms(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=4, dt=0.0)
    X, g, Vt = _state(cfg), _state(cfg, 1), _state(cfg, 2)
    eye = np.eye(H, dtype=np.float32)[None]
    np.testing.assert_allclose(oracle.mix(cfg, X, g, Vt, eye), X, rtol=1e-7)
    M = _params(cfg)["M"]
    Y = oracle.mix(cfg, X, g, Vt, M)
    ref = np.einsum("oh,byxhc->byxoc", M[0].astype(np.float64),
                    X.astype(np.float64).reshape(1, 8, 8, H, cfg.D)).reshape(X.shape)
    np.testing.assert_allclose(Y, ref, rtol=1e-6, atol=1e-7)
    cfg = OracleConfig(B=1, G=8, H=H, D=4, dt=0.1)
    Y = oracle.mix(cfg, X, g, Vt, eye)
    np.testing.assert_allclose(Y, X + 0.1 * g.astype(np.float64) * Vt, rtol=1e-6, atol=1e-7)
    Y2 = oracle.mix(cfg, X, g, Vt, 2 * M)
    np.testing.assert_allclose(Y2, 2 * oracle.mix(cfg, X, g, Vt, M), rtol=1e-6, atol=1e-7)


# ---- S7 conservation ------------------------------------------------------------------------

def test_conserve_per_cell_sums_and_guard(oracle):
    """conservation 1, the shipped per-(cell, head) renormalisation
    (slime/core/pseudopod.cu:160-165,196-203): every cell's head sum of Y equals
    that of X; a cell whose head sum of Y is within the 1e-6 guard keeps its values;
    the per-(b, head) totals are then conserved as well."""
    cfg = OracleConfig(B=2, G=8, H=H, D=4, conservation=1)
    r = _rng(17)
    X = r.random((2, 8, 8, cfg.C), dtype=np.float32)
    Y = (X * r.uniform(0.5, 1.5, X.shape)).astype(np.float32)
    Y[1, 3, 4, 2 * 4:3 * 4] = np.array([1e-7, -1e-7, 2e-7, 0.0], np.float32)  # guard cell
    Yc, mi, mo = oracle.conserve(cfg, X, Y)
    sx = X.astype(np.float64).reshape(2, 8, 8, H, 4).sum(-1)
    sy = Yc.astype(np.float64).reshape(2, 8, 8, H, 4).sum(-1)
    other = np.ones(sx.shape, bool)
    other[1, :, :, 2] = False
    np.testing.assert_allclose(sy[other], sx[other], rtol=1e-6)
    # batch 1, head 2 holds the guard cell: its mass is missing from the head total
    # after the per-cell pass, and the global pass puts it back by one factor over
    # the head, so every other cell of that head keeps one common ratio
    ratio = sy[1, :, :, 2] / sx[1, :, :, 2]
    ratio = np.delete(ratio.reshape(-1), 3 * 8 + 4)
    np.testing.assert_allclose(ratio, ratio[0], rtol=1e-6)
    assert ratio[0] > 1.0 + 1e-4
    np.testing.assert_allclose(mo, mi, rtol=1e-12)
    # a state that already matches X cell by cell is left as it is
    Yi, _, _ = oracle.conserve(cfg, X, X)
    np.testing.assert_allclose(Yi, X, rtol=1e-6)
    # against the global-only mode the cells differ, the totals agree
    Yg, _, mo0 = oracle.conserve(OracleConfig(B=2, G=8, H=H, D=4), X, Y)
    assert norm_err(Yg, Yc) > 1e-2
    np.testing.assert_allclose(mo0, mo, rtol=1e-12)


def test_conserve_sums_and_guard(oracle):
    cfg = OracleConfig(B=2, G=8, H=H, D=4)
    X, Y = _state(cfg), _state(cfg, 8) * 3.0
    Yc, mi, mo = oracle.conserve(cfg, X, Y)
    xs = X.astype(np.float64).reshape(2, -1, H, cfg.D).sum(axis=(1, 3))
    np.testing.assert_allclose(mi, xs, rtol=1e-12)
    np.testing.assert_allclose(mo, xs, rtol=1e-6)
    ys = Yc.astype(np.float64).reshape(2, -1, H, cfg.D).sum(axis=(1, 3))
    np.testing.assert_allclose(ys, xs, rtol=1e-6)
    # zero-sum head: the |sum| > 1e-6 guard leaves it unscaled
    Y = Y.copy()
    Y[0, ..., 0:cfg.D] = 0.0
    Yc, _, _ = oracle.conserve(cfg, X, Y)
    assert np.all(Yc[0, ..., 0:cfg.D] == 0.0)


# ---- full step ------------------------------------------------------------------------------

def _numpy_step(cfg, X, p):
    """Vectorised numpy restatement of one S1-S7 step (independent of the C++ loops)."""
    G, C, D = cfg.G, cfg.C, cfg.D
    x = X.astype(np.float64)
    out = np.empty_like(x)
    for b in range(cfg.B):
        q = b // (cfg.B // cfg.pods)
        xb = x[b]
        P = np.maximum(xb @ p["WP"][q].astype(np.float64), 0)
        I = _gelu(xb @ p["WI"][q].astype(np.float64))
        V = xb @ p["WV"][q].astype(np.float64)
        xh = xb.reshape(G, G, H, D)
        U = np.zeros_like(xh)
        s = np.empty((G, G, H, 9))
        Vt = np.zeros_like(xh)
        for k in range(9):
            dy, dx = k // 3 - 1, k % 3 - 1
            sh = lambda a: np.roll(a, (-dy, -dx), axis=(0, 1))  # noqa: E731
            U += p["K"][q][None, None, :, k, None] * sh(xh)
            s[..., k] = (P.reshape(G, G, H, D) * sh(I).reshape(G, G, H, D)).sum(-1) / math.sqrt(D)
        a = np.exp(s - s.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        for k in range(9):
            dy, dx = k // 3 - 1, k % 3 - 1
            Vt += a[..., k, None] * np.roll(V.reshape(G, G, H, D), (-dy, -dx), axis=(0, 1))
        if cfg.growth_per_cell:
            mu, sg = p["mu"][q][..., None], p["sigma"][q][..., None]
        else:
            mu, sg = p["mu"][q][None, None, :, None], p["sigma"][q][None, None, :, None]
        if cfg.growth_fn == 1:
            g = np.exp(-(U - mu) ** 2 / (2 * sg.astype(np.float64) ** 2))
        elif cfg.growth_fn == 2:
            g = U * np.exp(-U * U)
        else:
            g = 2 * np.exp(-((U - mu) / (sg + 1e-7)) ** 2) - 1
        Z = xh + cfg.dt * g * Vt
        Y = np.einsum("oh,yxhc->yxoc", p["M"][q].astype(np.float64), Z)
        if cfg.conservation == 1:
            cx, cy = xh.sum(axis=3, keepdims=True), Y.sum(axis=3, keepdims=True)
            Y = Y * np.where(np.abs(cy) > 1e-6, cx / np.where(cy == 0, 1, cy), 1.0)
        sx = xh.sum(axis=(0, 1, 3))
        sy = Y.sum(axis=(0, 1, 3))
        scale = np.where(np.abs(sy) > 1e-6, sx / sy, 1.0)
        out[b] = (Y * scale[None, None, :, None]).reshape(G, G, C)
    return out


@pytest.mark.parametrize("per_cell,pods,fn,cons", [(False, 1, 0, 0), (True, 2, 0, 0), (False, 2, 1, 0),
                                                   (True, 1, 2, 1), (False, 1, 0, 1)])
def test_step_matches_numpy_restatement(oracle, per_cell, pods, fn, cons):
    cfg = OracleConfig(B=2, G=8, H=H, D=8, pods=pods, growth_per_cell=per_cell, growth_fn=fn,
                       conservation=cons)
    p, X = _params(cfg, w_std=0.1), _state(cfg)
    Y, mi, mo = oracle.step(cfg, X, p, 1)
    ref = _numpy_step(cfg, X, p)
    assert norm_err(Y, ref) < 1e-6
    np.testing.assert_allclose(mo, mi, rtol=1e-6)


def test_step_zero_dt_identity_mixing_is_identity(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=8, dt=0.0)
    p, X = _params(cfg), _state(cfg)
    p["M"] = np.eye(H, dtype=np.float32)[None]
    Y, _, _ = oracle.step(cfg, X, p, 3)
    np.testing.assert_allclose(Y, X, rtol=1e-6)


# ---- fitness ---------------------------------------------------------------------------------

def test_jacobi_matches_lapack_golden(oracle):
    """Eigenvalues fixed by construction (A = Q diag(lam) Q^T) and LAPACK eigvalsh."""
    from tests.golden.make_golden import load_jacobi
    for A, lam, eig_lapack in load_jacobi():
        eig, sweeps = oracle.jacobi_eigs(A)
        assert sweeps <= 30
        # |a_pq| <= 1e-6 is never rotated and the sweeps stop at sum |a_pq| <
        # 1e-6 n: each diagonal entry is then within 1e-6 n of an eigenvalue.
        bound = 1e-6 * A.shape[0]
        np.testing.assert_allclose(eig, lam, rtol=0, atol=bound)
        np.testing.assert_allclose(eig, eig_lapack, rtol=0, atol=bound)


def test_jacobi_closed_forms(oracle):
    eig, sweeps = oracle.jacobi_eigs(np.eye(64))
    np.testing.assert_allclose(eig, 1.0)
    assert sweeps == 1
    d = np.linspace(3, 0.5, 16)
    eig, _ = oracle.jacobi_eigs(np.diag(d[::-1]))
    np.testing.assert_allclose(eig, d)
    v = _rng(2).normal(size=32)
    eig, _ = oracle.jacobi_eigs(np.outer(v, v))
    np.testing.assert_allclose(eig[0], v @ v, rtol=1e-9)
    assert np.max(np.abs(eig[1:])) < 1e-6 * (v @ v)
    # a 2x2 rotation problem with a known answer: eigenvalues 3 and 1
    eig, _ = oracle.jacobi_eigs(np.array([[2.0, 1.0], [1.0, 2.0]]))
    np.testing.assert_allclose(eig, [3.0, 1.0], rtol=1e-12)


def test_effective_rank_closed_forms(oracle):
    n = 64
    er = oracle.effective_rank(np.ones(n))
    p = 1.0 / (n + 1e-7)
    np.testing.assert_allclose(er, math.exp(-n * p * math.log(p + 1e-7)), rtol=1e-12)
    assert abs(er - n) < 1e-3
    sv = np.zeros(n)
    sv[0] = 2.5
    assert abs(oracle.effective_rank(sv) - 1.0) < 1e-6


def test_gram_and_coherence(oracle):
    cfg = OracleConfig(B=2, G=8, H=H, D=4)
    hist = _rng(3).random((4, 2, 8, 8, cfg.C), dtype=np.float32)
    A = oracle.gram(cfg, hist[-1])
    xh = hist[-1].astype(np.float64).reshape(2, 64, H, cfg.D)
    ref = np.einsum("bnhi,bnhj->bhij", xh, xh) / 64
    np.testing.assert_allclose(A, ref, rtol=1e-12)
    coh = oracle.coherence(cfg, hist)
    for b in range(2):
        for h in range(H):
            rho = [np.corrcoef(hist[t - 1, b, ..., h * cfg.D:(h + 1) * cfg.D].ravel(),
                               hist[t, b, ..., h * cfg.D:(h + 1) * cfg.D].ravel())[0, 1]
                   for t in range(1, 4)]
            np.testing.assert_allclose(coh[b, h], (np.mean(rho) + 1) / 2, rtol=1e-10)
    same = np.repeat(hist[:1], 3, axis=0)
    np.testing.assert_allclose(oracle.coherence(cfg, same), 1.0, rtol=1e-12)
    flip = np.stack([hist[0], -hist[0]])
    np.testing.assert_allclose(oracle.coherence(cfg, flip), 0.0, atol=1e-12)


def test_fitness_composes_rank_and_coherence(oracle):
    cfg = OracleConfig(B=1, G=8, H=H, D=8)
    hist = _rng(4).random((3, 1, 8, 8, cfg.C), dtype=np.float32)
    er, coh, fit = oracle.fitness(cfg, hist)
    A = oracle.gram(cfg, hist[-1])
    for h in range(H):
        ev = np.linalg.eigvalsh(A[0, h])[::-1]
        sv = np.sort(np.sqrt(np.abs(ev)))[::-1]
        p = sv / (sv.sum() + 1e-7)
        np.testing.assert_allclose(er[0, h], math.exp(-(p * np.log(p + 1e-7)).sum()), rtol=1e-8)
    np.testing.assert_allclose(fit, er * coh, rtol=1e-12)


# ---- organism adapters --------------------------------------------------------------------------

def test_field_adapters(oracle):
    conc = _rng(6).random((8, 8), dtype=np.float32)
    X = oracle.init_from_field(conc, 64)
    c = np.arange(64, dtype=np.float32) * np.float32(0.1)
    np.testing.assert_allclose(X, conc[..., None] * np.sin(c.astype(np.float64)), rtol=1e-6,
                               atol=1e-7)
    np.testing.assert_allclose(oracle.field_from_state(X), X.astype(np.float64).mean(-1),
                               rtol=1e-6, atol=1e-7)


# ---- golden regression (fixtures written by tests/golden/make_golden.py) --------------------------

def test_oracle_reproduces_committed_golden(oracle):
    from tests.golden.make_golden import check_golden
    check_golden(oracle)


# ---- backward (config c5's gradient): pinned by central finite differences -------------------
# The analytic gradient of L = mean((step(X) - T)^2) is compared with
# (L(x + e) - L(x - e)) / 2e of the oracle's own fp64 forward. Perturbations are
# powers of two, exact in fp32 at these magnitudes, so the differences carry only
# the O(e^2) truncation error. A dropped term, sign or transposed operand in any
# stage's chain rule moves some sampled entry by far more than the tolerance.

def _fd_entries(oracle, cfg, X, p, T, key, idxs, eps):
    out = []
    for idx in idxs:
        hi = {k: v.copy() for k, v in p.items()}
        lo = {k: v.copy() for k, v in p.items()}
        xh, xl = X.copy(), X.copy()
        if key == "X":
            xh[idx] += eps
            xl[idx] -= eps
        else:
            hi[key][idx] += eps
            lo[key][idx] -= eps
        out.append((oracle.step_loss(cfg, xh, hi, T) - oracle.step_loss(cfg, xl, lo, T)) / (2 * eps))
    return np.array(out)


@pytest.mark.parametrize("per_cell,pods,guard", [(False, 2, False), (True, 1, False), (False, 1, True)])
def test_backward_matches_finite_differences(oracle, per_cell, pods, guard):
    cfg = OracleConfig(B=2, G=6, H=H, D=4, pods=pods, growth_per_cell=per_cell)
    p, X = _params(cfg, w_std=0.2), _state(cfg)
    if guard:
        p["M"][0, 3, :] = 0.0  # head 3's output is identically zero: the S7 guard path
    T = _rng(9).random(X.shape, dtype=np.float32)
    loss, gr = oracle.step_backward(cfg, X, p, T)
    assert abs(loss - oracle.step_loss(cfg, X, p, T)) <= 1e-15 * max(loss, 1.0)
    r = _rng(11)
    checks = {
        "X": (2.0 ** -10, [tuple(r.integers(0, s) for s in X.shape) for _ in range(16)]),
        "WP": (2.0 ** -10, [tuple(r.integers(0, s) for s in p["WP"].shape) for _ in range(6)]),
        "WI": (2.0 ** -10, [tuple(r.integers(0, s) for s in p["WI"].shape) for _ in range(6)]),
        "WV": (2.0 ** -10, [tuple(r.integers(0, s) for s in p["WV"].shape) for _ in range(6)]),
        "K": (2.0 ** -12, [tuple(r.integers(0, s) for s in p["K"].shape) for _ in range(6)]),
        "mu": (2.0 ** -14, [tuple(r.integers(0, s) for s in p["mu"].shape) for _ in range(4)]),
        "sigma": (2.0 ** -16, [tuple(r.integers(0, s) for s in p["sigma"].shape) for _ in range(4)]),
        "M": (2.0 ** -12, [tuple(r.integers(0, s) for s in p["M"].shape) for _ in range(6)]),
    }
    if guard:
        # Perturbing the zeroed row lifts |sum Y_3| above the guard, where the
        # conserved output no longer depends on that row's scale: the loss is
        # discontinuous there, so only entries off that row are differenced.
        checks["M"] = (2.0 ** -12, [(0, o, h) for o, h in ((0, 3), (1, 5), (4, 4), (7, 2))])
    for key, (eps, idxs) in checks.items():
        fd = _fd_entries(oracle, cfg, X, p, T, key, idxs, eps)
        an = np.array([gr[key][i] for i in idxs], dtype=np.float64)
        scale = np.max(np.abs(gr[key]))
        assert scale > 0, key
        np.testing.assert_allclose(an, fd, rtol=2e-3, atol=2e-4 * scale, err_msg=key)


def test_backward_dt_zero_is_conserved_linear_map(oracle):
    # dt = 0 and M = I: Y = X exactly with scale 1, so L = mean((X - T)^2). The
    # conservation terms cancel (gY = gY' - Q/B through Y, + Q/B through the input
    # mass), leaving dL/dX = 2 (X - T) / N.
    cfg = OracleConfig(B=1, G=5, H=H, D=2, dt=0.0)
    p, X = _params(cfg), _state(cfg)
    p["M"] = np.eye(H, dtype=np.float32)[None]
    T = _rng(5).random(X.shape, dtype=np.float32)
    loss, gr = oracle.step_backward(cfg, X, p, T)
    N = X.size
    Xd, Td = X.astype(np.float64), T.astype(np.float64)
    assert abs(loss - np.mean((Xd - Td) ** 2)) <= 1e-12
    np.testing.assert_allclose(gr["X"], 2 * (Xd - Td) / N, rtol=1e-5, atol=1e-9)
    # with dt = 0 nothing depends on the projections, the potential or the growth
    for k in ("WP", "WI", "WV", "K", "mu", "sigma"):
        assert np.all(gr[k] == 0), k


def test_backward_rejects_chained_projections(oracle):
    cfg = OracleConfig(B=1, G=4, H=H, D=2, pvi_chain=True)
    p, X = _params(cfg), _state(cfg)
    with pytest.raises(ValueError):
        oracle.step_backward(cfg, X, p, X)
