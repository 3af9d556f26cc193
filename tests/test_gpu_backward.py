"""GPU backward (slime_ca_backward, configuration c5): the gradient of
L = mean((step(X) - T)^2) against the CPU oracle's fp64 gradient (itself pinned by
finite differences in tests/test_oracle.py), and at the c5 shape against central
finite differences of an independent fp64 numpy forward on 64 sampled cells.

Tolerances (normalised max error, max|gpu - ref| / max|ref| per tensor), as the
forward's: fp32 state 1e-5, bf16 state 2e-2.
"""
import numpy as np
import pytest

from slime_amd import Pseudopod, make_params, make_state, round_bf16
from slime_amd.synthetic import CAConfig
from tests.conftest import norm_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = {"fp32": 1e-5, "bf16": 2e-2}
NAMES = ("WP", "WI", "WV", "K", "mu", "sigma", "M")


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _cfg(B, G, D, dtype, **kw):
    return CAConfig("bw", B=B, G=G, H=8, D=D, dtype=dtype, steps=1, w_std=0.05, **kw)


def _inputs(cfg, seed=1, peaked=False):
    if peaked:  # peaked attention: the S4 backward carries a large share of the gradients
        from tests.conftest import peaked_params
        p = peaked_params(cfg, seed=seed)
    else:
        p = make_params(cfg, seed=seed)
    X = make_state(cfg, seed=seed + 1)
    T = np.random.default_rng(seed + 2).random(X.shape, dtype=np.float32)
    if cfg.dtype == "bf16":
        p = {k: (round_bf16(v) if k in ("WP", "WI", "WV") else v) for k, v in p.items()}
        X, T = round_bf16(X), round_bf16(T)
    return p, X, T


def _dev(a, dtype):
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
    return t.to(torch.bfloat16 if dtype == "bf16" else torch.float32).contiguous()


@pytest.mark.parametrize("dtype,D,pods,per_cell,B,G,peaked", [
    # the peaked-attention weights of tests.conftest.peaked_params
    ("bf16", 64, 2, False, 2, 16, True),
    ("fp32", 64, 1, True, 2, 16, True),
    ("fp32", 16, 2, False, 2, 16, False),
    ("fp32", 32, 1, True, 2, 16, False),
    ("bf16", 64, 1, False, 2, 16, False),
    ("bf16", 64, 2, True, 2, 16, False),
    # C = 256: one wave per cell in the cell pass, one 256-column tile per operand in dW
    ("bf16", 32, 2, False, 2, 16, False),
    # C = 128: the 128 x 128 weight-gradient tiles
    ("bf16", 16, 1, True, 2, 16, False),
    # the smallest grid: 64 cells per pod, fewer than 8 whole cell-pass iterations
    ("fp32", 8, 1, False, 1, 8, False),
    ("fp32", 8, 3, True, 3, 8, False),
    # bf16, D = 64 on the smallest grid: the LDS-ring cell pass with rows of 8 cells (4
    # iterations, every column slot reused), per-cell growth, two pods of one entry each
    ("bf16", 64, 2, True, 2, 8, True),
])
def test_backward_matches_oracle(oracle, dtype, D, pods, per_cell, B, G, peaked):
    cfg = _cfg(B=B, G=G, D=D, dtype=dtype, pods=pods, growth_per_cell=per_cell)
    print(f"[case] backward {dtype} D={D} pods={pods} per_cell={per_cell} peaked={peaked}", flush=True)
    p, X, T = _inputs(cfg, peaked=peaked)
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, per_cell, pods) as e:
        e.set_params(p)
        loss, gx, grads = e.backward(_dev(X, dtype), _dev(T, dtype))
        torch.cuda.synchronize()
        gx = gx.cpu().numpy()
        grads = {k: v.cpu().numpy() for k, v in grads.items()}
    from oracle import OracleConfig
    ocfg = OracleConfig(B=cfg.B, G=cfg.G, H=8, D=D, pods=pods, growth_per_cell=per_cell)
    rloss, ref = oracle.step_backward(ocfg, X, p, T)
    tol = TOL[dtype]
    print(f"  loss {loss:.8e} ref {rloss:.8e}")
    assert abs(loss - rloss) <= tol * rloss
    errs = {"X": norm_err(gx, ref["X"])}
    for k in NAMES:
        errs[k] = norm_err(grads[k], ref[k])
    print("  normalised errors " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for k, v in errs.items():
        assert v <= tol, (k, v)


def test_backward_rejects_chained_projections():
    from slime_amd._lib import SlimeError
    cfg = _cfg(B=1, G=16, D=16, dtype="fp32")
    p, X, T = _inputs(cfg)
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, "fp32", cfg.dt, False, 1, True) as e:
        e.set_params(p)
        with pytest.raises(SlimeError):
            e.backward(_dev(X, "fp32"), _dev(T, "fp32"))


# ---- c5: 512 x 512 grid, batch 4, bf16 -------------------------------------------------------

def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


class _LocalStep:
    """fp64 numpy restatement of one step on batch entry 0, keeping what a local
    finite difference needs: the unperturbed output Y (before conservation), the
    per-head sums A_o = sum X_o, B_o = sum Y_o, sum Y_o^2 and sum T_o Y_o."""

    def __init__(self, X0, p, T0, D, dt):
        self.G, self.C, self.D, self.dt = X0.shape[0], X0.shape[-1], D, dt
        self.p = {k: np.asarray(v[0], np.float64) for k, v in p.items()}
        self.X = X0.astype(np.float64)
        self.T = T0.astype(np.float64)
        G, C = self.G, self.C
        Xf = self.X.reshape(-1, C)
        P = np.maximum(Xf @ self.p["WP"], 0).reshape(G, G, C)
        I = _gelu(Xf @ self.p["WI"]).reshape(G, G, C)
        V = (Xf @ self.p["WV"]).reshape(G, G, C)
        self.Y = self._stencil(self.X, P, I, V)
        Yh, Th = self._heads(self.Y), self._heads(self.T)
        self.A = self._heads(self.X).sum(axis=(0, 1, 3))
        self.Bs = Yh.sum(axis=(0, 1, 3))
        self.Syy = (Yh * Yh).sum(axis=(0, 1, 3))
        self.Sty = (Th * Yh).sum(axis=(0, 1, 3))

    def _heads(self, a):
        return a.reshape(a.shape[0], a.shape[1], 8, self.D)

    def _stencil(self, X, P, I, V):
        # S2-S6 on a (possibly cropped) window; returns Y on the window's interior
        # rows/cols [1, n-1) when cropped, or on the whole torus when not.
        D, p = self.D, self.p
        Xh, Ph, Ih, Vh = (self._heads(a) for a in (X, P, I, V))
        sh = lambda a, dy, dx: np.roll(a, (-dy, -dx), axis=(0, 1))
        U = sum(p["K"][None, None, :, k, None] * sh(Xh, k // 3 - 1, k % 3 - 1) for k in range(9))
        g = 2 * np.exp(-((U - p["mu"][None, None, :, None]) / (p["sigma"][None, None, :, None] + 1e-7)) ** 2) - 1
        s = np.stack([(Ph * sh(Ih, k // 3 - 1, k % 3 - 1)).sum(-1) / np.sqrt(D) for k in range(9)], -1)
        a = np.exp(s - s.max(-1, keepdims=True))
        a /= a.sum(-1, keepdims=True)
        Vt = sum(a[..., k, None] * sh(Vh, k // 3 - 1, k % 3 - 1) for k in range(9))
        Z = Xh + self.dt * g * Vt
        Y = np.einsum("oh,yxhc->yxoc", p["M"], Z)
        return Y.reshape(X.shape)

    def loss_delta(self, y, x, ch, eps):
        """L(X + eps e_{y,x,ch}) * N - L(X) * N on batch entry 0, from a 7 x 7 window."""
        G, C = self.G, self.C
        ys, xs = (np.arange(-3, 4) + y) % G, (np.arange(-3, 4) + x) % G
        Xw = self.X[np.ix_(ys, xs)].copy()
        Xw[3, 3, ch] += eps
        Xf = Xw.reshape(-1, C)
        P = np.maximum(Xf @ self.p["WP"], 0).reshape(7, 7, C)
        I = _gelu(Xf @ self.p["WI"]).reshape(7, 7, C)
        V = (Xf @ self.p["WV"]).reshape(7, 7, C)
        Yw = self._stencil(Xw, P, I, V)[2:5, 2:5]  # the 3 x 3 cells that change
        iy, ix = np.ix_(ys[2:5], xs[2:5])
        Y0, Tw = self.Y[iy, ix], self.T[iy, ix]
        h = ch // self.D
        A1 = self.A.copy()
        A1[h] += eps
        dB = self._heads(Yw - Y0).sum(axis=(0, 1, 3))
        r0, r1 = self.A / self.Bs, A1 / (self.Bs + dB)
        Y0h, Y1h, Th = self._heads(Y0), self._heads(Yw), self._heads(Tw)
        # far field: every cell outside the 3 x 3 window keeps Y, only r changes
        syy = self.Syy - (Y0h * Y0h).sum(axis=(0, 1, 3))
        sty = self.Sty - (Th * Y0h).sum(axis=(0, 1, 3))
        far = ((r1 ** 2 - r0 ** 2) * syy - 2 * (r1 - r0) * sty).sum()
        near = (((r1[None, None, :, None] * Y1h - Th) ** 2).sum()
                - ((r0[None, None, :, None] * Y0h - Th) ** 2).sum())
        return far + near


@pytest.mark.parametrize("G", [128, 136])
def test_weight_gradients_over_several_row_chunks(G):
    """bf16, D = 64, a batch of 2 on a G^2 grid: 2 G^2 rows per pod, so the weight
    gradients run as several 16,384-row chunks on the 256 x 256 tiles, added in chunk
    order (G = 136 leaves a partial last chunk). The loss is a mean over the batch and
    the mass rescale is per (batch entry, head), so every parameter gradient of the
    batch is half the sum of the single-entry ones (one or two chunks each), and the
    batch's dL/dX at entry i is half that entry's own."""
    cfg = _cfg(B=2, G=G, D=64, dtype="bf16")
    print(f"[case] backward over row chunks bf16 D64 B2 G{G}", flush=True)
    p, X, T = _inputs(cfg)

    def grads(Xb, Tb):
        with Pseudopod(Xb.shape[0], G, 8, 64, "bf16", cfg.dt, False, 1) as e:
            e.set_params(p)
            loss, gx, g = e.backward(_dev(Xb, "bf16"), _dev(Tb, "bf16"))
            torch.cuda.synchronize()
            return loss, gx.cpu().numpy(), {k: v.cpu().numpy().astype(np.float64) for k, v in g.items()}

    loss2, gx2, g2 = grads(X, T)
    parts = [grads(X[i:i + 1], T[i:i + 1]) for i in range(2)]
    assert abs(loss2 - 0.5 * (parts[0][0] + parts[1][0])) <= 1e-9 * loss2
    for k in NAMES:
        err = norm_err(g2[k], 0.5 * (parts[0][2][k] + parts[1][2][k]))
        print(f"  {k}: normalised error {err:.2e}")
        assert err <= 1e-5, (k, err)
    for i in range(2):
        err = norm_err(gx2[i], 0.5 * parts[i][1][0])
        print(f"  dX entry {i}: normalised error {err:.2e}")
        assert err <= 1e-5


def test_c5_gradient_matches_finite_differences_on_64_cells():
    from slime_amd import CONFIGS
    cfg = CONFIGS["c5"]
    print("[case] backward c5 B4 G512 bf16, 64 sampled cells", flush=True)
    p, X, T = _inputs(cfg)
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, False, 1) as e:
        e.set_params(p)
        loss, gx, _ = e.backward(_dev(X, "bf16"), _dev(T, "bf16"), params=False)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(gx).all())
        g0 = gx[0].cpu().numpy()
    ref = _LocalStep(X[0], p, T[0], cfg.D, cfg.dt)
    N = float(X.size)
    rng = np.random.default_rng(7)
    picks = [(int(rng.integers(cfg.G)), int(rng.integers(cfg.G)), int(rng.integers(cfg.C)))
             for _ in range(64)]
    eps = 1e-3
    fd = np.array([(ref.loss_delta(y, x, c, eps) - ref.loss_delta(y, x, c, -eps)) / (2 * eps * N)
                   for y, x, c in picks])
    got = np.array([g0[y, x, c] for y, x, c in picks])
    err = float(np.max(np.abs(got - fd)) / np.max(np.abs(fd)))
    print(f"  loss {loss:.6e}; 64 sampled cells: normalised error {err:.3e}")
    assert np.isfinite(loss) and loss > 0
    assert err <= TOL["bf16"]
