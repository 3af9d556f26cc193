"""The reference's per-head weight tensors embedded as dense C x C matrices
(slime_amd.refweights) reproduce the per-head products of multi_head_ca_kernel
(slime/core/pseudopod.cu:79-119), written here as that kernel's own index loops,
through the oracle's chained projection (CPU only)."""
import numpy as np
import pytest

from oracle import OracleConfig
from slime_amd.refweights import from_reference_weights

H, D, CHANNELS, HIDDEN = 8, 64, 512, 256


def _gelu_tanh(x):
    import torch
    return torch.nn.functional.gelu(torch.from_numpy(np.asarray(x, np.float64)),
                                    approximate="tanh").numpy()


def _reference_weights(seed=11):
    r = np.random.default_rng(seed)
    return (r.normal(0, 0.05, (H, CHANNELS, HIDDEN)).astype(np.float32),
            r.normal(0, 0.05, (H, CHANNELS, HIDDEN)).astype(np.float32),
            r.normal(0, 0.05, (H, HIDDEN, CHANNELS)).astype(np.float32),
            (np.eye(H) + r.normal(0, 0.01, (H, H))).astype(np.float32),
            r.normal(0, 0.1, (H, 3, 3)).astype(np.float32))


def _reference_head(x_h, h, wp, wi, wv):
    """One head of one cell as the reference's loops index it (flat weight
    arrays, weight_idx exactly as at pseudopod.cu:86-88, 102-103, 115-117),
    the neighbourhood replaced by the cell itself."""
    wp, wi, wv = (np.asarray(a, np.float64).ravel() for a in (wp, wi, wv))
    perception = np.zeros(D)
    for i in range(D):
        for c in range(D):
            perception[i] += x_h[c] * wp[h * CHANNELS * HIDDEN + c * HIDDEN + i]
        perception[i] = max(0.0, perception[i])
    interaction = np.zeros(D)
    for i in range(D):
        for j in range(D):
            interaction[i] += perception[j] * wi[h * CHANNELS * HIDDEN + j * HIDDEN + i]
    interaction = _gelu_tanh(interaction)
    output = np.zeros(D)
    for i in range(D):
        for j in range(HIDDEN):
            output[i] += interaction[j % D] * wv[h * HIDDEN * CHANNELS + j * CHANNELS + i]
    return perception, interaction, output


def test_embedding_shapes_and_zero_blocks():
    wp, wi, wv, m, k = _reference_weights()
    p = from_reference_weights(wp, wi, wv, m, k)
    C = H * D
    for n in ("WP", "WI", "WV"):
        assert p[n].shape == (1, C, C) and p[n].dtype == np.float32
        off = p[n][0].copy()
        for h in range(H):
            off[h * D:(h + 1) * D, h * D:(h + 1) * D] = 0
        assert not off.any(), n
    assert p["K"].shape == (1, H, 9) and np.array_equal(p["K"][0, 3], k[3].ravel())
    assert p["K"][0, 2, 3 * (1 + 1) + (-1 + 1)] == k[2, 2, 0]  # tap (dy=+1, dx=-1)
    assert np.array_equal(p["M"][0], m)


def test_embedded_chain_equals_reference_per_head_loops(oracle):
    wp, wi, wv, m, k = _reference_weights()
    p = from_reference_weights(wp, wi, wv, m, k)
    cfg = OracleConfig(B=1, G=8, H=H, D=D, pvi_chain=True)
    X = np.random.default_rng(5).random((1, 8, 8, H * D), dtype=np.float32)
    P, I, V = oracle.project(cfg, X, p["WP"], p["WI"], p["WV"])
    for (y, x) in [(0, 0), (3, 5), (7, 2)]:
        cell = X[0, y, x].astype(np.float64)
        for h in (0, 3, 7):
            rp, ri, rv = _reference_head(cell[h * D:(h + 1) * D], h, wp, wi, wv)
            blk = slice(h * D, (h + 1) * D)
            np.testing.assert_allclose(P[0, y, x, blk], rp, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(I[0, y, x, blk], ri, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(V[0, y, x, blk], rv, rtol=1e-5, atol=1e-6)


def test_value_fold_is_needed():
    """Taking only the first D rows of the value slab (no fold) would not match:
    the reference's output sums all HIDDEN rows through j % D."""
    wp, wi, wv, m, k = _reference_weights()
    p = from_reference_weights(wp, wi, wv, m, k)
    assert not np.allclose(p["WV"][0, :D, :D], wv[0, :D, :D])
    np.testing.assert_allclose(p["WV"][0, :D, :D], wv[0, :, :D].reshape(HIDDEN // D, D, D).sum(0),
                               rtol=1e-6, atol=1e-7)


def test_short_slabs_are_rejected():
    wp, wi, wv, m, k = _reference_weights()
    with pytest.raises(ValueError):
        from_reference_weights(wp[:, :32], wi, wv, m, k)


def _reference_head_neighbourhood(X, y, x, h, wp, wi, wv):
    """As _reference_head, with the perception loop of pseudopod.cu:79-95 over the
    3 x 3 neighbourhood (dy, dx outer, channel c inner, as the kernel runs it) and
    the border wrapped (toroidal) where the kernel clamps."""
    G = X.shape[1]
    wp_f = np.asarray(wp, np.float64).ravel()
    perception = np.zeros(D)
    for i in range(D):
        for dy in range(3):
            for dx in range(3):
                nb = X[0, (y + dy - 1) % G, (x + dx - 1) % G, h * D:(h + 1) * D].astype(np.float64)
                for c in range(D):
                    perception[i] += nb[c] * wp_f[h * CHANNELS * HIDDEN + c * HIDDEN + i]
        perception[i] = max(0.0, perception[i])
    wi_f, wv_f = (np.asarray(a, np.float64).ravel() for a in (wi, wv))
    interaction = np.zeros(D)
    for i in range(D):
        for j in range(D):
            interaction[i] += perception[j] * wi_f[h * CHANNELS * HIDDEN + j * HIDDEN + i]
    interaction = _gelu_tanh(interaction)
    output = np.zeros(D)
    for i in range(D):
        for j in range(HIDDEN):
            output[i] += interaction[j % D] * wv_f[h * HIDDEN * CHANNELS + j * CHANNELS + i]
    return perception, interaction, output


def test_embedded_perception_chain_equals_reference_neighbourhood_loops(oracle):
    """pvi_chain 2 (the 3 x 3 neighbourhood sum before the perception product) against
    the reference kernel's own loops, at border cells, where the wrap matters, and an
    interior one."""
    wp, wi, wv, m, k = _reference_weights()
    p = from_reference_weights(wp, wi, wv, m, k)
    cfg = OracleConfig(B=1, G=8, H=H, D=D, pvi_chain=2)
    X = np.random.default_rng(6).random((1, 8, 8, H * D), dtype=np.float32)
    P, I, V = oracle.project(cfg, X, p["WP"], p["WI"], p["WV"])
    for (y, x) in [(0, 0), (3, 5), (7, 2), (0, 7)]:
        for h in (0, 5):
            rp, ri, rv = _reference_head_neighbourhood(X, y, x, h, wp, wi, wv)
            blk = slice(h * D, (h + 1) * D)
            np.testing.assert_allclose(P[0, y, x, blk], rp, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(I[0, y, x, blk], ri, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(V[0, y, x, blk], rv, rtol=1e-5, atol=1e-6)
    # and it differs from projecting the cell itself (pvi_chain 1)
    P1, _, _ = oracle.project(OracleConfig(B=1, G=8, H=H, D=D, pvi_chain=1), X, p["WP"], p["WI"],
                              p["WV"])
    assert not np.allclose(P1, P, rtol=1e-2)
