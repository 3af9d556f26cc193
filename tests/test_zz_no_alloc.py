"""slime_ca_fitness_static, the allocation-free fitness entry point, through the C
ABI against slime_ca_fitness on the same histories: two calls in a row, the second
on a smaller history (fewer batch entries, a smaller grid, a shorter history and a
narrower head), so stale partial sums in the shared static buffer would show.
Both calls use the same chunk count as the handle's fitness, so the outputs agree
bit for bit. Also: the size limit is reported as SLIME_EINVAL before any device
work, and the entry point launches nothing when it rejects its arguments."""
import ctypes

import numpy as np
import pytest

from slime_amd import Pseudopod, _lib, make_params, make_state
from slime_amd.synthetic import CAConfig

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _needs_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _history(cfg, T, seed):
    """T states of the CA from a seeded start, on the device."""
    p = make_params(cfg, seed=seed)
    X = make_state(cfg, seed=seed + 1)
    tdt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt) as e:
        e.set_params(p)
        hist = torch.empty((T, cfg.B, cfg.G, cfg.G, cfg.C), dtype=tdt, device="cuda")
        hist[0] = torch.from_numpy(X).cuda().to(tdt)
        for t in range(1, T):
            e.forward(hist[t - 1], out=hist[t])
        torch.cuda.synchronize()
    return hist


def _handle_fitness(cfg, hist):
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt) as e:
        out = e.fitness(hist)
        torch.cuda.synchronize()
        return [o.cpu().numpy() for o in out]


def _static_fitness(cfg, hist):
    lib = _lib.load()
    c = _lib.Config(cfg.B, cfg.G, cfg.H, cfg.D, _lib.SLIME_BF16 if cfg.dtype == "bf16" else _lib.SLIME_F32,
                    cfg.dt, 0, 1, 0)
    outs = [torch.full((cfg.B, cfg.H), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.slime_ca_fitness_static(ctypes.byref(c), ctypes.c_void_p(hist.data_ptr()), int(hist.shape[0]),
                                     *[ctypes.c_void_p(o.data_ptr()) for o in outs], stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def test_static_fitness_matches_handle_fitness_on_two_calls():
    big = CAConfig("nalloc-big", B=4, G=32, H=8, D=64, dtype="bf16", steps=1, w_std=0.05, blobs=True)
    small = CAConfig("nalloc-small", B=1, G=16, H=8, D=32, dtype="fp32", steps=1, w_std=0.05)
    for cfg, T, seed in ((big, 8, 3), (small, 3, 7)):
        print(f"[case] slime_ca_fitness_static B={cfg.B} G={cfg.G} D={cfg.D} {cfg.dtype} T={T}", flush=True)
        hist = _history(cfg, T, seed)
        ref = _handle_fitness(cfg, hist)
        got = _static_fitness(cfg, hist)
        for name, g, r in zip(("erank", "coherence", "fitness"), got, ref):
            assert np.all(np.isfinite(g)), name
            np.testing.assert_array_equal(g, r, err_msg=name)
        print(f"  erank {got[0].mean():.6f}, coherence {got[1].mean():.6f}: equal to slime_ca_fitness")


def test_static_fitness_rejects_what_does_not_fit():
    lib = _lib.load()
    # 2048 (batch, head) Grams of 64 x 64 fp64 need 64 MiB even as one chunk.
    c = _lib.Config(256, 16, 8, 64, _lib.SLIME_BF16, 0.1, 0, 1, 0)
    dummy = torch.empty(16, dtype=torch.float32, device="cuda")
    p = ctypes.c_void_p(dummy.data_ptr())
    rc = lib.slime_ca_fitness_static(ctypes.byref(c), p, 8, p, p, p, ctypes.c_void_p(0))
    assert rc == _lib.SLIME_EINVAL
    assert b"static scratch" in lib.slime_ca_last_error()
    rc = lib.slime_ca_fitness_static(ctypes.byref(c), p, 1, p, p, p, ctypes.c_void_p(0))  # T < 2
    assert rc == _lib.SLIME_EINVAL


def test_static_fitness_calls_on_two_streams_are_ordered():
    """Two calls back to back on two streams, with no synchronisation between them:
    the second waits for the first's event before its kernels write the shared
    scratch, so both results equal slime_ca_fitness's."""
    cfg_a = CAConfig("nalloc-a", B=4, G=32, H=8, D=64, dtype="bf16", steps=1, w_std=0.05, blobs=True)
    cfg_b = CAConfig("nalloc-b", B=2, G=32, H=8, D=64, dtype="bf16", steps=1, w_std=0.05)
    print("[case] slime_ca_fitness_static on two streams", flush=True)
    ha, hb = _history(cfg_a, 8, 5), _history(cfg_b, 6, 9)
    ref_a, ref_b = _handle_fitness(cfg_a, ha), _handle_fitness(cfg_b, hb)
    lib = _lib.load()
    outs = []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for cfg, hist, st in ((cfg_a, ha, streams[0]), (cfg_b, hb, streams[1])):
        c = _lib.Config(cfg.B, cfg.G, cfg.H, cfg.D, _lib.SLIME_BF16, cfg.dt, 0, 1, 0)
        o = [torch.full((cfg.B, cfg.H), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
        rc = lib.slime_ca_fitness_static(ctypes.byref(c), ctypes.c_void_p(hist.data_ptr()),
                                         int(hist.shape[0]), *[ctypes.c_void_p(t.data_ptr()) for t in o],
                                         ctypes.c_void_p(st.cuda_stream))
        _lib.check(rc)
        outs.append(o)
    torch.cuda.synchronize()
    for got, ref in ((outs[0], ref_a), (outs[1], ref_b)):
        for name, g, r in zip(("erank", "coherence", "fitness"), got, ref):
            np.testing.assert_array_equal(g.cpu().numpy(), r, err_msg=name)
