"""Host replay of the projection GEMM's addresses and vmcnt waits (CPU only).

``tests/gemm_addr_replay.cpp`` runs the tile kernel's own address functions
(``slime_amd/csrc/gemm_addr.hpp``, shared with ``gemm_tile.hpp``) for every
workgroup, wave and lane of a launch and checks every direct load, LDS access and
store against its buffer, and every ``s_waitcnt vmcnt`` against the in-order
completion of the wave's loads and stores. The launches are the ones the library
makes (``slime_amd/csrc/api.cpp``): the forward [P|I|V] GEMM, the chained
projections' per-plane GEMMs, the backward tape's pre-activation GEMM and the
backward dX GEMM (K = 3C, fp32 output with an addend), on every BASELINE
configuration whose shape takes the MFMA path, with the MI355X's 256 CUs and
with CU counts that exercise the other branch of the tile schedule.
"""
import os
import subprocess

import pytest

from slime_amd.synthetic import CONFIGS, CAConfig

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "gemm_addr_replay.cpp")


@pytest.fixture(scope="module")
def replay(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("replay") / "gemm_addr_replay")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-o", exe, SRC], check=True)
    return exe


def _uses_mfma(M, N, K, elem, rows_per_batch, ncol):
    k_group = 128 if elem == 2 else 64
    return M % 256 == 0 and N % 256 == 0 and ncol % 256 == 0 and K % k_group == 0 \
        and rows_per_batch % 256 == 0


def launches(cfg: CAConfig):
    """(name, M, N, K, elem, rows_per_batch, bt_batch_stride, bt_elems, ncol, nplanes,
    epilogue) of each GEMM the library launches for this configuration."""
    C, elem = cfg.C, (2 if cfg.dtype == "bf16" else 4)
    M, rpb, stride = cfg.B * cfg.G * cfg.G, cfg.G * cfg.G, 3 * C * C
    wt = cfg.B * 3 * C * C  # per-batch transposed weights [B][3C][C]
    epi = "bf16" if cfg.dtype == "bf16" else "f32"
    yield ("forward [P|I|V]", M, 3 * C, C, elem, rpb, stride, wt, C, 3, epi)
    for p in range(3):  # chained projections: one GEMM per plane, Bt offset by p C^2
        yield (f"chained plane {p}", M, C, C, elem, rpb, stride, wt - p * C * C, C, 1, epi)
    yield ("backward tape I~", M, C, C, elem, rpb, stride, wt - C * C, C, 1, epi)
    rows_pod = (cfg.B // cfg.pods) * cfg.G * cfg.G
    yield ("backward dX", M, C, 3 * C, elem, rows_pod, stride, cfg.pods * 3 * C * C, C, 1, "f32add")


CASES = [cfg for cfg in CONFIGS.values()] + [
    CAConfig("persist", B=24, G=32, H=8, D=64, dtype="bf16", steps=1, w_std=0.05, pods=3),
    CAConfig("fp32-32", B=2, G=32, H=8, D=64, dtype="fp32", steps=1, w_std=0.05),
]


def _run(exe, args, n_cu, extra=()):
    r = subprocess.run([exe, *map(str, args[1:10]), str(n_cu), args[10], *extra],
                       capture_output=True, text=True, timeout=300)
    return r.returncode, r.stdout.strip()


@pytest.mark.parametrize("cfg", CASES, ids=[c.name for c in CASES])
def test_every_gemm_address_in_bounds_and_every_wait_exact(replay, cfg):
    ran = 0
    for args in launches(cfg):
        name, M, N, K, elem, rpb = args[:6]
        if not _uses_mfma(M, N, K, elem, rpb, args[8]):
            continue
        for n_cu in (256, 80, 7):
            rc, out = _run(replay, args, n_cu)
            print(f"  {cfg.name} {name} n_cu={n_cu}: {out}")
            assert rc == 0 and out.startswith("OK"), (cfg.name, name, n_cu, out)
            ran += 1
    if cfg.name == "c1":
        assert ran == 0  # 32x32 grid, D 8: the generic kernel runs
    else:
        assert ran > 0


def test_replay_reports_planted_mistakes(replay):
    """The checks fire: a weight buffer one 16-row group short of the c3 launch's
    last tile, and waits modelled one slab looser than the kernel's."""
    args = next(launches(CONFIGS["c3"]))
    short_bt = list(args)
    short_bt[7] = args[7] - 16 * args[3]
    rc, out = _run(replay, short_bt, 256)
    assert rc == 1 and "direct load from Bt" in out, out
    rc, out = _run(replay, args, 256, ("plant-loose-wait",))
    assert rc == 1 and "too loose" in out, out


@pytest.mark.parametrize("plant,message", [
    ("PLANT_FRAG_CHUNK", "cell fragment reads the wrong row or chunk"),
    ("PLANT_NO_UNSWAP", "staging read-back holds the wrong row, chunk or half"),
])
def test_layout_check_reports_planted_mistakes(tmp_path, plant, message):
    """The LDS data-path check fires when a fragment read takes the neighbouring
    16-byte chunk, or when the staged read-back keeps its rows' halves swapped."""
    exe = str(tmp_path / "replay_planted")
    subprocess.run(["g++", "-O2", "-std=c++17", f"-D{plant}", "-o", exe, SRC], check=True)
    rc, out = _run(exe, next(launches(CONFIGS["c3"])), 256)
    assert rc == 1 and message in out, out
