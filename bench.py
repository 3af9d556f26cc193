"""Benchmark: CA cell-updates/s of the multi-head neural-CA step on one MI355X.

Workload ("c3"): 128x128 toroidal grid, 8 heads, head_dim 64,
batch 64, bf16 state and weights with fp32 accumulation, synthetic seeded input
resident in HBM. One step = S1 projections ([P|I|V] GEMM, 1,048,576 x 512 x 1536)
+ the fused stencil (S2-S6) + mass conservation (S7) over the whole batch; one
cell-update = one (batch, y, x) cell advanced one step across all 8 heads x 64
channels. The timed region is a single slime_ca_step call of K steps.

Prints one JSON line. ``roofline`` describes the dominant kernel, measured with
HIP events on the library's stream in a second pass of K steps;
``cpu_baseline`` times the CPU oracle on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "CA cell-updates/s (128², 8 heads, d=64) on 1 MI355X; % HBM / MFMA peak"
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_TFLOPS = {"bf16": 2500.0, "fp32": 157.3}  # dense MFMA


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def stencil_bytes_per_cell(cfg) -> int:
    """Algorithmic HBM bytes of the fused stencil per cell-update: read X, P, I, V
    and write Y once (C channels each), plus per-cell mu, sigma when present."""
    elem = 2 if cfg.dtype == "bf16" else 4
    return 5 * cfg.C * elem + (2 * cfg.H * 4 if cfg.growth_per_cell else 0)


def gemm_flops_per_cell(cfg) -> int:
    """2 * C * 3C multiply-adds per cell for the fused [P|I|V] projection."""
    return 2 * cfg.C * 3 * cfg.C


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    committed under profiles/; None when no measurement is committed."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data.get(workload, {}).get(kernel, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def load_ceilings() -> dict:
    """Rates measured on the card (profiles/ceilings.json); empty when not committed."""
    try:
        with open(os.path.join(ROOT, "profiles", "ceilings.json")) as f:
            return {k: v for k, v in json.load(f).items() if not k.startswith("_")}
    except (OSError, ValueError):
        return {}


def cpu_model() -> str:
    """The host CPU's model name (as lscpu reports it, from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(cfg, params, X, seconds: float):
    """The CPU oracle on batch entry 0 of the workload: one warm-up step, then five
    samples of k steps each (k sized so the five take about `seconds`); the median
    sample's rate."""
    import statistics

    import numpy as np

    import oracle
    from slime_amd import round_bf16
    ocfg = oracle.OracleConfig(B=1, G=cfg.G, H=cfg.H, D=cfg.D, pods=1,
                               growth_per_cell=cfg.growth_per_cell, dt=cfg.dt)
    p = {k: (round_bf16(v[:1]) if k in ("WP", "WI", "WV") else v[:1]) for k, v in params.items()}
    x1 = np.ascontiguousarray(X[0:1])
    t0 = time.perf_counter()
    oracle.step(ocfg, x1, p, 1)  # warm-up (page-in, thread pool); sizes the samples
    k = max(1, int(round(seconds / 5 / (time.perf_counter() - t0))))
    per_step = []
    for _ in range(5):
        t0 = time.perf_counter()
        oracle.step(ocfg, x1, p, k)
        per_step.append((time.perf_counter() - t0) / k)
    med = statistics.median(per_step)
    cells = cfg.G * cfg.G
    return {
        "value": cells / med,
        "unit": "cell-updates/s",
        "cores": oracle.num_threads(),
        "kind": "port",
        "cpu_model": cpu_model(),
        "sample": f"CPU oracle (fp64, OpenMP) on batch entry 0 of the same workload "
                  f"({cells} cells): 1 warm-up step, then the median of 5 samples of {k} "
                  f"step(s) each ({min(per_step) * 1e3:.0f}-{max(per_step) * 1e3:.0f} ms per step)",
    }


# ---- rocprofv3 kernel-trace summaries ------------------------------------------------
# Algorithmic work per launch of the kernels of each workload: ("B", bytes) for an
# HBM-bound kernel, ("F", flops) for a matrix-core one, per cell of the launch
# (_TRACE_CELLS: 1,048,576 cells in c3 and c5, 16 pods x 128 x 128 = 262,144 in c4).
# Reads and writes are counted once per cell.
_TRACE_CELLS = {"c3": 1 << 20, "c5": 1 << 20, "c4": 16 * 128 * 128}



def _trace_work(workload: str) -> dict:
    C = 512
    if workload == "c3":
        return {
            "gemm_mfma_kernel<unsigned short>": ("[P\\|I\\|V] projection GEMM", "F", 2 * C * 3 * C),
            "stencil_mfma_kernel<unsigned short>": ("S2-S6 + mass partials, bf16 out", "B", 5 * C * 2),
            "stencil_mfma_kernel<float>": ("last step of a call, fp32 out", "B", 4 * C * 2 + C * 4),
            "rescale_kernel<float, unsigned short>": ("final rescale, fp32 -> bf16", "B", C * 4 + C * 2),
            "weight_prep_kernel<unsigned short>": ("per-batch scaled weights", None, None),
            "mass_finalize_kernel": ("S7 factors", None, None),
        }
    if workload == "c5":
        return {
            "bw_cell_ring_kernel": (
                "S7-S4 per (cell, head), tape for the gathers", "B",
                5 * C * 2 + C * 4 + 3 * C * 4 + C * 2 + 2 * 8 * 9 * 4),
            "bw_gather_tile_kernel<unsigned short>": (
                "gV, gI~, potential transpose", "B", 3 * C * 4 + 2 * C * 2 + 2 * 8 * 9 * 4 + 2 * C * 2 + C * 4),
            "gemm_mfma_add_kernel<unsigned short>": ("dX GEMM + direct part", "F", 2 * C * 3 * C),
            "bw_dw_mfma2_kernel": ("weight gradients", "F", 2 * C * 3 * C),
            "gemm_mfma_tape_kernel<unsigned short>": ("tape projections, I also before GELU", "F", 2 * C * 3 * C),
            "gemm_mfma_kernel<unsigned short>": ("forward projections (the forward timing)", None, None),
            "stencil_mfma_kernel<float, false, true>": (
                "tape step, fp32 out, loss sums (reads T)", "B", 5 * C * 2 + C * 4),
            "stencil_mfma_kernel<float>": ("forward timing: last step, fp32 out", "B", 4 * C * 2 + C * 4),
            "stencil_mfma_kernel<unsigned short>": ("forward step", "B", 5 * C * 2),
            "bw_loss_partial_kernel<unsigned short>": ("loss partials", "B", C * 4 + C * 2),
        }
    if workload == "c4":
        return {
            "fitness_finalize_kernel<64>": ("Jacobi eigenvalues, effective rank, fitness", None, None),
            "gemm_mfma_kernel<unsigned short>": ("[P\\|I\\|V] projection GEMM", "F", 2 * C * 3 * C),
            "stencil_mfma_kernel<float>": ("single-step calls: fp32 out", "B", 4 * C * 2 + C * 4),
            "fitness_partial_kernel<unsigned short, 64>": (
                "8-state history read once, fp64 Gram of the last", "B", 8 * C * 2),
            "stencil_mfma_kernel<unsigned short>": ("rollout: bf16 states", "B", 5 * C * 2),
            "rescale_kernel<float, unsigned short>": ("single-step calls only", "B", C * 4 + C * 2),
            "weight_prep_kernel<unsigned short>": ("per-pod scaled weights", None, None),
            "mass_finalize_kernel": ("S7 factors", None, None),
            "fill_f64_kernel": ("the rollout's unit factors of state 0", None, None),
        }
    return {}


def _short_name(full: str) -> str:
    """The kernel's name and template arguments, without namespaces or parameters."""
    name = full.replace("void ", "", 1)
    for pre in ("slime::(anonymous namespace)::", "slime::"):
        name = name.replace(pre, "")
    return name.split("(")[0].strip()


def _work_key(name: str, work: dict) -> str:
    """The key of `work` for a kernel: its full name when listed (variants whose work
    differs), else the name with the boolean template arguments removed (the
    growth-function instantiations do the same work per launch)."""
    import re
    return name if name in work else re.sub(r", (true|false)", "", name)


def trace_summary(path: str, workload: str, cells: int = 0) -> str:
    """Markdown table of a rocprofv3 --stats kernel CSV: calls and durations of each
    kernel and, for the kernels of `workload` with a known algorithmic work, the
    achieved rate and its fraction of the MI355X peak (`cells` per launch: the
    workload's own when 0)."""
    import csv
    work = _trace_work(workload)
    cells = cells or _TRACE_CELLS.get(workload, 1 << 20)
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((_short_name(r["Name"]), int(r["Calls"]), float(r["AverageNs"]),
                         float(r["TotalDurationNs"]), float(r["Percentage"]), float(r["MinNs"]),
                         float(r["MaxNs"])))
    lines = ["| kernel | what | calls | avg µs | min µs | max µs | total ms | % GPU time | "
             "work per launch | achieved | of peak |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    for name, calls, avg, tot, pct, mn, mx in sorted(rows, key=lambda r: -r[3]):
        if _work_key(name, work) not in work:
            continue
        what, kind, per_cell = work[_work_key(name, work)]
        cols = [f"`{name}`", what, str(calls), f"{avg / 1e3:.1f}", f"{mn / 1e3:.1f}", f"{mx / 1e3:.1f}",
                f"{tot / 1e6:.2f}", f"{pct:.2f}"]
        if kind == "B":
            b = per_cell * cells
            rate = b / (avg * 1e-9) / 1e12
            cols += [f"{b / 1e9:.3f} GB", f"{rate:.2f} TB/s", f"{rate * 1e3 / PEAK_HBM_GBS:.1%} of 8 TB/s"]
        elif kind == "F":
            fl = per_cell * cells
            rate = fl / (avg * 1e-9) / 1e12
            cols += [f"{fl:.4g} flop", f"{rate:.0f} TFLOP/s",
                     f"{rate / PEAK_TFLOPS['bf16']:.1%} of 2.5 PFLOP/s"]
        else:
            cols += ["-", "-", "-"]
        lines.append("| " + " | ".join(cols) + " |")
    return "\n".join(lines)


# ---- rocprofv3 --pmc HBM traffic summaries ------------------------------------------
# The kernels whose traffic bench.py reports, keyed as pmc_traffic.json keys them, with
# the short names of their workload's launches (boolean template arguments removed).
_TRAFFIC_KERNELS = {"c3": {"stencil": "stencil_mfma_kernel<unsigned short>",
                           "gemm": "gemm_mfma_kernel<unsigned short>"}}


def _counter_means(run_dir: str, counter: str) -> dict:
    """Mean per dispatch of `counter` (KiB as rocprofv3 reads it) by kernel short name,
    with the number of dispatches, from <run_dir>/run_counter_collection.csv."""
    import csv
    import collections
    sums, disp = collections.defaultdict(float), collections.defaultdict(set)
    with open(os.path.join(run_dir, "run_counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            k = _short_name(r["Kernel_Name"])
            sums[k] += float(r["Counter_Value"])
            disp[k].add(r["Dispatch_Id"])
    return {k: (sums[k] / len(disp[k]), len(disp[k])) for k in sums}


def traffic_summary(root: str, workload: str = "c3") -> tuple:
    """HBM bytes per launch from four rocprofv3 --pmc runs under `root`: p_FETCH_SIZE and
    p_WRITE_SIZE over the bench command, pc_FETCH_SIZE and pc_WRITE_SIZE over the 1 GiB
    copy of `python3 -m slime_amd.calibrate --mib 1024`. Each counter is scaled by what
    it reads for that copy (1 GiB read, 1 GiB written). Returns (markdown, json dict)."""
    fetch = _counter_means(os.path.join(root, "p_FETCH_SIZE"), "FETCH_SIZE")
    write = _counter_means(os.path.join(root, "p_WRITE_SIZE"), "WRITE_SIZE")
    cf = _counter_means(os.path.join(root, "pc_FETCH_SIZE"), "FETCH_SIZE")["__amd_rocclr_copyBuffer"]
    cw = _counter_means(os.path.join(root, "pc_WRITE_SIZE"), "WRITE_SIZE")["__amd_rocclr_copyBuffer"]
    kib = 1 << 20  # the copy moves 1 GiB each way
    f_fac, w_fac = kib / cf[0], kib / cw[0]
    lines = [f"Calibration: the 1 GiB copy reads FETCH_SIZE = {cf[0]:,.0f} KiB (mean of {cf[1]} "
             f"dispatches) and WRITE_SIZE = {cw[0]:,.0f} KiB, so HBM bytes = FETCH_SIZE × "
             f"{f_fac:.4f} × 1024 and WRITE_SIZE × {w_fac:.4f} × 1024.", "",
             "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | read GB | write GB | total GB |",
             "|---|---|---|---|---|---|---|"]
    out = {}
    names = {v: k for k, v in _TRAFFIC_KERNELS.get(workload, {}).items()}
    for k in sorted(fetch, key=lambda n: -fetch[n][0]):
        if k not in write:
            continue
        rd, wr = fetch[k][0] * f_fac * 1024, write[k][0] * w_fac * 1024
        lines.append(f"| `{k}` | {fetch[k][1]} | {fetch[k][0]:,.0f} | {write[k][0]:,.0f} | "
                     f"{rd / 1e9:.3f} | {wr / 1e9:.3f} | {(rd + wr) / 1e9:.3f} |")
        kk = _work_key(k, {})
        if kk in names:
            out[names[kk]] = {"read_bytes": round(rd), "write_bytes": round(wr),
                              "bytes_per_launch": round(rd + wr)}
    return "\n".join(lines), {workload: out}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c3")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--backward", action="store_true",
                    help="time the c5 gradient (slime_ca_backward) instead of the headline")
    ap.add_argument("--ensemble", action="store_true",
                    help="time the c4 ensemble: 16 pods' steps and the fused fitness")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="print a markdown roofline table of a rocprofv3 kernel_stats.csv "
                         "(no GPU needed) for --config c3, c4 or c5, then exit")
    ap.add_argument("--traffic-summary", metavar="DIR",
                    help="print the HBM bytes per launch from the four rocprofv3 --pmc runs "
                         "under DIR (p_FETCH_SIZE, p_WRITE_SIZE, pc_FETCH_SIZE, pc_WRITE_SIZE; "
                         "no GPU needed) as markdown and pmc_traffic.json's JSON, then exit")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.config))
        return 0
    if args.traffic_summary:
        md, js = traffic_summary(args.traffic_summary, args.config)
        print(md)
        print()
        print(json.dumps(js, indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this "
              "build (the path shards by batch with no collective)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from slime_amd import CONFIGS, Pseudopod, make_params, make_state

    if args.backward:
        return bench_backward(args)
    if args.ensemble:
        return bench_ensemble(args)
    cfg = CONFIGS[args.config]
    log(f"config {cfg}")
    params = make_params(cfg, seed=1)
    X = make_state(cfg, seed=2)
    tdt = torch.bfloat16 if cfg.dtype == "bf16" else torch.float32
    x = torch.from_numpy(X).to("cuda").to(tdt).contiguous()
    y = torch.empty_like(x)
    K, W = args.steps, args.warmup
    cells = cfg.cell_updates_per_step

    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, cfg.growth_per_cell,
                   cfg.pods) as ca:
        ca.set_params(params)
        log(f"MFMA projection path: {ca.uses_mfma}")
        if W > 0:
            ca.forward(x, out=y, n_steps=W)
        torch.cuda.synchronize()
        log("warmup done")

        # ---- timed region: exactly K steps ------------------------------------------
        stream = torch.cuda.current_stream()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        ca.forward(x, out=y, n_steps=K)
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        dev_ms = ev0.elapsed_time(ev1)
        log(f"timed {K} steps: {wall * 1e3:.2f} ms wall, {dev_ms:.2f} ms device")
        mass_in, mass_out = ca.mass()
        drift = float(np.max(np.abs(mass_out - mass_in) / np.abs(mass_in)))
        finite = bool(torch.isfinite(y.float()).all())

        # ---- per-kernel durations (HIP events on the library's stream) ----------------
        ca.set_timing(True)
        ca.forward(x, out=y, n_steps=K)
        t = ca.timings()
        ca.set_timing(False)

    ms_per_step = wall * 1e3 / K
    value = cells * K / wall
    gemm_ms = t["gemm_ms"] / max(t["gemm_launches"], 1)
    sten_ms = t["stencil_ms"] / max(t["stencil_launches"], 1)
    sb = stencil_bytes_per_cell(cfg) * cells
    gf = gemm_flops_per_cell(cfg) * cells
    wl = f"{cfg.name}"
    kernels = {
        "stencil": {"bound": "hbm", "achieved": sb / (sten_ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "avg_ms": sten_ms, "algorithmic_bytes": sb,
                    "traffic": load_traffic("stencil", wl)},
        "projection_gemm": {"bound": "mfma", "achieved": gf / (gemm_ms * 1e-3) / 1e12,
                            "peak": PEAK_TFLOPS[cfg.dtype], "unit": "TFLOP/s", "avg_ms": gemm_ms,
                            "algorithmic_flops": gf, "traffic": load_traffic("gemm", wl)},
    }
    # Beside the datasheet fractions: the fraction of what the card sustains (the
    # stencil reads four planes and writes one, a copy-like stream; the GEMM against a
    # register-only MFMA loop).
    ceil = load_ceilings()
    measured = {"stencil": ceil.get("hbm_copy_gbs"),
                "projection_gemm": ceil.get("mfma_bf16_tflops_random") if cfg.dtype == "bf16" else None}
    for name, k in kernels.items():
        k["frac"] = k["achieved"] / k["peak"]
        if measured[name]:
            k["measured_peak"] = measured[name]
            k["frac_of_measured"] = k["achieved"] / measured[name]
    dom_name = "stencil" if sten_ms >= gemm_ms else "projection_gemm"
    dom = kernels[dom_name]
    roofline = {"kernel": dom_name, "bound": dom["bound"], "achieved": dom["achieved"],
                "peak": dom["peak"], "unit": dom["unit"], "frac": dom["frac"],
                "traffic": dom["traffic"]}
    log(f"stencil {sten_ms:.3f} ms ({kernels['stencil']['frac']:.1%} of HBM), gemm {gemm_ms:.3f} ms "
        f"({kernels['projection_gemm']['frac']:.1%} of MFMA)")

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline")
        cpu = cpu_baseline(cfg, params, X, args.cpu_seconds)

    out = {
        "metric": METRIC, "value": value, "unit": "cell-updates/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": cfg.dtype,
        "data": "synthetic: seeded U[0,1) state with 5% blobs, N(0,0.05) weights, "
                "mu~U[0.1,0.3], sigma~U[0.01,0.05]",
        "config": {"workload": f"{cfg.name}: {cfg.G}x{cfg.G} toroidal grid, {cfg.H} heads, "
                               f"head_dim {cfg.D}, batch {cfg.B}, {cfg.dtype}, "
                               f"{K} steps per call",
                   "grid": cfg.G, "heads": cfg.H, "head_dim": cfg.D, "batch": cfg.B,
                   "steps_per_call": K, "parallelism": "single GPU"},
        "device_ms_per_step": dev_ms / K,
        "mass_drift_max": drift, "finite": finite,
        "roofline": roofline, "kernels": kernels, "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


def _time(fn, reps: int):
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e3


def bench_backward(args) -> int:
    """c5: one forward step plus the gradient of the MSE loss,
    with and without the weight gradients; prints one JSON line."""
    import numpy as np
    import torch

    from slime_amd import CONFIGS, Pseudopod, make_params, make_state
    cfg = CONFIGS["c5"]
    log(f"config {cfg}")
    p = make_params(cfg, seed=1)
    x = torch.from_numpy(make_state(cfg, seed=2)).to("cuda").to(torch.bfloat16).contiguous()
    t = torch.rand(x.shape, generator=torch.Generator().manual_seed(3)).to("cuda").to(torch.bfloat16)
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, False, 1) as ca:
        ca.set_params(p)
        y = torch.empty_like(x)
        ca.forward(x, out=y)
        ca.backward(x, t)
        reps = max(args.steps // 2, 1)
        fwd = _time(lambda: ca.forward(x, out=y), reps)
        bwd_x = _time(lambda: ca.backward(x, t, params=False), reps)
        bwd = _time(lambda: ca.backward(x, t, params=True), reps)
        loss, _, _ = ca.backward(x, t, params=False)
    cells = cfg.cell_updates_per_step
    out = {"metric": "c5 forward + gradient time (512x512, 8 heads, d=64, batch 4, bf16)",
           "unit": "ms", "higher_is_better": False, "n_gpus": 1, "dtype": cfg.dtype,
           "data": "synthetic: seeded U[0,1) state with 5% blobs, U[0,1) target",
           "config": {"workload": "c5", "grid": cfg.G, "batch": cfg.B, "heads": cfg.H,
                      "head_dim": cfg.D},
           "forward_ms": fwd, "backward_dx_ms": bwd_x, "backward_all_ms": bwd,
           "cell_updates_per_s_backward_dx": cells / (bwd_x * 1e-3), "loss": loss, "reps": reps}
    print(json.dumps(out), flush=True)
    return 0


def bench_ensemble(args) -> int:
    """c4: 16 pods with independent weights, batch entry = pod, an 8-state history
    by slime_ca_rollout (the single-step calls timed beside it), then the fused
    fitness over it; prints one JSON line."""
    import torch

    from slime_amd import CONFIGS, Pseudopod, make_params, make_state
    cfg = CONFIGS["c4"]
    log(f"config {cfg}")
    p = make_params(cfg, seed=1)
    x0 = torch.from_numpy(make_state(cfg, seed=2, B=1)).to("cuda").to(torch.bfloat16)
    x0 = x0.expand(cfg.B, -1, -1, -1).contiguous()  # shared initial grid
    T = cfg.steps
    with Pseudopod(cfg.B, cfg.G, cfg.H, cfg.D, cfg.dtype, cfg.dt, False, cfg.pods) as ca:
        ca.set_params(p)
        hist = torch.empty((T,) + tuple(x0.shape), dtype=torch.bfloat16, device="cuda")
        box = {}

        def rollout():  # slime_ca_rollout: each state kept before its mass rescale
            hist[0].copy_(x0)
            box["scales"] = ca.rollout(hist)

        def single_steps():  # T - 1 calls of slime_ca_step, each rescaling its output
            hist[0].copy_(x0)
            for i in range(1, T):
                ca.forward(hist[i - 1], out=hist[i])

        single_steps()
        rollout()
        ca.fitness_scaled(hist, box["scales"])
        reps = max(args.steps // 2, 1)
        single_ms = _time(single_steps, reps)
        roll_ms = _time(rollout, reps)
        fit_ms = _time(lambda: ca.fitness_scaled(hist, box["scales"]), reps * 4)
        er, coh, fit = ca.fitness_scaled(hist, box["scales"])
        torch.cuda.synchronize()
    steps = T - 1
    out = {"metric": "c4 ensemble: step throughput and fused fitness latency",
           "unit": "cell-updates/s", "higher_is_better": True, "n_gpus": 1, "dtype": cfg.dtype,
           "data": "synthetic: 16 pods of seeded weights on one shared seeded grid",
           "config": {"workload": "c4", "pods": cfg.pods, "grid": cfg.G, "batch": cfg.B,
                      "history": T},
           "value": cfg.cell_updates_per_step * steps / (roll_ms * 1e-3),
           "rollout_ms": roll_ms, "single_step_calls_ms": single_ms, "steps": steps,
           "fitness_us": fit_ms * 1e3,
           "fitness_mean": float(fit.mean()), "erank_mean": float(er.mean()),
           "coherence_mean": float(coh.mean())}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
