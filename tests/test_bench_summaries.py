"""bench.py's profile generators (--trace-summary, --traffic-summary), run on small
hand-made rocprofv3 CSVs whose figures are known: the achieved rates, the fractions of
peak and the counter scaling must come out as computed here by hand."""
import csv
import importlib.util
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _write_stats(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        for name, calls, avg in rows:
            w.writerow([name, calls, calls * avg, avg, 50.0, avg, avg, 0.0])


def _row(summary, needle):
    rows = [ln for ln in summary.splitlines() if needle in ln]
    assert len(rows) == 1, summary
    return [c.strip() for c in re.split(r"(?<!\\)\|", rows[0].strip().strip("|"))]  # cells; "\|" is text


def test_trace_summary_rates_and_fractions(bench, tmp_path):
    p = tmp_path / "run_kernel_stats.csv"
    _write_stats(p, [
        ("void slime::(anonymous namespace)::gemm_mfma_kernel<unsigned short>(slime::GemmArgs)", 4, 2.0e6),
        ("void slime::(anonymous namespace)::stencil_mfma_kernel<unsigned short, false>(slime::StencilArgs)",
         4, 1.0e6),
    ])
    s = bench.trace_summary(str(p), "c3")
    g = _row(s, "gemm_mfma_kernel")
    # 2 * 512 * 1536 flop per cell x 2^20 cells in 2 ms
    flops = 2 * 512 * 1536 * (1 << 20)
    assert g[3] == "2000.0" and g[8] == f"{flops:.4g} flop"
    assert g[9] == f"{flops / 2e-3 / 1e12:.0f} TFLOP/s"
    assert g[10] == f"{flops / 2e-3 / 1e12 / 2500:.1%} of 2.5 PFLOP/s"
    st = _row(s, "stencil_mfma_kernel<unsigned short, false>")
    b = 5 * 512 * 2 * (1 << 20)
    assert st[9] == f"{b / 1e-3 / 1e12:.2f} TB/s"
    assert st[10] == f"{b / 1e-3 / 1e12 / 8:.1%} of 8 TB/s"
    assert float(st[10].split("%")[0]) > 60  # 5.37 GB in 1 ms is 67 % of 8 TB/s, not 0


def test_trace_summary_c5_names_the_ring_cell_pass(bench, tmp_path):
    p = tmp_path / "run_kernel_stats.csv"
    _write_stats(p, [("void slime::(anonymous namespace)::bw_cell_ring_kernel(slime::BackwardArgs)", 2, 4.0e6),
                     ("void slime::(anonymous namespace)::bw_dw_mfma2_kernel(slime::BackwardArgs, slime::DwArgs)",
                      1, 1.9e6)])
    s = bench.trace_summary(str(p), "c5")
    c = _row(s, "bw_cell_ring_kernel")
    assert float(c[9].split()[0]) > 3.0  # 15.6 GB in 4 ms
    d = _row(s, "bw_dw_mfma2_kernel")
    assert d[9] == f"{2 * 512 * 1536 * (1 << 20) / 1.9e-3 / 1e12:.0f} TFLOP/s"


def _write_pmc(dirpath, counter, rows):
    os.makedirs(dirpath, exist_ok=True)
    with open(os.path.join(dirpath, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_ALL)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (name, value) in enumerate(rows):
            w.writerow([i, name, counter, value])


def test_traffic_summary_scales_by_the_calibration_copy(bench, tmp_path):
    # the kernel's name carries its variant arguments (growth function, loss sums)
    st = "void slime::(anonymous namespace)::stencil_mfma_kernel<unsigned short, false, false>(slime::StencilArgs)"
    gm = "void slime::(anonymous namespace)::gemm_mfma_kernel<unsigned short>(slime::GemmArgs)"
    # two dispatches each (the mean is taken), in two SE rows for one dispatch of the copy
    _write_pmc(tmp_path / "p_FETCH_SIZE", "FETCH_SIZE", [(st, 1000.0), (st, 3000.0), (gm, 500.0), (gm, 500.0)])
    _write_pmc(tmp_path / "p_WRITE_SIZE", "WRITE_SIZE", [(st, 400.0), (st, 400.0), (gm, 100.0), (gm, 300.0)])
    _write_pmc(tmp_path / "pc_FETCH_SIZE", "FETCH_SIZE", [("__amd_rocclr_copyBuffer", 524288.0)])
    _write_pmc(tmp_path / "pc_WRITE_SIZE", "WRITE_SIZE", [("__amd_rocclr_copyBuffer", 1048576.0)])
    md, js = bench.traffic_summary(str(tmp_path), "c3")
    s = js["c3"]["stencil"]
    assert s["read_bytes"] == 2000 * 2 * 1024 and s["write_bytes"] == 400 * 1024
    assert s["bytes_per_launch"] == s["read_bytes"] + s["write_bytes"]
    g = js["c3"]["gemm"]
    assert g["read_bytes"] == 500 * 2 * 1024 and g["write_bytes"] == 200 * 1024
    assert "FETCH_SIZE × 2.0000" in md and "WRITE_SIZE × 1.0000" in md


def test_trace_summary_c4_counts_its_own_cells(bench, tmp_path):
    p = tmp_path / "run_kernel_stats.csv"
    _write_stats(p, [("void slime::(anonymous namespace)::stencil_mfma_kernel<unsigned short, false>"
                      "(slime::StencilArgs)", 14, 0.5e6)])
    st = _row(bench.trace_summary(str(p), "c4"), "stencil_mfma_kernel")
    b = 5 * 512 * 2 * 16 * 128 * 128  # 16 pods x 128 x 128 cells
    assert st[8] == f"{b / 1e9:.3f} GB" and st[9] == f"{b / 0.5e-3 / 1e12:.2f} TB/s"


def test_trace_summary_tells_the_loss_summing_tape_step_from_the_plain_fp32_step(bench, tmp_path):
    p = tmp_path / "run_kernel_stats.csv"
    pre = "void slime::(anonymous namespace)::stencil_mfma_kernel"
    _write_stats(p, [(pre + "<float, false, true>(slime::StencilArgs)", 4, 1.0e6),
                     (pre + "<float, false, false>(slime::StencilArgs)", 2, 1.0e6)])
    s = bench.trace_summary(str(p), "c5")
    tape, plain = _row(s, "<float, false, true>"), _row(s, "<float, false, false>")
    C, cells = 512, 1 << 20
    assert tape[8] == f"{(5 * C * 2 + C * 4) * cells / 1e9:.3f} GB"  # reads T as well
    assert plain[8] == f"{(4 * C * 2 + C * 4) * cells / 1e9:.3f} GB"
