"""Calibration runs: a plain device copy of a known size for the rocprofv3 HBM
counters, and (``--ceilings``) the measured MFMA and HBM ceilings of the GPU.

``python -m slime_amd.calibrate --mib 1024`` copies a buffer of that many MiB
(device to device, torch's copy kernel) a few times. Profiled with
``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``), the counter reading of one
copy dispatch against the known byte count gives the factor that converts the
counters of the CA kernels into HBM bytes.

``python -m slime_amd.calibrate --ceilings`` prints one JSON line with the bf16
MFMA rate of a register-resident MFMA loop (random and all-zero operands) and the
streaming read / write / copy HBM bandwidth (``slime_amd/csrc/probe.hip``): what
this card sustains, beside the datasheet's 2.5 PFLOP/s and 8 TB/s.

``python -m slime_amd.calibrate --lds-banks`` runs the LDS bank probes of
``probe.hip``, one dispatch each, and prints one JSON line per dispatch naming it,
in dispatch order. Run it under ``rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT``:
the conflict cycles per LDS instruction of each dispatch give the projection GEMM's
patterns (old and current layouts) and, from single-lane displacements of a linear
pattern, which lanes gfx950 serves together and over how many bank groups.
"""
from __future__ import annotations

import argparse


def ceilings() -> dict:
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libslime_probe.so"))
    lib.slime_probe_mfma_tflops.restype = ctypes.c_double
    lib.slime_probe_hbm_gbs.restype = ctypes.c_double
    return {
        "mfma_bf16_tflops_random": lib.slime_probe_mfma_tflops(1),
        "mfma_bf16_tflops_zeros": lib.slime_probe_mfma_tflops(0),
        "hbm_read_gbs": lib.slime_probe_hbm_gbs(0),
        "hbm_write_gbs": lib.slime_probe_hbm_gbs(1),
        "hbm_copy_gbs": lib.slime_probe_hbm_gbs(2),
    }


LDS_PATTERNS = ["linear 16-byte reads", "GEMM fragment reads", "GEMM fragment reads, earlier swizzle",
                "GEMM staging writes", "GEMM staging reads", "earlier staging writes (144-byte rows)",
                "earlier staging reads (144-byte rows)"]


def lds_bank_runs():
    """(label, probe call) of every LDS bank dispatch, in order."""
    runs = [(f"pattern {k}: {name}", ("pattern", k)) for k, name in enumerate(LDS_PATTERNS)]
    for width, write in ((16, 0), (8, 0), (8, 1)):
        op = f"{'write' if write else 'read'} {width} B"
        for who, ks in ((63, range(0, 63)), (0, range(1, 64))):
            runs += [(f"pair {op}: lane {who} at lane {k}'s slot + 2048", ("pair", width, write, who, k, 2048))
                     for k in ks]
    for k in (15, 31, 47, 59):
        runs += [(f"pair read 16 B: lane 63 at lane {k}'s slot + {d}", ("pair", 16, 0, 63, k, d))
                 for d in (256, 512, 1024, 4096, 128, 64)]
    return runs


def lds_banks() -> None:
    import ctypes
    import json
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.abspath(__file__)), "libslime_probe.so"))
    for i, (label, call) in enumerate(lds_bank_runs()):
        rc = lib.slime_probe_lds_pattern(call[1]) if call[0] == "pattern" else lib.slime_probe_lds_pair(*call[1:])
        if rc != 0:
            raise RuntimeError(f"LDS probe failed: {label}")
        print(json.dumps({"dispatch": i, "probe": label, "args": list(call)}))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--ceilings", action="store_true")
    ap.add_argument("--lds-banks", action="store_true")
    args = ap.parse_args()
    if args.lds_banks:
        lds_banks()
        return
    if args.ceilings:
        import json
        print(json.dumps(ceilings()))
        return
    import torch
    n = args.mib * 1024 * 1024 // 4
    src = torch.rand(n, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {args.mib} MiB x {args.reps} (read {args.mib} MiB + write {args.mib} MiB per copy)")


if __name__ == "__main__":
    main()
