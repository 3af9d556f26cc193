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


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--ceilings", action="store_true")
    args = ap.parse_args()
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
