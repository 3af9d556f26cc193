"""Plain device copy of a known size, used to calibrate rocprofv3 HBM counters.

``python -m slime_amd.calibrate --mib 1024`` copies a buffer of that many MiB
(device to device, torch's copy kernel) a few times. Profiled with
``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``), the counter reading of one
copy dispatch against the known byte count gives the factor that converts the
counters of the CA kernels into HBM bytes.
"""
from __future__ import annotations

import argparse


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=3)
    args = ap.parse_args()
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
