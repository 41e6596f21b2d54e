"""Plain device-to-device copy of a known size: the calibration kernel for HBM traffic counters.

    python calib_copy.py --mib 1024 --reps 4

Under `rocprofv3 --pmc FETCH_SIZE` (then `--pmc WRITE_SIZE`) each copy dispatch must read and write
exactly mib MiB; the ratio of the counter to that size is the factor by which the same counters of the
engine's kernels are scaled to bytes.
"""
from __future__ import annotations

import argparse
import json


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=4)
    args = ap.parse_args()
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("calib_copy needs a GPU")
    n = args.mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    src.fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.reps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.reps
    print(json.dumps({"copy_bytes": n, "reps": args.reps, "ms_per_copy": round(ms, 4),
                      "GB_s_read_plus_write": round(2 * n / ms / 1e6, 1)}), flush=True)


if __name__ == "__main__":
    main()
