#!/usr/bin/env python3
"""Calibration workload for the HBM traffic counters: a plain elementwise kernel of known size.

y = x + 1 over float32 vectors of --mib MiB each (reads --mib MiB, writes --mib MiB per dispatch),
--reps dispatches. Run under `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE`; the ratio of the
known bytes to the counter's reading per dispatch is the factor that turns the same counter's
reading on the decode kernel into bytes.

    rocprofv3 --pmc FETCH_SIZE -d out -o calib -- python3 fleet-amd-task_amd/harness/copy_calib.py
"""
import argparse

import torch


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args()
    n = a.mib * (1 << 20) // 4
    x = torch.zeros(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(a.reps):
        torch.add(x, 1.0, out=y)
    torch.cuda.synchronize()
    print(f"copy_calib: {a.reps} dispatches of y = x + 1, {a.mib} MiB read + {a.mib} MiB written each", flush=True)


if __name__ == "__main__":
    main()
