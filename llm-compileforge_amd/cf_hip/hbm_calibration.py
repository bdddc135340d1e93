"""Device-to-device copy of a known size, for calibrating HBM byte counters.

Run under `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE): each copy kernel
reads and writes exactly --mib MiB, so the counter's reading for it gives
the factor between the counter and true bytes, which is then applied to the
decode kernel's reading.

    python llm-compileforge_amd/cf_hip/hbm_calibration.py --mib 1024 --reps 5
"""

from __future__ import annotations

import argparse

import torch


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()
    n = args.mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {args.mib} MiB x {args.reps}", flush=True)


if __name__ == "__main__":
    main()
