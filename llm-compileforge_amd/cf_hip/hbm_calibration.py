"""HBM measurement helpers: counter calibration and the practical read rate.

Default mode -- a device-to-device copy of a known size, for calibrating HBM
byte counters.  Run under `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE):
each copy kernel reads and writes exactly --mib MiB, so the counter's
reading for it gives the factor between the counter and true bytes, which is
then applied to the decode kernel's reading.

    python llm-compileforge_amd/cf_hip/hbm_calibration.py --mib 1024 --reps 5

--read-probe -- the practical HBM read rate for the decode kernel's access
shape: 4,096 independent waves each read whole chunks (2 KiB .. 64 KiB) at
random offsets of an 8 GiB buffer (cf_hbm_read_probe in libcf_hip.so), 2 GiB
per launch, timed with HIP events on the launch stream; prints one line per
chunk size and a JSON summary.

    python llm-compileforge_amd/cf_hip/hbm_calibration.py --read-probe
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch


def copy_calibration(mib: int, reps: int) -> None:
    n = mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0")
    src.fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {mib} MiB x {reps}", flush=True)


def read_probe(buf_gib: int = 8, total_gib: int = 2, reps: int = 5) -> dict:
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from cf_hip._abi import check, lib

    dev = torch.device("cuda:0")
    buf_bytes = buf_gib << 30
    buf = torch.empty(buf_bytes, dtype=torch.uint8, device=dev)
    buf.fill_(3)
    waves = 4096
    sink = torch.zeros(waves * 64, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    out = {}
    for chunk in (2048, 4096, 8192, 16384, 32768, 65536):
        per_wave = max(1, (total_gib << 30) // chunk // waves)
        n_chunks = buf_bytes // chunk
        ids = torch.randperm(n_chunks, device=dev, generator=gen)[: waves * per_wave].to(torch.int32)

        def launch() -> None:
            check(lib().cf_hbm_read_probe(buf.data_ptr(), buf_bytes, ids.data_ptr(), waves, per_wave, chunk,
                                          sink.data_ptr(), stream.cuda_stream), "cf_hbm_read_probe")

        for _ in range(2):
            launch()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            launch()
        end.record(stream)
        end.synchronize()
        ms = start.elapsed_time(end) / reps
        gbs = waves * per_wave * chunk / (ms / 1e3) / 1e9
        out[chunk] = gbs
        print(f"chunk {chunk:6d} B: {gbs:8.1f} GB/s ({ms * 1e3:.1f} us per {waves * per_wave * chunk / 2**30:.2f} GiB)",
              flush=True)
    summary = {"probe": "random whole-chunk reads, 4096 waves, 8 GiB buffer", "gbs_by_chunk_bytes": out}
    print(json.dumps(summary), flush=True)
    return summary


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--read-probe", action="store_true")
    args = ap.parse_args()
    if args.read_probe:
        read_probe()
    else:
        copy_calibration(args.mib, args.reps)


if __name__ == "__main__":
    main()
