"""Benchmark: paged decode with an FP8 KV cache on one MI355X.

Workload (default): BASELINE.json configs[2], Llama-3-8B attention shape --
batch 64, 32 query / 8 KV heads, head_dim 128, OCP e4m3 KV with per-KV-head
scales (sources bf16 N(0,1) with 1% outliers x8), block_size 16, context
U{1024..8192}, sequences 0..31 sharing a 1024-token prefix.  A step is one
decode attention call (one layer) over the whole batch; tokens/s = B / step.
Two copies of the cache pool alternate between steps so the 256 MB
Infinity Cache does not hold the previous step's KV.

Before the W warm-up steps the GPU is brought to a steady step time
(`settle`: untimed steps until three timed batches agree; an idle MI355X
runs its first ~100-200 launches of this workload 10-15 % slower while its
clocks ramp).  The K timed steps are bracketed by device synchronizations
and timed with HIP events on the launch stream.

Prints one JSON line (rank 0).  The CPU baseline is the oracle's
restatement of the reference CPU path (gather + dequantize + SDPA) on a
bounded sample of the same workload, timed on this host's cores.

`--config block_tables` times per-step block-table upkeep for 256 decoding
requests (full rebuild + upload vs the block pool's device deltas) and
copy-on-write block copies over Llama-3-8B-shaped FP8 slabs.

`--config c5_mixed` times BASELINE.json configs[4] instead: one mixed
step = FP8 write of the step's 4344 new K/V rows, then decode attention of
248 sequences and chunked-prefill attention of 8 x 512-token chunks side by
side on two streams (HBM-bound and MFMA-bound kernels overlap; the
one-stream step time is reported too); tokens/s counts the step's new
tokens (decodes + chunk rows).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "llm-compileforge_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFS = 2500.0
METRIC = "paged-decode tokens/s + HBM GB/s (% peak), Llama-3-8B shape FP8 KV, 1 MI355X"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(case, kc, vc, ks, vs, sample: int, budget_s: float) -> dict:
    """Times the oracle's CPU restatement on the first `sample` sequences."""
    import torch

    from oracle.paged_attention import paged_attention_cpu

    cores, host = cpu_share()
    torch.set_num_threads(cores)
    idx = list(range(sample))
    used = sorted({b for i in idx for b in case.block_tables[i]})
    remap = {b: j for j, b in enumerate(used)}
    sel = torch.tensor(used, device=kc.device)
    k_cpu = kc[sel].contiguous().cpu()
    v_cpu = vc[sel].contiguous().cpu()
    bt = {f"r{i}": [remap[b] for b in case.block_tables[i]] for i in idx}
    sl = {f"r{i}": case.seq_lens[i] for i in idx}
    q = case.q[:sample].float().cpu()
    kss = ks.cpu() if ks is not None else None
    vss = vs.cpu() if vs is not None else None
    paged_attention_cpu(q, k_cpu, v_cpu, bt, sl, case.block_size, case.scale, kss, vss)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        paged_attention_cpu(q, k_cpu, v_cpu, bt, sl, case.block_size, case.scale, kss, vss)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": sample / med,
        "unit": "tokens/s",
        "cores": cores,
        "host": host,
        "kind": "port",
        "sample": f"first {sample} of {case.batch} sequences of {case.name} "
        f"({sum(case.seq_lens[:sample])} context tokens), median of {len(times)} runs",
    }


def cpu_share() -> tuple[int, dict]:
    """Threads for the CPU baseline and a description of the host.

    All CPUs this process may run on (its affinity mask), capped by
    OMP_NUM_THREADS when the environment sets it: a GPU box gives each GPU a
    share of the host's cores and says so there, and more torch threads than
    that share only contend."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    cores = avail
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        cores = min(cores, int(omp))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return max(1, cores), {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": avail,
                           "omp_num_threads": omp or None}


def settle(step, batch: int, max_steps: int, min_steps: int = 0, tol: float = 0.005) -> dict:
    """Untimed steps until the GPU's step time is steady.

    An idle MI355X runs its first ~100-200 launches of this workload
    10-15 % slower than it runs them a few tens of ms later (its clocks
    ramp up under load; measured: 122.5 us per c3 step over the first 20
    timed steps after 20 warm-up steps, 108.2 us once settled), so a short
    warm-up alone would time the ramp.  Batches of `batch` steps are timed
    with HIP events until three in a row agree within `tol` (after at least
    `min_steps`), at most `max_steps` steps; the W warm-up steps and the
    timed K steps follow.
    `step(i)` runs step i.  Returns the batches' per-step times."""
    import torch

    times: list[float] = []
    i = 0
    while i < max_steps:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(batch):
            step(i)
            i += 1
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / batch)
        if (i >= min_steps and len(times) >= 3
                and all(abs(times[-k] - times[-k - 1]) <= tol * times[-k] for k in (1, 2))):
            break
    return {"steps": i, "batch_steps": batch, "us_per_step_by_batch": [round(t * 1e3, 1) for t in times],
            "rule": f"batches of {batch} untimed steps until three in a row agree within {tol:.1%} "
                    f"(at least {min_steps}, at most {max_steps} steps), before the W warm-up steps"}


def load_traffic(config: str, kernel: str | None = None) -> float | None:
    """Calibrated HBM bytes per launch (FETCH_SIZE / WRITE_SIZE counter
    runs, profiles/traffic_<config>.json) of the config's main kernel, or of
    `kernel` where the file lists several."""
    path = ROOT / "profiles" / f"traffic_{config}.json"
    if path.exists():
        try:
            data = json.loads(path.read_text())
            entry = data["kernels"][kernel] if kernel is not None else data
            return float(entry["hbm_bytes_per_launch"])
        except (KeyError, ValueError, TypeError):
            return None
    return None


def bench_mixed(args) -> dict:
    """One c5 step per iteration: kv write + decode + chunked prefill."""
    import torch

    from cf_hip import ops, workloads
    from kernels.paged_attention import chunked_prefill_attention

    dev = torch.device("cuda:0")
    case = workloads.make_mixed_case(args.config, device=dev, seed=0)
    alg = workloads.mixed_algorithmic(case)
    pools = [workloads.materialize_mixed(case, args.layout) for _ in range(args.pools)]
    steps_fns = []
    for t in pools:
        plan = ops.DecodePlan(t["q_decode"], t["k_cache"], t["v_cache"], t["decode_tables"], t["decode_lens"],
                              case.scale, case.block_size, t["k_scale"], t["v_scale"], args.partition)
        ws = ops.new_workspace(ops.prefill_workspace_bytes(case.q_prefill.shape[0], len(case.prefill_lens),
                                                           case.q_prefill.shape[1], case.num_kv_heads,
                                                           case.q_prefill.shape[2]), dev)
        out_p = torch.empty_like(t["q_prefill"])

        def prefill(t=t, ws=ws, out_p=out_p):
            chunked_prefill_attention(t["q_prefill"], t["k_cache"], t["v_cache"], t["prefill_tables"],
                                      t["prefill_lens"], t["q_start"], case.block_size, case.scale,
                                      k_scale=t["k_scale"], v_scale=t["v_scale"], out=out_p, workspace=ws)

        def step(t=t, plan=plan, prefill=prefill, serial=False):
            ops.kv_write_fp8(t["k_new"], t["v_new"], t["slots"], t["k_cache"], t["v_cache"], t["k_scale"],
                             t["v_scale"])
            if serial:
                plan.run()
                prefill()
            else:
                ops.run_concurrent(plan.run, prefill, dev)

        steps_fns.append(step)
    torch.cuda.synchronize()
    log(f"c5: {alg['decode_tokens']} decodes, {alg['prefill_tokens']} chunk rows; decode bytes "
        f"{alg['decode_bytes'] / 1e9:.2f} GB, prefill {alg['prefill_flops'] / 1e9:.1f} GFLOP")
    one = args.one_stream
    settled = None
    if not args.no_settle:
        settled = settle(lambda i: steps_fns[i % len(steps_fns)](serial=one), batch=5, min_steps=40,
                         max_steps=150)
        log(f"settle: {settled['steps']} steps, us/step by batch {settled['us_per_step_by_batch']}")
    for i in range(args.warmup):
        steps_fns[i % len(steps_fns)](serial=one)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        steps_fns[i % len(steps_fns)](serial=one)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    # The same steps on one stream (kernels one after another), for the
    # per-kernel durations below and as the no-overlap reference.
    ms_serial = ms_step
    if not one:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            steps_fns[i % len(steps_fns)](serial=True)
        torch.cuda.synchronize()
        ms_serial = (time.perf_counter() - t0) * 1e3 / args.steps
    # per-kernel durations: one-stream steps with launch-stamped events, all
    # created beforehand (5 launches a step, 2 events each)
    ops.KernelTimer.reserve(10 * args.steps + 16)
    with ops.KernelTimer() as timer:
        for i in range(args.steps):
            steps_fns[i % len(steps_fns)](serial=True)
        torch.cuda.synchronize()
    us = {}
    for name in ("cf_kv_write_fp8", "cf_decode_mfma", "cf_decode_merge", "cf_prefill_plan", "cf_prefill_mfma"):
        ms, n = timer.query(name)
        us[name] = ms / max(n, 1) * 1e3
    timer.reset()
    log(f"{ms_step * 1e3:.1f} us/step (one stream: {ms_serial * 1e3:.1f}); "
        + ", ".join(f"{k} {v:.1f} us" for k, v in us.items()))
    dec_s = us["cf_decode_mfma"] / 1e6
    pre_s = us["cf_prefill_mfma"] / 1e6
    dec_gbs = alg["decode_bytes"] / dec_s / 1e9
    pre_tf = alg["prefill_flops"] / pre_s / 1e12
    tokens = alg["decode_tokens"] + alg["prefill_tokens"]
    return {
        "metric": "mixed chunked-prefill + decode step tokens/s, Llama-3-8B shape FP8 KV, 1 MI355X",
        "value": tokens / (ms_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 KV / bf16 q / f32 accumulate",
        "data": "synthetic (seeded), random-init",
        "config": {"workload": args.config, "decodes": alg["decode_tokens"], "chunk_rows": alg["prefill_tokens"],
                   "chunks": len(case.prefill_lens), "num_q_heads": case.q_prefill.shape[1],
                   "num_kv_heads": case.num_kv_heads, "head_dim": case.q_prefill.shape[2],
                   "block_size": case.block_size, "kv_layout": args.layout, "cache_pools_rotated": args.pools,
                   "parallelism": "single GPU"},
        "kernel_us": us,
        "settle": settled,
        "overlap": {"decode_prefill_streams": 1 if one else 2, "ms_per_step_one_stream": ms_serial,
                    "note": "kernel_us are one-stream durations; value is the two-stream step"},
        "algorithmic": alg,
        "roofline": {"bound": "hbm", "kernel": "cf_decode_mfma", "achieved": dec_gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": dec_gbs / HBM_PEAK_GBS,
                     "traffic": load_traffic(args.config, "cf_decode_mfma")},
        "roofline_prefill": {"bound": "mfma", "kernel": "cf_prefill_mfma", "achieved": pre_tf,
                             "peak": BF16_MFMA_PEAK_TFS, "unit": "TFLOP/s", "frac": pre_tf / BF16_MFMA_PEAK_TFS,
                             "traffic": load_traffic(args.config, "cf_prefill_mfma")},
    }


def bench_block_tables(args) -> dict:
    """Per-step block-table upkeep for B decoding requests (default 256):
    rebuilding and uploading the [B, Mb] tables every step, as a dict-based
    caller does, against the block pool's incremental device tables; plus
    copy-on-write block copies over Llama-3-8B-shaped FP8 slabs."""
    import random

    import numpy as np
    import torch

    from cf_hip import ops
    from compiler.cache_policy import CachePolicy
    from python_runtime.engine import CacheManager
    from python_runtime.engine.block_manager import BlockManager, RequestBatch

    dev = torch.device("cuda:0")
    B = args.batch or 256
    bs = 16
    rng = random.Random(0)
    lens = [rng.randint(1024, 8192) for _ in range(B)]
    grow = 2 * (args.steps + args.warmup) + 20 + bs  # tokens appended over both timed paths and the scatter timing
    cols = -(-(max(lens) + grow) // bs)
    nb = sum(-(-(n + grow) // bs) for n in lens) + 64
    bm = BlockManager(nb, bs)
    ids = [f"req{i}" for i in range(B)]
    # half the requests share a 1024-token prefix, as a radix hit gives them
    bm.allocate(ids[0], lens[0])
    for i in range(1, B):
        if i < B // 2:
            bm.share_prefix(ids[0], ids[i], 1024)
            bm.ensure_blocks(ids[i], lens[i])
        else:
            bm.allocate(ids[i], lens[i])
    for rid, n in zip(ids, lens):
        bm.set_len(rid, n)
    bm.bind_device(B, cols, dev)
    bm.sync_device()
    host_tables = {rid: bm.get_blocks(rid) for rid in ids}
    batch = RequestBatch(ids)
    cur = np.asarray(lens, dtype=np.int64)
    one = np.ones(B, dtype=np.int64)

    def step_rebuild():
        # a dict-based caller: host tables -> padded int32 [B, Mb] + lengths, uploaded whole
        slots, _ = bm.prepare_writes_batch(batch, cur, one)
        cur[:] += 1
        for i in np.nonzero((cur - 1) % bs == 0)[0]:
            host_tables[ids[i]] = bm.get_blocks(ids[i])
        mat = np.full((B, cols), -1, np.int32)
        for i, rid in enumerate(ids):
            t = host_tables[rid]
            mat[i, : len(t)] = t
        tables = torch.from_numpy(mat).to(dev)
        lens_t = torch.from_numpy(cur.astype(np.int32)).to(dev)
        slots_t = torch.from_numpy(slots).to(dev)
        return tables, lens_t, slots_t

    def step_deltas():
        # the block pool: only the changed cells and lengths go to the device
        slots, _ = bm.prepare_writes_batch(batch, cur, one)
        cur[:] += 1
        tables, lens_t = bm.sync_device()
        return tables, lens_t, torch.from_numpy(slots).to(dev, non_blocking=True)

    res = {}
    for name, fn in (("rebuild", step_rebuild), ("deltas", step_deltas)):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        res[name] = (time.perf_counter() - t0) * 1e6 / args.steps
    t, l_ = bm.sync_device()
    tcpu, lcpu = t.cpu().numpy(), l_.cpu().numpy()
    for i, rid in enumerate(ids):
        r = bm.row_of(rid)
        blocks = bm.get_blocks(rid)
        assert lcpu[r] == cur[i] and (tcpu[r, : len(blocks)] == blocks).all() and (tcpu[r, len(blocks):] == -1).all(), \
            "device tables diverged"
    log(f"B={B}: rebuild {res['rebuild']:.1f} us/step, deltas {res['deltas']:.1f} us/step")

    # copy-on-write copies over Llama-3-8B-shaped FP8 slabs (32 layers, 8 KV heads, D 128)
    mgr = CacheManager(CachePolicy.for_llama(32, 8, 128, kv_dtype="float8_e4m3fn"), num_blocks=2048, device=dev)
    pairs = np.stack([np.arange(0, 512), np.arange(1024, 1536)], axis=1).astype(np.int32)
    block_bytes = sum(s[0].numel() * s.element_size() for s in mgr.paged_slabs())  # K + V of one block
    for _ in range(3):
        BlockManager.copy_blocks(pairs, mgr.paged_slabs())
    torch.cuda.synchronize()
    ops.KernelTimer.reserve(2 * 20 + 2 * 20 + 16)
    with ops.KernelTimer() as timer:
        for _ in range(10):
            BlockManager.copy_blocks(pairs, mgr.paged_slabs())
        torch.cuda.synchronize()
    ms, n = timer.query("cf_copy_blocks")
    apply_ms, apply_n = 0.0, 0
    with ops.KernelTimer() as timer2:
        for _ in range(20):
            step_deltas()
        torch.cuda.synchronize()
    apply_ms, apply_n = timer2.query("cf_block_tables_apply")
    copy_s = ms / 10 / 1e3  # one copy_blocks call = K and V slabs
    moved = 2 * len(pairs) * block_bytes  # read + write
    gbs = moved / copy_s / 1e9
    log(f"COW copy of {len(pairs)} blocks ({block_bytes / 2**20:.2f} MiB each, K+V, 32 layers): "
        f"{copy_s * 1e6:.1f} us, {gbs:.0f} GB/s; table scatter {apply_ms / max(apply_n, 1) * 1e3:.1f} us")
    return {
        "metric": "block-table upkeep per decode step (host + upload), B requests, 1 MI355X",
        "value": res["deltas"],
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["deltas"] / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32 tables",
        "data": "synthetic (seeded)",
        "config": {"workload": "block_tables", "requests": B, "block_size": bs, "ctx": "U{1024..8192}",
                   "shared_prefix": "requests 0..B/2-1 share 1024 tokens", "table_cols": cols,
                   "parallelism": "single GPU"},
        "rebuild_us_per_step": res["rebuild"],
        "deltas_us_per_step": res["deltas"],
        "table_scatter_us": apply_ms / max(apply_n, 1) * 1e3,
        "roofline": {"bound": "hbm", "kernel": "cf_copy_blocks", "achieved": gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                     "work": f"{len(pairs)} block copies of {block_bytes} B (read + write)"},
    }


def bench_fp8(args) -> dict:
    """FP8 quantization kernels at the c3 pool size: per-KV-head amax ->
    scale (reads the bf16 pool), quantize into the paired layout (K tiles
    token-major, V tiles channel-major), each over K and V; plus the c5
    step's paged FP8 write of 4344 new rows.  Durations from launch-stamped
    HIP events; GB/s = algorithmic bytes (elements read + codes written)
    / duration."""
    import torch

    from cf_hip import layout as L
    from cf_hip import ops, workloads

    dev = torch.device("cuda:0")
    case = workloads.make_case("c3_llama3_8b", device=dev, seed=0)
    nb, bs, hkv, d = case.k.shape
    n = case.k.numel()
    kc, vc = L.alloc_kv_cache(nb, bs, hkv, d, torch.float8_e4m3fn, dev, "paired")
    ks = torch.empty(hkv, dtype=torch.float32, device=dev)
    vs = torch.empty(hkv, dtype=torch.float32, device=dev)
    mixed = workloads.make_mixed_case("c5_mixed", device=dev, seed=0)
    t = workloads.materialize_mixed(mixed, "paired")

    def step():
        ops.fp8_amax_scale(case.k, out=ks)
        ops.fp8_amax_scale(case.v, out=vs)
        ops.fp8_quantize_kv(case.k, case.v, ks, vs, kc, vc)
        ops.fp8_quantize(case.k, ks, out=kc)
        ops.fp8_quantize(case.v, vs, out=vc)
        ops.kv_write_fp8(t["k_new"], t["v_new"], t["slots"], t["k_cache"], t["v_cache"], t["k_scale"], t["v_scale"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer = ops.KernelTimer()
    timer.reserve(2 * 6 * (args.steps + 1) + 16)
    with timer:
        step()
        torch.cuda.synchronize()
        timer.reset()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    res = {}
    src_bytes = n * case.k.element_size()
    rows_new = t["k_new"].shape[0] * t["k_new"].shape[1] * t["k_new"].shape[2]
    work = {
        "cf_fp8_amax": ("amax -> scale over a bf16 [NB, 16, 8, 128] pool (K or V)", src_bytes, 2),
        "cf_kv_quantize_fp8": ("quantize the K and V bf16 pools into the paired e4m3 layout, one launch",
                               2 * (src_bytes + n), 1),
        "cf_fp8_quantize": ("quantize one bf16 pool into the paired e4m3 layout (K or V alone)", src_bytes + n, 2),
        "cf_kv_write_fp8": ("paged FP8 write of the c5 step's new K and V rows",
                            2 * rows_new * t["k_new"].element_size() + 2 * rows_new, 1),
    }
    for name, (what, nbytes, per_step) in work.items():
        ms, cnt = timer.query(name)
        assert cnt == per_step * args.steps, (name, cnt)
        us = ms / cnt * 1e3
        res[name] = {"what": what, "us": us, "bytes": nbytes, "gbs": nbytes / (us / 1e6) / 1e9,
                     "frac": nbytes / (us / 1e6) / 1e9 / HBM_PEAK_GBS}
        log(f"{name}: {us:.1f} us, {res[name]['gbs']:.0f} GB/s ({res[name]['frac'] * 100:.1f} % of 8 TB/s)")
    timer.reset()
    q = res["cf_kv_quantize_fp8"]
    return {
        "metric": "FP8 KV quantize GB/s (% of HBM peak), Llama-3-8B-shaped K and V pools, 1 MI355X",
        "value": q["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 -> e4m3", "data": "synthetic (seeded)",
        "config": {"workload": "fp8_quantize", "pool": [nb, bs, hkv, d], "kv_layout": "paired",
                   "write_rows": int(t["k_new"].shape[0]), "parallelism": "single GPU"},
        "kernels": res,
        "roofline": {"bound": "hbm", "kernel": "cf_kv_quantize_fp8", "achieved": q["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": q["frac"], "traffic": None},
    }


def bench_copy(args) -> dict:
    """A plain device copy of 1 GiB (torch's copy kernel), K times: the
    known-size reference the FETCH_SIZE / WRITE_SIZE counters are scaled by
    (each launch reads and writes exactly 2^30 bytes)."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    gbs = 2 * n / (ms / 1e3) / 1e9
    log(f"copy 1 GiB: {ms * 1e3:.1f} us, {gbs:.0f} GB/s read + write")
    return {
        "metric": "device copy of 1 GiB (read + write GB/s), 1 MI355X",
        "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic", "config": {"workload": "copy_1gib", "bytes_read": n, "bytes_written": n,
                                        "parallelism": "single GPU"},
    }


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c3_llama3_8b")
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--partition", type=int, default=512)
    ap.add_argument("--layout", default="paired")
    ap.add_argument("--q-dtype", choices=["bf16", "float16", "float32"], default=None,
                    help="cast the decode queries (fp16 takes the MFMA kernel's fp16 operands, fp32 the generic "
                         "kernel); the line then names its own metric")
    ap.add_argument("--pools", type=int, default=2, help="cache copies rotated between steps")
    ap.add_argument("--cpu-sample", type=int, default=8)
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-settle", action="store_true",
                    help="skip the untimed steps that bring the GPU to a steady step time before the warm-up")
    ap.add_argument("--one-stream", action="store_true",
                    help="c5_mixed: decode and prefill one after another only (per-kernel profiles)")
    ap.add_argument("--no-shared-prefix", action="store_true",
                    help="do not pass the shared-prefix statement (every sequence reads its whole table)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the decode kernel shards per sequence / KV head with no exchange).", file=sys.stderr)
        sys.exit(2)

    import torch

    from cf_hip import ops, workloads

    dev = torch.device("cuda:0")
    log(f"device {torch.cuda.get_device_name(dev)}; building {args.config}")
    if args.config == "c5_mixed":
        result = bench_mixed(args)
        print(json.dumps(result), flush=True)
        return
    if args.config == "block_tables":
        result = bench_block_tables(args)
        print(json.dumps(result), flush=True)
        return
    if args.config == "fp8_quantize":
        result = bench_fp8(args)
        print(json.dumps(result), flush=True)
        return
    if args.config == "copy_1gib":
        result = bench_copy(args)
        print(json.dumps(result), flush=True)
        return
    case = workloads.make_case(args.config, device=dev, seed=0, batch=args.batch)
    if args.q_dtype is not None:
        case.q = case.q.to({"bf16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}[args.q_dtype])
    pools = []
    for i in range(args.pools):
        pools.append(workloads.materialize(case, args.layout))
    tables = case.tables_tensor(dev)
    lens = case.seq_lens_tensor(dev)
    # The radix cache's statement of shared prefix blocks (what a serving
    # loop passes along with the tables): the LCP of neighbouring tables.
    shared = None
    if not args.no_shared_prefix:
        shared = torch.tensor(ops.shared_prefix_lens(case.block_tables, case.seq_lens, case.block_size),
                              dtype=torch.int32, device=dev)
    plans = [
        ops.DecodePlan(case.q, kc, vc, tables, lens, case.scale, case.block_size, ks, vs, args.partition,
                       shared_prefix_lens=shared)
        for kc, vc, ks, vs in pools
    ]
    ab = workloads.algorithmic_bytes(case)
    torch.cuda.synchronize()
    log(f"batch {case.batch}, {ab['tokens']} context tokens, unique bytes {ab['unique'] / 1e6:.1f} MB")

    settled = None
    if not args.no_settle:
        settled = settle(lambda i: plans[i % len(plans)].run(), batch=20, min_steps=240, max_steps=800)
        log(f"settle: {settled['steps']} steps, us/step by batch {settled['us_per_step_by_batch']}")
    for i in range(args.warmup):
        plans[i % len(plans)].run()
    torch.cuda.synchronize()
    log("warmup done")

    # Timed region: K steps, nothing else on the stream, bracketed by device
    # synchronizations.  The step time is the GPU interval between two HIP
    # events recorded on the launch stream around the K steps; the host's
    # wall clock over the same region (which adds the first launch's
    # submission latency and the final synchronization's wake-up, ~2 us per
    # step at K = 20) is reported beside it.
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        plans[i % len(plans)].run()
    ev1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    ms_step_wall = (t1 - t0) * 1e3 / args.steps

    # Kernel durations: the same K steps again with the library's timing hook
    # on.  Each launch then carries two HIP events that hipExtLaunchKernel
    # records at the kernel's start and end on the launch stream.  Stamping
    # adds host work and a completion signal per launch, so this pass runs
    # slower than the timed one above and is not a step timing.  Every event
    # the pass needs is created before it (cf_profile_reserve) and the pass
    # is preceded by K stamped steps: an event created inside the pass costs
    # host time, the GPU then idles between launches, and kernels that start
    # after an idle gap read several us longer.  The decode kernel's figure
    # is the median of its K launches.
    timer = ops.KernelTimer()
    timer.reserve(8 * args.steps + 16)
    with timer:
        for i in range(args.steps):
            plans[i % len(plans)].run()
        torch.cuda.synchronize()
        timer.reset()
        t0 = time.perf_counter()
        for i in range(args.steps):
            plans[i % len(plans)].run()
        torch.cuda.synchronize()
        ms_step_stamped = (time.perf_counter() - t0) * 1e3 / args.steps
    kernel_name = "cf_decode_mfma"
    dec_ms = timer.durations(kernel_name)
    if not dec_ms:
        kernel_name = "cf_decode_generic"
        dec_ms = timer.durations(kernel_name)
    red_ms = timer.durations("cf_decode_merge") + timer.durations("cf_decode_reduce")
    timer.reset()
    if len(dec_ms) != args.steps:
        log(f"warning: expected {args.steps} {kernel_name} launches, timed {len(dec_ms)}")

    def median(xs: list[float]) -> float:
        ys = sorted(xs)
        if not ys:
            return float("nan")
        m = len(ys) // 2
        return ys[m] if len(ys) % 2 else 0.5 * (ys[m - 1] + ys[m])

    dec_med_ms = median(dec_ms)
    red_med_ms = median(red_ms) if red_ms else 0.0
    log(f"{ms_step * 1e3:.1f} us/step (HIP events; wall clock {ms_step_wall * 1e3:.1f}; "
        f"{ms_step_stamped * 1e3:.1f} with stamped launches); decode kernel "
        f"median {dec_med_ms * 1e3:.1f} us (mean {sum(dec_ms) / max(len(dec_ms), 1) * 1e3:.1f}, "
        f"{len(dec_ms)} launches), merge median {red_med_ms * 1e3:.1f} us")
    # One kernel of a step cannot outlast the step.  Should the stamped
    # median read longer anyway (a profiler intercepting the launches, a
    # throttled part), the line records it and bases the kernel fraction on
    # the step instead of failing.
    kernel_within_step = bool(dec_med_ms <= ms_step)
    if not kernel_within_step:
        log(f"note: the stamped {kernel_name} median ({dec_med_ms * 1e3:.1f} us) reads longer than the step "
            f"({ms_step * 1e3:.1f} us); roofline.frac uses the step")

    kernel_s = (dec_med_ms if kernel_within_step else ms_step) / 1e3
    achieved = ab["unique"] / kernel_s / 1e9
    traffic = load_traffic(args.config)

    # The reference's dict signature (request id -> block list / length) on
    # the same batch, kept out of the timed region: per call, the host work
    # (table packing, validation, shared-prefix statement, staging) and the
    # whole call with the GPU work.
    from kernels.paged_attention import paged_attention

    dict_tables = {f"req{b:04d}": list(t) for b, t in enumerate(case.block_tables)}
    dict_lens = {f"req{b:04d}": int(n) for b, n in enumerate(case.seq_lens)}
    kc0, vc0, ks0, vs0 = pools[0]
    for _ in range(3):
        paged_attention(case.q, kc0, vc0, dict_tables, dict_lens, case.block_size, case.scale, k_scale=ks0,
                        v_scale=vs0)
    torch.cuda.synchronize()
    n_dict = 20
    # back to back: the calls' throughput (GPU-bound when the host keeps up)
    t0 = time.perf_counter()
    for i in range(n_dict):
        kc_i, vc_i, ks_i, vs_i = pools[i % len(pools)]
        paged_attention(case.q, kc_i, vc_i, dict_tables, dict_lens, case.block_size, case.scale, k_scale=ks_i,
                        v_scale=vs_i)
    torch.cuda.synchronize()
    dict_us = (time.perf_counter() - t0) * 1e6 / n_dict
    # host cost: each call timed from an idle GPU to its return, so no wait
    # on queued GPU work is counted
    host_s = 0.0
    for i in range(n_dict):
        kc_i, vc_i, ks_i, vs_i = pools[i % len(pools)]
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        paged_attention(case.q, kc_i, vc_i, dict_tables, dict_lens, case.block_size, case.scale, k_scale=ks_i,
                        v_scale=vs_i)
        host_s += time.perf_counter() - h0
    torch.cuda.synchronize()
    log(f"dict API: {dict_us:.1f} us/call back to back, host {host_s * 1e6 / n_dict:.1f} us/call")

    short = {torch.float8_e4m3fn: ("FP8", "e4m3"), torch.bfloat16: ("BF16", "bf16"), torch.float16: ("FP16", "f16"),
             torch.float32: ("FP32", "f32")}
    kv_name, kv_short = short[case.kv_dtype]
    q_short = short[case.q.dtype][1]
    result = {
        # BASELINE.json's metric for its config (c3); other configs name theirs
        "metric": METRIC if args.config == "c3_llama3_8b" and args.q_dtype is None else
        f"paged-decode tokens/s + HBM GB/s (% peak), {args.config} {kv_name} KV"
        + (f" / {q_short} q" if args.q_dtype is not None else "") + ", 1 MI355X",
        "value": case.batch / (ms_step / 1e3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{kv_short} KV / {q_short} q / f32 accumulate",
        "data": "synthetic (seeded), random-init",
        "config": {
            "workload": args.config,
            "batch": case.batch,
            "num_q_heads": case.q.shape[1],
            "num_kv_heads": case.num_kv_heads,
            "head_dim": case.head_dim,
            "block_size": case.block_size,
            "context_tokens": ab["tokens"],
            # the MFMA kernel balances 32-token tiles over all waves (no
            # fixed partitions); the generic kernel splits into partitions
            "split_kv": ("32-token tiles balanced over all waves + merge" if kernel_name == "cf_decode_mfma"
                         else f"{args.partition}-token partitions + log-sum-exp reduce"),
            "kv_layout": args.layout,
            "cache_pools_rotated": args.pools,
            "shared_prefix_statement": shared is not None,
            "parallelism": "single GPU",
        },
        "settle": settled,
        "ms_per_step_wall_clock": ms_step_wall,
        "ms_per_step_stamped_launches": ms_step_stamped,
        "step_timing": "ms_per_step = HIP events on the launch stream around the K steps (GPU interval); "
                       "ms_per_step_wall_clock = host clock over the same synchronized region",
        "hbm_gbs_step": ab["unique"] / (ms_step / 1e3) / 1e9,
        "hbm_frac_step": ab["unique"] / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS,
        "kernel_us": {"decode": dec_med_ms * 1e3, "merge": red_med_ms * 1e3, "decode_kernel": kernel_name,
                      "decode_mean": sum(dec_ms) / max(len(dec_ms), 1) * 1e3,
                      "decode_min": min(dec_ms, default=float("nan")) * 1e3,
                      "decode_max": max(dec_ms, default=float("nan")) * 1e3, "launches": len(dec_ms),
                      "statistic": "median of K launch-stamped launches (events created before the pass)"},
        "kernel_within_step": kernel_within_step,
        "algorithmic_bytes": {"unique": ab["unique"], "logical": ab["logical"]},
        "dict_api": {"us_per_call": dict_us, "host_us_per_call": host_s * 1e6 / n_dict,
                     "note": "kernels.paged_attention.paged_attention (request-id dicts) on the same batch: "
                             "us_per_call over 20 calls back to back; host_us_per_call = one call's host time "
                             "from an idle GPU (table packing, staging, descriptors, launches, the output dict)"},
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "frac_step": ab["unique"] / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBS,
            "traffic": traffic,
            "work": "algorithmic unique bytes per launch (KV rows of every sequence, shared rows once, + q + out "
                    "+ tables + lengths + scales) / the kernel's median duration over K launch-stamped launches "
                    "(the step time instead when that median exceeds the step: see kernel_within_step); "
                    "frac_step uses the timed step",
        },
    }
    if not args.no_cpu_baseline:
        kc, vc, ks, vs = pools[0]
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(case, kc, vc, ks, vs, min(args.cpu_sample, case.batch),
                                              args.cpu_budget)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
