"""GPU parity of the paged decode kernels against the CPU oracle.

Tolerances: fp32 max-abs 1e-5; bf16 and fp8
max-abs 2e-2 with cosine >= 0.9999.  Small and mid sizes compare with the
float64 oracle directly; full benchmark sizes use size-independent
properties (block-permutation invariance, shared prefix == copied prefix,
rerun and grouped/ungrouped agreement) plus an oracle check on a sample of
sequences that includes the longest one.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import layout as L
from cf_hip import ops, workloads
from kernels.paged_attention import paged_attention, paged_attention_tensors
from tests.gpu_util import assert_close, oracle_decode

pytestmark = pytest.mark.gpu


def _run(case, kc, vc, ks, vs, dev, pt=512, tables=None, lens=None):
    t = tables if tables is not None else case.tables_tensor(dev)
    s = lens if lens is not None else case.seq_lens_tensor(dev)
    out = paged_attention_tensors(case.q, kc, vc, t, s, case.block_size, case.scale, k_scale=ks, v_scale=vs,
                                  partition_tokens=pt)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("layout", ["paired", "native", "token_major"])
@pytest.mark.parametrize("config,batch", [("c1_opt125m", None), ("c2_tinyllama", None), ("c3_llama3_8b", 6),
                                          ("c4_llama3_70b", 3)])
def test_configs_match_oracle(gpu, config, batch, layout):
    print(f"[case] {config} batch={batch} layout={layout}", flush=True)
    case = workloads.make_case(config, device=gpu, seed=21, batch=batch)
    kc, vc, ks, vs = workloads.materialize(case, layout)
    out = _run(case, kc, vc, ks, vs, gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, case.q.dtype, f"{config}/{layout}")


@pytest.mark.parametrize("pt", [16, 48, 64, 256])
def test_partition_sizes_agree(gpu, pt):
    """Split-KV partition sizes on the generic (partitioned) path: fp32
    caches only run there, so every size really changes the split (at the
    full c2 batch the launch holds >= 1024 workgroups from 256-token
    partitions down, so none of these is shortened), and the log-sum-exp
    reduce runs."""
    print(f"[case] c2 shape, fp32 caches, partitions={pt}", flush=True)
    case = workloads.make_case("c2_tinyllama", device=gpu, seed=3)
    case.q = case.q.float()
    case.kv_dtype = torch.float32
    kc, vc, ks, vs = workloads.materialize(case, "native")
    with ops.KernelTimer() as timer:
        out = _run(case, kc, vc, ks, vs, gpu, pt=pt)
        assert timer.query("cf_decode_generic")[1] == 1 and timer.query("cf_decode_mfma")[1] == 0
        assert timer.query("cf_decode_reduce")[1] == 1
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.float32, f"pt={pt}")


@pytest.mark.parametrize("hq,hkv,d,bs", [(8, 8, 64, 16), (8, 2, 128, 16), (16, 1, 64, 16), (32, 2, 128, 16),
                                         (4, 4, 32, 8), (8, 2, 64, 32), (6, 3, 80, 16), (8, 4, 256, 16)])
@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn])
def test_shapes_and_dtypes(gpu, hq, hkv, d, bs, kv_dtype):
    print(f"[case] hq={hq} hkv={hkv} d={d} bs={bs} kv={kv_dtype}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(hq * 1000 + d + bs)
    b, nb = 5, 64
    lens = [1, bs, bs + 1, 7 * bs - 3, 700]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).tolist()
    tables, pos = [], 0
    for n in lens:
        k = (n + bs - 1) // bs
        tables.append(perm[pos:pos + k])
        pos += k
    q_dtype = kv_dtype if kv_dtype in (torch.float32, torch.float16) else torch.bfloat16
    q = torch.randn(b, hq, d, generator=g, device=gpu).to(q_dtype)
    ksrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu).to(q_dtype)
    vsrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu).to(q_dtype)
    case = workloads.DecodeCase("adhoc", q, ksrc, vsrc, tables, lens, bs, 1 / math.sqrt(d), kv_dtype)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _run(case, kc, vc, ks, vs, gpu, pt=4 * bs)
    assert out.dtype == q_dtype
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, q_dtype, f"{hq}/{hkv}/{d}/{bs}/{kv_dtype}")


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 2, 64)])
def test_fp16_queries_take_the_mfma_path(gpu, hq, hkv, d, kv_dtype):
    """fp16 queries over fp16 or e4m3 caches (block size 16, native layout)
    run the MFMA kernel (fp16 operands) and match the float64 oracle; the
    shared-prefix statement is exercised too."""
    print(f"[case] fp16 q hq={hq} hkv={hkv} d={d} kv={kv_dtype}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(hq + d)
    lens = [700, 1024, 1024 + 33, 40, 2000, 1]
    nb = 600
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(9)).tolist()
    shared = perm[:64]  # sequences 1 and 2 share a 1024-token prefix
    tables, pos = [], 64
    for i, n in enumerate(lens):
        k = (n + 15) // 16
        if i in (1, 2):
            own = perm[pos:pos + k - 64]
            pos += k - 64
            tables.append(shared + own)
        else:
            tables.append(perm[pos:pos + k])
            pos += k
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu).to(torch.float16)
    ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.float16)
    vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.float16)
    case = workloads.DecodeCase("fp16", q, ksrc, vsrc, tables, lens, 16, 1 / math.sqrt(d), kv_dtype)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    sh = torch.tensor(ops.shared_prefix_lens(tables, lens, 16), dtype=torch.int32, device=gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    with ops.KernelTimer() as timer:
        out = paged_attention_tensors(q, kc, vc, case.tables_tensor(gpu), case.seq_lens_tensor(gpu), 16, case.scale,
                                      k_scale=ks, v_scale=vs, shared_prefix_lens=sh)
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 1 and timer.query("cf_decode_generic")[1] == 0
    assert out.dtype == torch.float16
    assert_close(out.float().cpu().numpy(), ref, torch.float16, f"fp16 q / {kv_dtype}")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("hq,hkv,d,layout", [(32, 8, 128, "paired"), (16, 2, 64, "native"),
                                             (8, 8, 64, "token_major"), (32, 8, 128, "token_major")])
def test_fp32_queries_take_the_mfma_path(gpu, hq, hkv, d, layout, kv_dtype):
    """fp32 queries over bf16 or e4m3 caches run the MFMA kernel: each query
    channel split exactly into three bf16 terms, P carried as two fp16 (e4m3
    V) or three bf16 (bf16 V) terms.  fp32 output within the fp32 bound
    (max-abs 1e-5) of the float64 oracle, with the shared-prefix statement
    and a sequence long enough to be split over several waves."""
    print(f"[case] fp32 q hq={hq} hkv={hkv} d={d} kv={kv_dtype} layout={layout}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(7 * hq + d)
    lens = [700, 1024, 1024 + 33, 40, 6000, 1, 0, 300]
    nb = 1000
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(4)).tolist()
    shared = perm[:64]  # sequences 1 and 2 share a 1024-token prefix
    tables, pos = [], 64
    for i, n in enumerate(lens):
        k = max(1, (n + 15) // 16)
        if i in (1, 2):
            own = perm[pos:pos + k - 64]
            pos += k - 64
            tables.append(shared + own)
        else:
            tables.append(perm[pos:pos + k])
            pos += k
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu) * 2.0
    ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    case = workloads.DecodeCase("fp32q", q, ksrc, vsrc, tables, lens, 16, 1 / math.sqrt(d), kv_dtype)
    kc, vc, ks, vs = workloads.materialize(case, layout)
    sh = torch.tensor(ops.shared_prefix_lens(tables, lens, 16), dtype=torch.int32, device=gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    with ops.KernelTimer() as timer:
        out = paged_attention_tensors(q, kc, vc, case.tables_tensor(gpu), case.seq_lens_tensor(gpu), 16, case.scale,
                                      k_scale=ks, v_scale=vs, shared_prefix_lens=sh)
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 1 and timer.query("cf_decode_generic")[1] == 0
    assert out.dtype == torch.float32
    assert_close(out.cpu().numpy(), ref, torch.float32, f"fp32 q / {kv_dtype} / {layout}")


def test_fp32_queries_c3_batch(gpu):
    """The c3 workload (e4m3 with 1 % x8 outliers, per-head scales, shared
    prefix) at batch 8 with fp32 queries: MFMA path, fp32 bound."""
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=12, batch=8)
    case.q = case.q.float()
    kc, vc, ks, vs = workloads.materialize(case, "paired")
    sh = torch.tensor(ops.shared_prefix_lens(case.block_tables, case.seq_lens, 16), dtype=torch.int32, device=gpu)
    out = paged_attention_tensors(case.q, kc, vc, case.tables_tensor(gpu), case.seq_lens_tensor(gpu), 16, case.scale,
                                  k_scale=ks, v_scale=vs, shared_prefix_lens=sh)
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), oracle_decode(case, kc, vc, ks, vs), torch.float32, "c3 fp32 q")


def test_edge_lengths(gpu):
    """Zero length -> zeros; length past the table -> truncated to it."""
    case = workloads.make_case("c2_tinyllama", device=gpu, seed=4, batch=4)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    tables = case.tables_tensor(gpu)
    cap = tables.shape[1] * 16
    lens = torch.tensor([0, 10**6, 1, 17], dtype=torch.int32, device=gpu)
    out = _run(case, kc, vc, ks, vs, gpu, tables=tables, lens=lens).float().cpu().numpy()
    assert np.all(out[0] == 0)
    eff = [0, cap, 1, 17]
    ref = oracle_decode(case, kc, vc, ks, vs, tables=tables.cpu().tolist(), lens=eff)
    assert_close(out[1:], ref[1:], case.q.dtype, "edge lengths")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cache_without_blocks(gpu, dtype):
    """A cache of zero blocks (its data pointer may be NULL): every table
    entry is outside the pool, so every output is zero and the cache is
    never read."""
    print(f"[case] empty cache {dtype}", flush=True)
    q = torch.randn(2, 4, 64, device=gpu).to(dtype)
    kc = torch.empty(0, 16, 2, 64, dtype=dtype, device=gpu)
    vc = torch.empty(0, 16, 2, 64, dtype=dtype, device=gpu)
    tables = torch.tensor([[0, 1], [5, 2]], dtype=torch.int32, device=gpu)
    lens = torch.tensor([20, 3], dtype=torch.int32, device=gpu)
    out = paged_attention_tensors(q, kc, vc, tables, lens, 16, 0.125)
    torch.cuda.synchronize()
    assert out.shape == q.shape and torch.count_nonzero(out).item() == 0


def test_dict_api_matches_tensor_api_and_reference_rules(gpu):
    case = workloads.make_case("c2_tinyllama", device=gpu, seed=5, batch=6)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    rids = [f"r{i}" for i in range(case.batch)]
    bt = dict(zip(rids, case.block_tables))
    sl = {r: n for r, n in zip(rids, case.seq_lens) if r != "r2"}  # r2: whole table
    sl["r3"] = 10**6  # beyond capacity: truncated
    out = paged_attention(case.q, kc, vc, bt, sl, block_size=16)
    assert list(out) == rids
    lens = [len(t) * 16 if i in (2, 3) else n for i, (t, n) in enumerate(zip(case.block_tables, case.seq_lens))]
    ref = oracle_decode(case, kc, vc, ks, vs, lens=lens)
    got = torch.stack([out[r] for r in rids]).float().cpu().numpy()
    assert_close(got, ref, case.q.dtype, "dict api")
    with pytest.raises(RuntimeError):
        paged_attention(case.q, kc, vc, {"x": [0]}, {"x": 0})
    with pytest.raises(IndexError):
        paged_attention(case.q, kc, vc, {"x": [kc.shape[0]]}, {"x": 3})


def test_dict_api_back_to_back_calls(gpu):
    """Dict-API calls issued back to back (uploads on the side stream, ring
    slots reused while earlier kernels are still queued, one call that grows
    a slot) give bitwise the results of the same calls made one at a time."""
    import random

    case = workloads.make_case("c2_tinyllama", device=gpu, seed=8, batch=8)
    kc, vc, ks, vs = workloads.materialize(case)
    nb = kc.shape[0]
    rng = random.Random(3)
    calls = []
    for i in range(8):
        sel = rng.sample(range(case.batch), k=rng.randint(1, case.batch))
        bt = {f"r{b}": list(case.block_tables[b]) for b in sel}
        sl = {f"r{b}": case.seq_lens[b] for b in sel}
        if i == 4:  # a 70,000-entry table: more than a slot holds, so the slot grows
            r0 = next(iter(bt))
            bt[r0] = bt[r0] + [rng.randrange(nb) for _ in range(70000)]
        calls.append((case.q[sel].contiguous(), bt, sl))
    print("[case] dict API back to back, 8 calls", flush=True)
    torch.cuda.synchronize()
    outs = [paged_attention(q, kc, vc, bt, sl, block_size=16) for q, bt, sl in calls]
    torch.cuda.synchronize()
    for (q, bt, sl), out in zip(calls, outs):
        ref = paged_attention(q, kc, vc, bt, sl, block_size=16)
        torch.cuda.synchronize()
        assert list(out) == list(bt)
        for r in bt:
            assert torch.equal(out[r], ref[r]), r


def test_full_c3_properties(gpu):
    """Full headline config, native layout, no shared-prefix statement:
    block-permutation invariance (bitwise), shared prefix == copied prefix
    (bitwise), and the oracle on a sample of sequences."""
    print("[case] c3 full size", flush=True)
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=0)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _run(case, kc, vc, ks, vs, gpu)
    # 1. permutation of physical block ids
    nb = kc.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(2)).to(gpu)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb, device=gpu)
    kc2, vc2 = L.alloc_kv_cache(nb, 16, 8, 128, torch.float8_e4m3fn, gpu)
    kc2.copy_(kc[perm])
    vc2.copy_(vc[perm])
    t2 = inv[case.tables_tensor(gpu).long()].to(torch.int32)
    out2 = _run(case, kc2, vc2, ks, vs, gpu, tables=t2)
    assert torch.equal(out, out2)
    del kc2, vc2
    # 2. copied prefix
    pre = case.meta["shared_prefix_blocks"]
    tables = case.tables_tensor(gpu)
    shared = tables[0, :pre].long()
    kc3, vc3 = L.alloc_kv_cache(nb + pre, 16, 8, 128, torch.float8_e4m3fn, gpu)
    kc3[:nb].copy_(kc)
    vc3[:nb].copy_(vc)
    kc3[nb:].copy_(kc[shared])
    vc3[nb:].copy_(vc[shared])
    t3 = tables.clone()
    t3[1, :pre] = torch.arange(nb, nb + pre, device=gpu, dtype=torch.int32)
    out3 = _run(case, kc3, vc3, ks, vs, gpu, tables=t3)
    assert torch.equal(out, out3)
    del kc3, vc3
    # 3. oracle on a sample of sequences (shared and private)
    idx = [0, 1, 31, 32, 63]
    sub = workloads.DecodeCase("c3_sample", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], 16, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kc, vc, ks, vs)
    assert_close(out[idx].float().cpu().numpy(), ref, torch.bfloat16, "c3 sample")


def test_hal_backend_paged_attention(gpu):
    from python_runtime.hal import registry
    from python_runtime.hal.hip_backend import HipBackend, register_hip_backend

    register_hip_backend()
    be = registry.create("hip")
    assert isinstance(be, HipBackend)
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=9, batch=3)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = be.execute("paged_attention", [case.q, kc, vc, case.tables_tensor(gpu), case.seq_lens_tensor(gpu)],
                     k_scale=ks, v_scale=vs, scale=case.scale)
    torch.cuda.synchronize()
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "hal")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("n,hq,hkv,d", [(30000, 32, 8, 128), (40000, 32, 2, 128), (20000, 4, 4, 64),
                                        (25000, 16, 2, 64), (3000, 8, 1, 64)])
def test_long_single_sequence_split_over_many_waves(gpu, kv_dtype, n, hq, hkv, d):
    """One long sequence: every KV head's run is split over hundreds of
    waves, so the merge combines more than its register path holds -- up to
    ~1,000 partials per head (several 256-partial chunks) with one KV head
    or two, G from 1 to 16 (one to two 16-byte output slices per thread)."""
    print(f"[case] long single sequence kv={kv_dtype} n={n} hq={hq} hkv={hkv} d={d}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(12)
    nb = (n + 15) // 16 + 3
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).tolist()
    q = torch.randn(1, hq, d, generator=g, device=gpu).to(torch.bfloat16)
    ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    case = workloads.DecodeCase("long", q, ksrc, vsrc, [perm[: (n + 15) // 16]], [n], 16, 1 / math.sqrt(d), kv_dtype)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _run(case, kc, vc, ks, vs, gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "long sequence")


@pytest.mark.parametrize("hq,hkv,d", [(32, 4, 64), (32, 8, 128), (64, 8, 128), (16, 1, 64)])
def test_merge_partial_counts(gpu, hq, hkv, d):
    """One sequence of t tiles per KV head splits into about t partials per
    head, so the lengths sweep the merge across its two paths: one partial,
    the most its one-wave register path holds (64 / (G * D / 64)), and past
    that (the chunked LDS path) up to four and more times as many."""
    g_ = hq // hkv
    kmax = 64 // (g_ * d // 64)
    for tiles in sorted({1, kmax, kmax + 1, 2 * kmax + 1, 4 * kmax, 4 * kmax + 1, 4 * kmax + 3}):
        n = 32 * tiles - 5
        print(f"[case] merge partials hq={hq} hkv={hkv} d={d} tiles={tiles} n={n}", flush=True)
        g = torch.Generator(device=gpu).manual_seed(tiles)
        nb = (n + 15) // 16 + 3
        perm = torch.randperm(nb, generator=torch.Generator().manual_seed(tiles)).tolist()
        q = torch.randn(1, hq, d, generator=g, device=gpu).to(torch.bfloat16)
        ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
        vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
        case = workloads.DecodeCase("parts", q, ksrc, vsrc, [perm[: (n + 15) // 16]], [n], 16, 1 / math.sqrt(d),
                                    torch.float8_e4m3fn)
        kc, vc, ks, vs = workloads.materialize(case, "paired")
        out = _run(case, kc, vc, ks, vs, gpu)
        ref = oracle_decode(case, kc, vc, ks, vs)
        assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"{tiles} tiles")


@pytest.mark.parametrize("kv_dtype,bs,d", [(torch.float32, 16, 64), (torch.float32, 16, 256), (torch.bfloat16, 8, 80)])
def test_generic_path_many_partitions(gpu, kv_dtype, bs, d):
    """The generic (VALU) path on a small batch: the partition length shrinks
    to 32 tokens, so a 20000-token sequence leaves 625 partials per query head
    for the merge (more than its 256 threads, in several groups per channel)."""
    print(f"[case] generic many partitions kv={kv_dtype} bs={bs} d={d}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(31)
    lens = [20000, 5]
    hq, hkv = 4, 2
    nb = sum((n + bs - 1) // bs for n in lens) + 2
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(4)).tolist()
    tables, pos = [], 0
    for n in lens:
        k = (n + bs - 1) // bs
        tables.append(perm[pos:pos + k])
        pos += k
    q_dtype = torch.float32 if kv_dtype == torch.float32 else torch.bfloat16
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu).to(q_dtype)
    ksrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu).to(q_dtype)
    vsrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu).to(q_dtype)
    case = workloads.DecodeCase("generic", q, ksrc, vsrc, tables, lens, bs, 1 / math.sqrt(d), kv_dtype)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _run(case, kc, vc, ks, vs, gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, q_dtype, f"generic {kv_dtype}/{bs}/{d}")


def test_generic_path_many_query_heads_per_kv_head(gpu):
    """64 query heads over one fp32 KV head: the default 512-token partition
    does not fit a workgroup's LDS, so the generic path shrinks it."""
    print("[case] generic G=64", flush=True)
    g = torch.Generator(device=gpu).manual_seed(17)
    lens, hq, hkv, d, bs = [3000, 77], 64, 1, 128, 16
    nb = sum((n + bs - 1) // bs for n in lens) + 1
    tables, pos = [], 0
    for n in lens:
        k = (n + bs - 1) // bs
        tables.append(list(range(pos, pos + k)))
        pos += k
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu)
    ksrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu)
    vsrc = torch.randn(nb, bs, hkv, d, generator=g, device=gpu)
    case = workloads.DecodeCase("g64", q, ksrc, vsrc, tables, lens, bs, 1 / math.sqrt(d), torch.float32)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _run(case, kc, vc, ks, vs, gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.float32, "generic G=64")


def test_repeated_calls_share_a_workspace(gpu):
    """Repeated calls on one workspace give bit-identical outputs, also after
    a call with another batch shape in between."""
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=13, batch=16)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    need = ops.decode_workspace_bytes(16, 32, 8, 128, tables.shape[1], 16)
    ws = ops.new_workspace(need, gpu)
    outs = []
    for i in range(4):
        if i == 2:  # a differently shaped call in between
            ops.paged_decode(case.q[:3], kc, vc, tables[:3], lens[:3], case.scale, 16, ks, vs, workspace=ws)
        outs.append(ops.paged_decode(case.q, kc, vc, tables, lens, case.scale, 16, ks, vs, workspace=ws).clone())
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(outs[0].float().cpu().numpy(), ref, torch.bfloat16, "repeated")


def test_invalid_block_ids_contribute_nothing(gpu):
    """Tensor API: a table entry outside [0, NB) drops that block's tokens."""
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=14, batch=4)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    nb = kc.shape[0]
    tables = case.tables_tensor(gpu)
    bad = tables.clone()
    bad[0, 3] = nb + 7  # a full middle block of sequence 0
    bad[1, 5] = -2
    out = _run(case, kc, vc, ks, vs, gpu, tables=bad)
    t0 = case.block_tables[0][:3] + case.block_tables[0][4:]
    t1 = case.block_tables[1][:5] + case.block_tables[1][6:]
    lens = [case.seq_lens[0] - 16, case.seq_lens[1] - 16, case.seq_lens[2], case.seq_lens[3]]
    ref = oracle_decode(case, kc, vc, ks, vs, tables=[t0, t1, case.block_tables[2], case.block_tables[3]], lens=lens)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "invalid ids")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("scale", [-0.09, 0.0, 0.5])
def test_softmax_scales(gpu, scale, kv_dtype):
    """Negative, zero (uniform weights) and large softmax scales."""
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=17, batch=5)
    case.kv_dtype = kv_dtype
    kc, vc, ks, vs = workloads.materialize(case, "native")
    case.scale = scale
    out = _run(case, kc, vc, ks, vs, gpu)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"decode scale {scale} {kv_dtype}")


def _sample_ids(lens: list[int], fixed: list[int], n_random: int, seed: int) -> list[int]:
    """`fixed` ids, the longest and shortest sequence, and n_random more."""
    rng = np.random.default_rng(seed)
    ids = set(i for i in fixed if i < len(lens))
    ids.add(int(np.argmax(lens)))
    ids.add(int(np.argmin(lens)))
    rest = [i for i in range(len(lens)) if i not in ids]
    ids.update(int(i) for i in rng.choice(rest, size=min(n_random, len(rest)), replace=False))
    return sorted(ids)


def _permuted_paired(kc, vc, gpu, seed: int):
    """The same cache contents under a seeded permutation of the physical
    block ids: (k, v, inverse map old id -> new id)."""
    nb, bs, hkv, d = kc.shape
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed)).to(gpu)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb, device=gpu)
    k2, v2 = L.alloc_kv_cache(nb, bs, hkv, d, kc.dtype, gpu, "paired")
    k2.copy_(kc[perm])
    v2.copy_(vc[perm])
    return k2, v2, inv


def test_full_c3_as_benchmarked(gpu):
    """BASELINE configs[2] exactly as bench.py times it: batch 64, paired KV
    layout, the shared-prefix statement, a DecodePlan rerun step after step.
    Oracle on 20 sequences (sharers at group edges, private ones, the
    longest and the shortest); reruns bitwise identical; block-permutation
    invariance (bitwise) over the whole batch."""
    print("[case] c3 full size, paired layout, shared-prefix statement (the benchmark step)", flush=True)
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=0)
    kc, vc, ks, vs = workloads.materialize(case, "paired")
    assert L.layout_of(kc, False) == "paired" and L.layout_of(vc, True) == "paired"
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    shared_list = ops.shared_prefix_lens(case.block_tables, case.seq_lens, 16)
    assert shared_list[1:32] == [1024] * 31 and not any(shared_list[32:])
    shared = torch.tensor(shared_list, dtype=torch.int32, device=gpu)
    plan = ops.DecodePlan(case.q, kc, vc, tables, lens, case.scale, 16, ks, vs, shared_prefix_lens=shared)
    with ops.KernelTimer() as timer:
        out = plan.run().clone()
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 1 and timer.query("cf_decode_generic")[1] == 0
    for _ in range(3):
        again = plan.run()
    torch.cuda.synchronize()
    assert torch.equal(again, out)
    idx = _sample_ids(case.seq_lens, [0, 1, 3, 4, 7, 8, 15, 16, 30, 31, 32, 33, 62, 63], 4, seed=1)
    assert len(idx) >= 16
    sub = workloads.DecodeCase("c3_sample", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], 16, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kc, vc, ks, vs)
    assert_close(out[idx].float().cpu().numpy(), ref, torch.bfloat16, f"c3 benchmarked step, {len(idx)} sequences")
    k2, v2, inv = _permuted_paired(kc, vc, gpu, seed=5)
    t2 = inv[tables.long()].to(torch.int32)
    out2 = ops.DecodePlan(case.q, k2, v2, t2, lens, case.scale, 16, ks, vs, shared_prefix_lens=shared).run()
    torch.cuda.synchronize()
    assert torch.equal(out2, out)


def test_full_c4_llama3_70b(gpu):
    """BASELINE configs[3] at full size: batch 128, 64 query / 8 KV heads,
    lognormal contexts up to 32,768 tokens, paired layout.  Oracle on 16
    sequences including the longest; block-permutation invariance
    (bitwise) over the whole batch; a second call bitwise identical."""
    print("[case] c4 full size (batch 128), paired layout", flush=True)
    case = workloads.make_case("c4_llama3_70b", device=gpu, seed=0)
    assert case.batch == 128 and case.q.shape[1] == 64 and case.num_kv_heads == 8
    kc, vc, ks, vs = workloads.materialize(case, "paired")
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    with ops.KernelTimer() as timer:
        out = _run(case, kc, vc, ks, vs, gpu)
        assert timer.query("cf_decode_mfma")[1] == 1
    again = _run(case, kc, vc, ks, vs, gpu)
    assert torch.equal(again, out)
    order = np.argsort(case.seq_lens)
    idx = _sample_ids(case.seq_lens, [0, 1, 64, 127, int(order[-2]), int(order[-3])], 10, seed=2)
    assert len(idx) >= 16 and int(np.argmax(case.seq_lens)) in idx
    print(f"[case] c4 oracle on {len(idx)} sequences, longest {max(case.seq_lens)} tokens", flush=True)
    sub = workloads.DecodeCase("c4_sample", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], 16, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kc, vc, ks, vs)
    assert_close(out[idx].float().cpu().numpy(), ref, torch.bfloat16, f"c4 full, {len(idx)} sequences")
    k2, v2, inv = _permuted_paired(kc, vc, gpu, seed=6)
    out2 = _run(case, k2, v2, ks, vs, gpu, tables=inv[tables.long()].to(torch.int32))
    assert torch.equal(out2, out)


@pytest.mark.parametrize("kv_dtype,q_dtype", [(torch.float8_e4m3fn, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                              (torch.float16, torch.float16)])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 2, 128), (32, 2, 64)])
def test_token_major_on_the_mfma_path(gpu, hq, hkv, d, kv_dtype, q_dtype):
    """Caches in the reference's own token-major layout ([NB, bs, Hkv, D]) run
    the MFMA kernel (V staged through LDS and read back transposed: 8-bit
    rows for e4m3, 16-bit for bf16 / fp16); lengths ending mid-block and
    mid-tile, one token, an invalid block id and a shared-prefix statement;
    outputs bitwise equal to the native layout's (the same operands reach
    the same MFMAs) and to the oracle's bound."""
    print(f"[case] token-major {kv_dtype} hq={hq} hkv={hkv} d={d}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(hq + 7 * d)
    lens = [1, 15, 33, 700, 1024 + 40, 1024 + 100, 2000]
    nb = 400
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(5)).tolist()
    shared = perm[:64]
    tables, pos = [], 64
    for i, n in enumerate(lens):
        k = (n + 15) // 16
        if i in (4, 5):
            tables.append(shared + perm[pos:pos + k - 64])
            pos += k - 64
        else:
            tables.append(perm[pos:pos + k])
            pos += k
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu).to(q_dtype)
    ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(q_dtype)
    vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(q_dtype)
    case = workloads.DecodeCase("tok", q, ksrc, vsrc, tables, lens, 16, 1 / math.sqrt(d), kv_dtype)
    kt, vt, ks, vs = workloads.materialize(case, "token_major")
    assert L.layout_of(kt, False) == "token_major" and L.layout_of(vt, True) == "token_major"
    kn, vn, _, _ = workloads.materialize(case, "native")
    tab = case.tables_tensor(gpu)
    bad = tab.clone()
    bad[3, 7] = nb + 3  # an invalid block in the middle of sequence 3
    sh = torch.tensor(ops.shared_prefix_lens(tables, lens, 16), dtype=torch.int32, device=gpu)
    with ops.KernelTimer() as timer:
        out_t = paged_attention_tensors(q, kt, vt, bad, case.seq_lens_tensor(gpu), 16, case.scale, k_scale=ks,
                                        v_scale=vs, shared_prefix_lens=sh)
        out_n = paged_attention_tensors(q, kn, vn, bad, case.seq_lens_tensor(gpu), 16, case.scale, k_scale=ks,
                                        v_scale=vs, shared_prefix_lens=sh)
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 2 and timer.query("cf_decode_generic")[1] == 0
    assert torch.equal(out_t, out_n)
    t3 = tables[3][:7] + tables[3][8:]
    eff = list(lens)
    eff[3] -= 16
    ref = oracle_decode(case, kt, vt, ks, vs, tables=tables[:3] + [t3] + tables[4:], lens=eff)
    assert_close(out_t.float().cpu().numpy(), ref, q_dtype, f"token-major {kv_dtype} {hq}/{hkv}/{d}")


@pytest.mark.parametrize("kv_dtype,q_dtype", [(torch.float8_e4m3fn, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                              (torch.float16, torch.float16)])
def test_head_major_tiles_on_the_mfma_path(gpu, kv_dtype, q_dtype):
    """K and V both stored as [NB, {K, V}, Hkv, bs, D] (one (block, head) tile
    of token rows per head, as the engine mixin's combined cache keeps a
    layer): V is token-major with head stride bs*D, which the MFMA kernel
    takes like the reference's layout; bitwise equal to the native layout."""
    print(f"[case] head-major tiles {kv_dtype}", flush=True)
    hq, hkv, d, nb = 32, 8, 128, 300
    g = torch.Generator(device=gpu).manual_seed(11)
    lens = [1, 17, 500, 1300, 2048]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(2)).tolist()
    tables, pos = [], 0
    for n in lens:
        tables.append(perm[pos:pos + (n + 15) // 16])
        pos += (n + 15) // 16
    q = torch.randn(len(lens), hq, d, generator=g, device=gpu).to(q_dtype)
    ksrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(q_dtype)
    vsrc = torch.randn(nb, 16, hkv, d, generator=g, device=gpu).to(q_dtype)
    case = workloads.DecodeCase("hm", q, ksrc, vsrc, tables, lens, 16, 1 / math.sqrt(d), kv_dtype)
    kn, vn, ks, vs = workloads.materialize(case, "native")
    store = torch.empty(nb, 2, hkv, 16, d, dtype=kv_dtype, device=gpu)
    kh, vh = store[:, 0].permute(0, 2, 1, 3), store[:, 1].permute(0, 2, 1, 3)
    raw = (lambda t: t.view(torch.uint8)) if kv_dtype == torch.float8_e4m3fn else (lambda t: t)
    raw(kh).copy_(raw(kn))
    raw(vh).copy_(raw(vn))
    assert vh.stride() == (2 * hkv * 16 * d, d, 16 * d, 1)
    tab, sl = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    with ops.KernelTimer() as timer:
        out_h = paged_attention_tensors(q, kh, vh, tab, sl, 16, case.scale, k_scale=ks, v_scale=vs)
        out_n = paged_attention_tensors(q, kn, vn, tab, sl, 16, case.scale, k_scale=ks, v_scale=vs)
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 2 and timer.query("cf_decode_generic")[1] == 0
    assert torch.equal(out_h, out_n)
    ref = oracle_decode(case, kn, vn, ks, vs)
    assert_close(out_h.float().cpu().numpy(), ref, q_dtype, f"head-major {kv_dtype}")


def test_full_c2_token_major(gpu):
    """Config 2 (bf16 caches) in the reference's token-major layout at full
    size: the MFMA path, bitwise equal to the paired layout's output, and the
    oracle on sampled sequences."""
    print("[case] c2 full size, token-major layout", flush=True)
    case = workloads.make_case("c2_tinyllama", device=gpu, seed=0)
    kt, vt, ks, vs = workloads.materialize(case, "token_major")
    kp, vp, _, _ = workloads.materialize(case, "paired")
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    with ops.KernelTimer() as timer:
        out_t = ops.DecodePlan(case.q, kt, vt, tables, lens, case.scale, 16, ks, vs).run()
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 1 and timer.query("cf_decode_generic")[1] == 0
    out_p = ops.DecodePlan(case.q, kp, vp, tables, lens, case.scale, 16, ks, vs).run()
    torch.cuda.synchronize()
    assert torch.equal(out_t, out_p)
    idx = _sample_ids(case.seq_lens, [0, 1, 31], 13, seed=4)
    sub = workloads.DecodeCase("c2_tok", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], 16, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kt, vt, ks, vs)
    assert_close(out_t[idx].float().cpu().numpy(), ref, torch.bfloat16, "c2 token-major")


def test_full_c3_token_major(gpu):
    """The headline config in the reference's token-major layout at full size:
    the MFMA path, bitwise equal to the paired layout's output, and the
    oracle on 16 sampled sequences."""
    print("[case] c3 full size, token-major layout", flush=True)
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=0)
    kt, vt, ks, vs = workloads.materialize(case, "token_major")
    kp, vp, _, _ = workloads.materialize(case, "paired")
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    sh = torch.tensor(ops.shared_prefix_lens(case.block_tables, case.seq_lens, 16), dtype=torch.int32, device=gpu)
    with ops.KernelTimer() as timer:
        out_t = ops.DecodePlan(case.q, kt, vt, tables, lens, case.scale, 16, ks, vs, shared_prefix_lens=sh).run()
        torch.cuda.synchronize()
        assert timer.query("cf_decode_mfma")[1] == 1
    out_p = ops.DecodePlan(case.q, kp, vp, tables, lens, case.scale, 16, ks, vs, shared_prefix_lens=sh).run()
    torch.cuda.synchronize()
    assert torch.equal(out_t, out_p)
    idx = _sample_ids(case.seq_lens, [0, 1, 31, 32, 63], 9, seed=3)
    sub = workloads.DecodeCase("c3_tok", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], 16, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kt, vt, ks, vs)
    assert_close(out_t[idx].float().cpu().numpy(), ref, torch.bfloat16, "c3 token-major")
