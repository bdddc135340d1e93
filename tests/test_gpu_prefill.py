"""GPU parity of the chunked-prefill kernel (and the c5 mixed step).

Small cases compare every row with the float64 oracle
(oracle.paged_attention.paged_prefill_fp64).  The full c5 step checks
size-independent properties: every prefill row equals the decode kernel
run with the row's truncated length (the semantics' own reduction), the
written FP8 codes equal the oracle encoder's bit for bit, and a sample of
rows and decodes matches the float64 oracle.  Tolerances: bf16 outputs
within 2e-2 of the exact value rounded to bf16, cosine >= 0.9999.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cf_hip import ops, workloads
from kernels.paged_attention import chunked_prefill_attention, paged_attention_tensors
from oracle import fp8 as ofp8
from oracle.paged_attention import paged_attention_fp64, paged_prefill_fp64
from tests.gpu_util import assert_close, codes

pytestmark = pytest.mark.gpu


def _write_new_rows(case, t):
    """The step's cache write: e4m3 through the product kernel, bf16 by
    plain indexing."""
    if t["k_scale"] is not None:
        ops.kv_write_fp8(t["k_new"], t["v_new"], t["slots"], t["k_cache"], t["v_cache"], t["k_scale"],
                         t["v_scale"])
    else:
        bs = case.block_size
        s = t["slots"]
        t["k_cache"][s // bs, s % bs] = t["k_new"].to(t["k_cache"].dtype)
        t["v_cache"][s // bs, s % bs] = t["v_new"].to(t["v_cache"].dtype)


def _cache_values(kc, vc, used):
    idx = torch.tensor(used, dtype=torch.long, device=kc.device)
    kc, vc = kc[idx], vc[idx]
    if kc.dtype == torch.float8_e4m3fn:
        return ofp8.decode(codes(kc)), ofp8.decode(codes(vc))
    return kc.float().cpu().numpy(), vc.float().cpu().numpy()


def _remap(tables):
    used = sorted({b for t in tables for b in t})
    remap = {b: i for i, b in enumerate(used)}
    return used, [[remap[b] for b in t] for t in tables]


def oracle_prefill(case, t, q=None, tables=None, lens=None, q_start=None, scale=None):
    tables = [list(x) for x in (tables if tables is not None else case.prefill_tables)]
    used, rt = _remap(tables)
    k, v = _cache_values(t["k_cache"], t["v_cache"], used)
    ks = t["k_scale"].cpu().numpy() if t["k_scale"] is not None else None
    vs = t["v_scale"].cpu().numpy() if t["v_scale"] is not None else None
    q = (q if q is not None else case.q_prefill).float().cpu().numpy()
    return paged_prefill_fp64(q, k, v, rt, list(lens if lens is not None else case.prefill_lens),
                              list(q_start if q_start is not None else case.q_start), case.block_size,
                              case.scale if scale is None else scale, ks, vs)


def _prefill(case, t, **kw):
    out = chunked_prefill_attention(
        kw.get("q", t["q_prefill"]), t["k_cache"], t["v_cache"], kw.get("tables", t["prefill_tables"]),
        kw.get("lens", t["prefill_lens"]), kw.get("q_start", t["q_start"]), case.block_size,
        kw.get("scale", case.scale),
        k_scale=t["k_scale"], v_scale=t["v_scale"], out=kw.get("out"),
    )
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 1, 128), (32, 2, 64), (4, 2, 128),
                                      (16, 8, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("layout", ["paired", "native", "token_major"])
def test_shapes_match_oracle(gpu, hq, hkv, d, kv_dtype, layout):
    print(f"[case] prefill hq={hq} hkv={hkv} d={d} kv={kv_dtype} layout={layout}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=hq + d, chunks=[1, 17, 64, 100, 33],
                                     cached=[0, 5, 300, 33, 1000], decode_lens=[], num_q_heads=hq,
                                     num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype)
    t = workloads.materialize_mixed(case, layout)
    _write_new_rows(case, t)
    out = _prefill(case, t)
    ref, covered = oracle_prefill(case, t)
    assert covered.all()
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"prefill {hq}/{hkv}/{d}/{kv_dtype}")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 1, 128), (32, 2, 64)])
@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.float8_e4m3fn])
@pytest.mark.parametrize("layout", ["paired", "token_major"])
def test_fp16_queries_match_oracle(gpu, hq, hkv, d, kv_dtype, layout):
    """fp16 queries (an fp16 model's prefill) over fp16 or e4m3 caches: the
    kernel's fp16 operand path (e4m3 K and V convert exactly to fp16) against
    the float64 oracle on the same fp16 queries, fp16 output."""
    print(f"[case] fp16-q prefill hq={hq} hkv={hkv} d={d} kv={kv_dtype} layout={layout}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=3 * hq + d, chunks=[1, 17, 64, 100, 33],
                                     cached=[0, 5, 300, 33, 1000], decode_lens=[], num_q_heads=hq,
                                     num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype)
    t = workloads.materialize_mixed(case, layout)
    _write_new_rows(case, t)
    q16 = t["q_prefill"].to(torch.float16)
    out = _prefill(case, t, q=q16)
    assert out.dtype == torch.float16
    ref, covered = oracle_prefill(case, t, q=q16)
    assert covered.all()
    assert_close(out.float().cpu().numpy(), ref, torch.float16, f"fp16-q prefill {hq}/{hkv}/{d}/{kv_dtype}")


def test_fp16_queries_reject_bf16_caches(gpu):
    """fp16 queries over a bf16 cache have no exact common MFMA operand type:
    refused (NotImplementedError), as the decode kernel refuses them."""
    case = workloads.make_mixed_case(device=gpu, seed=21, chunks=[8], cached=[0], decode_lens=[],
                                     num_q_heads=8, num_kv_heads=2, head_dim=64, kv_dtype=torch.bfloat16)
    t = workloads.materialize_mixed(case)
    with pytest.raises(NotImplementedError):
        _prefill(case, t, q=t["q_prefill"].to(torch.float16))


@pytest.mark.parametrize("seed", range(12))
def test_random_configurations(gpu, seed):
    """Seeded random steps over every supported head shape, cache dtype and
    layout: 1-6 chunks of 1-300 rows over cached prefixes of 0-2,000
    tokens, so the work lists run from a handful of items (all on the
    shared queue) to hundreds (per-XCD lists plus queue)."""
    rng = np.random.default_rng(1000 + seed)
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8, 16]))
    d = int(rng.choice([64, 128]))
    kv_dtype = [torch.bfloat16, torch.float8_e4m3fn][int(rng.integers(2))]
    layout = ["paired", "native", "token_major"][int(rng.integers(3))]
    n = int(rng.integers(1, 7))
    chunks = [int(x) for x in rng.integers(1, 301, n)]
    cached = [int(x) for x in rng.integers(0, 2001, n)]
    print(f"[case] random prefill seed={seed} hkv={hkv} g={g} d={d} kv={kv_dtype} layout={layout} "
          f"chunks={chunks} cached={cached}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=seed, chunks=chunks, cached=cached, decode_lens=[],
                                     num_q_heads=hkv * g, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype)
    t = workloads.materialize_mixed(case, layout)
    _write_new_rows(case, t)
    out = _prefill(case, t)
    ref, covered = oracle_prefill(case, t)
    assert covered.all()
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"random {seed}")


@pytest.mark.parametrize("chunks,cached", [([512], [0]), ([512], [4096]), ([1] * 40, list(range(0, 4000, 100))),
                                           ([700, 3], [17, 9000])])
def test_chunk_mixes(gpu, chunks, cached):
    print(f"[case] prefill chunks={chunks[:4]}.. cached={cached[:4]}..", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=5, chunks=chunks, cached=cached, decode_lens=[])
    t = workloads.materialize_mixed(case)
    _write_new_rows(case, t)
    out = _prefill(case, t)
    ref, _ = oracle_prefill(case, t)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "chunk mix")


@pytest.mark.parametrize("layout", ["paired", "token_major"])
def test_edge_rules(gpu, layout):
    """Overlapping and empty chunks, rows outside every chunk (left as they
    were), rows at negative positions (zeros), lengths past the table."""
    print(f"[case] prefill edge rules layout={layout}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=9, chunks=[40, 30, 20], cached=[10, 50, 0],
                                     decode_lens=[])
    t = workloads.materialize_mixed(case, layout)
    _write_new_rows(case, t)
    q_start = [3, 45, 41, 41, 80]  # chunk 1 overlaps chunk 0; chunk 2 is empty after the cut
    lens = [52, 20, 20, 5]  # chunk 3: 35 rows, 5 tokens -> 30 rows at negative positions
    tables = case.prefill_tables + [case.prefill_tables[2]]
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    qs_t = torch.tensor(q_start, dtype=torch.int32, device=gpu)
    tab_t = workloads._int_tensor(tables, gpu)
    sentinel = torch.full_like(t["q_prefill"], 7.0)
    out = _prefill(case, t, tables=tab_t, lens=lens_t, q_start=qs_t, out=sentinel.clone())
    ref, covered = oracle_prefill(case, t, tables=tables, lens=lens, q_start=q_start)
    got = out.float().cpu().numpy()
    assert (got[~covered] == 7.0).all()
    assert covered.sum() == 77 and not covered[:3].any() and not covered[80:].any()
    assert_close(got[covered], ref[covered], torch.bfloat16, "edge rules")
    assert (got[45:75] == 0).all()
    # a length past the table's capacity reads the table's tokens only
    cap = len(case.prefill_tables[0]) * 16
    lens2 = torch.tensor([cap + 100], dtype=torch.int32, device=gpu)
    qs2 = torch.tensor([0, 8], dtype=torch.int32, device=gpu)
    tab0 = workloads._int_tensor(case.prefill_tables[:1], gpu)  # exactly table 0's blocks
    out2 = _prefill(case, t, q=t["q_prefill"][:8], tables=tab0, lens=lens2, q_start=qs2)
    ref2, _ = oracle_prefill(case, t, q=case.q_prefill[:8], tables=case.prefill_tables[:1], lens=[cap + 100],
                             q_start=[0, 8])
    assert_close(out2.float().cpu().numpy(), ref2, torch.bfloat16, "past capacity")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("d", [64, 128])
def test_token_major_matches_native_bitwise(gpu, kv_dtype, d):
    """The reference's own cache layout ([NB, bs, Hkv, D] contiguous: V in
    token rows) gives the native layout's output bit for bit: the same
    operands reach the same products.  Seq 1's table holds an invalid (-1)
    entry among its cached blocks, and every chunk ends inside a tile."""
    print(f"[case] prefill token-major vs native kv={kv_dtype} d={d}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=21, chunks=[1, 33, 100], cached=[7, 250, 31],
                                     decode_lens=[], num_q_heads=16, num_kv_heads=4, head_dim=d,
                                     kv_dtype=kv_dtype)
    t = workloads.materialize_mixed(case, "native")
    _write_new_rows(case, t)
    tables = [list(x) for x in case.prefill_tables]
    tables[1][3] = -1
    tab = workloads._int_tensor(tables, gpu)
    out_native = _prefill(case, t, tables=tab)
    tm = dict(t, k_cache=t["k_cache"].contiguous(), v_cache=t["v_cache"].contiguous())
    assert tm["v_cache"].stride(1) == 4 * d and tm["v_cache"].stride(3) == 1
    out_tok = _prefill(case, tm, tables=tab)
    assert torch.equal(out_native, out_tok)
    assert torch.isfinite(out_tok.float()).all()


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize("scale", [-0.09, 0.0, 0.5])
def test_softmax_scales(gpu, scale, kv_dtype):
    """Negative, zero and large softmax scales (the kernel takes its running
    max on raw scores and negates q for a negative scale)."""
    case = workloads.make_mixed_case(device=gpu, seed=16, chunks=[40, 70], cached=[30, 200], decode_lens=[],
                                     kv_dtype=kv_dtype)
    t = workloads.materialize_mixed(case)
    _write_new_rows(case, t)
    out = _prefill(case, t, scale=scale)
    ref, _ = oracle_prefill(case, t, scale=scale)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"scale {scale}")


def test_repeated_calls_shrinking(gpu):
    """Back-to-back calls through one cached workspace, the second smaller:
    no state of the first leaks into the second."""
    big = workloads.make_mixed_case(device=gpu, seed=12, chunks=[300, 200], cached=[2000, 100], decode_lens=[])
    tb = workloads.materialize_mixed(big)
    _write_new_rows(big, tb)
    small = workloads.make_mixed_case(device=gpu, seed=13, chunks=[20], cached=[60], decode_lens=[])
    ts = workloads.materialize_mixed(small)
    _write_new_rows(small, ts)
    for _ in range(2):
        ob = _prefill(big, tb)
        os_ = _prefill(small, ts)
    assert_close(ob.float().cpu().numpy(), oracle_prefill(big, tb)[0], torch.bfloat16, "big")
    assert_close(os_.float().cpu().numpy(), oracle_prefill(small, ts)[0], torch.bfloat16, "small")


@pytest.mark.parametrize("layout", ["paired", "token_major"])
def test_c5_full_step(gpu, layout):
    """The full c5 step: write, decode, prefill on one stream (the
    benchmarked paired layout, and the reference's own token-major one)."""
    print(f"[case] c5 full step layout={layout}", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=0)
    t = workloads.materialize_mixed(case, layout)
    _write_new_rows(case, t)
    dec = paged_attention_tensors(t["q_decode"], t["k_cache"], t["v_cache"], t["decode_tables"], t["decode_lens"],
                                  16, case.scale, k_scale=t["k_scale"], v_scale=t["v_scale"])
    pre = _prefill(case, t)

    # written codes: bit-exact against the oracle encoder
    kc_new = t["k_cache"].view(torch.uint8)[t["slots"] // 16, t["slots"] % 16]
    vc_new = t["v_cache"].view(torch.uint8)[t["slots"] // 16, t["slots"] % 16]
    ks, vs = t["k_scale"].cpu().numpy(), t["v_scale"].cpu().numpy()
    want_k = ofp8.encode(case.k_new.float().cpu().numpy() / ks[None, :, None])
    want_v = ofp8.encode(case.v_new.float().cpu().numpy() / vs[None, :, None])
    assert np.array_equal(kc_new.cpu().numpy(), want_k)
    assert np.array_equal(vc_new.cpu().numpy(), want_v)

    # every prefill row == decode with the row's truncated length
    rows_tables, rows_lens = [], []
    for n, (c, ln) in enumerate(zip(case.meta["cached"], case.meta["chunks"])):
        rows_tables += [case.prefill_tables[n]] * ln
        rows_lens += [c + i + 1 for i in range(ln)]
    rt = workloads._int_tensor(rows_tables, gpu)
    rl = torch.tensor(rows_lens, dtype=torch.int32, device=gpu)
    as_decode = paged_attention_tensors(t["q_prefill"], t["k_cache"], t["v_cache"], rt, rl, 16, case.scale,
                                        k_scale=t["k_scale"], v_scale=t["v_scale"])
    torch.cuda.synchronize()
    assert_close(pre.float().cpu().numpy(), as_decode.float().cpu().numpy(), torch.bfloat16, "prefill vs decode")

    # sampled rows and decodes against the float64 oracle
    g = torch.Generator().manual_seed(1)
    sample = sorted(set(torch.randint(0, len(rows_lens), (48,), generator=g).tolist()) | {0, 511, 4095})
    used, remapped = _remap([rows_tables[i] for i in sample] + [case.decode_tables[i] for i in range(8)])
    k, v = _cache_values(t["k_cache"], t["v_cache"], used)
    qs = torch.cat([case.q_prefill[sample], case.q_decode[:8]]).float().cpu().numpy()
    lens = [rows_lens[i] for i in sample] + case.decode_lens[:8]
    ref = paged_attention_fp64(qs, k, v, remapped, lens, 16, case.scale, ks, vs)
    got = torch.cat([pre[sample], dec[:8]]).float().cpu().numpy()
    assert_close(got, ref, torch.bfloat16, "c5 sampled rows")


def test_c5_step_two_streams(gpu):
    """Decode and prefill side by side (ops.run_concurrent) give the same
    bits as one after another, on every call of a repeated step whose
    outputs the caller's stream then reads."""
    print("[case] c5 step, decode || prefill on two streams", flush=True)
    case = workloads.make_mixed_case(device=gpu, seed=0)
    t = workloads.materialize_mixed(case)
    _write_new_rows(case, t)
    plan = ops.DecodePlan(t["q_decode"], t["k_cache"], t["v_cache"], t["decode_tables"], t["decode_lens"],
                          case.scale, 16, t["k_scale"], t["v_scale"])
    dec_ref = plan.run().clone()
    pre_ref = _prefill(case, t).clone()
    out = torch.empty_like(pre_ref)

    def prefill():
        chunked_prefill_attention(t["q_prefill"], t["k_cache"], t["v_cache"], t["prefill_tables"],
                                  t["prefill_lens"], t["q_start"], 16, case.scale, k_scale=t["k_scale"],
                                  v_scale=t["v_scale"], out=out)

    for i in range(3):
        plan.out.zero_()
        out.zero_()
        ops.run_concurrent(plan.run, prefill, gpu, keep=(out,))
        # read on the caller's stream: ordered after both
        same_dec = torch.equal(plan.out, dec_ref)
        same_pre = torch.equal(out, pre_ref)
        torch.cuda.synchronize()
        assert same_dec and same_pre, f"call {i}: decode equal {same_dec}, prefill equal {same_pre}"


def test_run_concurrent_orders_work_when_a_callable_raises(gpu):
    """A side callable that raises after enqueuing work: the error reaches
    the caller, and the caller's stream still waits for what was enqueued."""
    x = torch.zeros(1 << 22, device=gpu)
    big = torch.randn(1 << 22, device=gpu)

    def side():
        x.copy_(big * 2.0 + 1.0)
        raise RuntimeError("side failed")

    with pytest.raises(RuntimeError, match="side failed"):
        ops.run_concurrent(lambda: None, side, gpu)
    got = (x - (big * 2.0 + 1.0)).abs().max()  # on the caller's stream
    assert float(got) == 0.0


def test_hal_op(gpu):
    from python_runtime.hal.hip_backend import HipBackend

    case = workloads.make_mixed_case(device=gpu, seed=14, chunks=[24, 9], cached=[40, 0], decode_lens=[])
    t = workloads.materialize_mixed(case)
    _write_new_rows(case, t)
    out = HipBackend().execute(
        "chunked_prefill_attention",
        [t["q_prefill"], t["k_cache"], t["v_cache"], t["prefill_tables"], t["prefill_lens"], t["q_start"]],
        scale=case.scale, k_scale=t["k_scale"], v_scale=t["v_scale"],
    )
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), oracle_prefill(case, t)[0], torch.bfloat16, "hal")


def test_rejects_unsupported(gpu):
    case = workloads.make_mixed_case(device=gpu, seed=15, chunks=[4], cached=[0], decode_lens=[],
                                     num_q_heads=6, num_kv_heads=2, head_dim=64)  # G = 3
    t = workloads.materialize_mixed(case)
    with pytest.raises(NotImplementedError):
        _prefill(case, t)
