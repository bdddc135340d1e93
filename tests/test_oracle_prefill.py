"""Pins the chunked-prefill oracle (oracle/paged_attention.py).

No reference function attends a chunk to a cached prefix; the semantics
are fixed by reduction: a chunk row at position p equals the reference's
decode (_paged_attention_cpu, kernels/paged_attention.py:21-73, restated
as paged_attention_cpu) with seq_len = p + 1, and a chunk with nothing
cached is causal self-attention (the reference's _flash_attention_fwd_cpu,
kernels/flash_attention.py:28-46: SDPA with is_causal=True).  The float64
brute force is checked against both, so an off-by-one causal mask, a
top-left instead of bottom-right alignment, a wrong GQA head or a wrong
block offset fails one of them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import workloads
from oracle.paged_attention import chunk_rows, paged_prefill_by_decode, paged_prefill_fp64


def _small_case(seed, chunks, cached, hq=8, hkv=2, d=32, kv_dtype=torch.float32):
    case = workloads.make_mixed_case(seed=seed, chunks=chunks, cached=cached, decode_lens=[],
                                     num_q_heads=hq, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype)
    # the cache after the step's write: pool with the new rows at their slots
    k = case.k_pool.float().clone()
    v = case.v_pool.float().clone()
    bs = case.block_size
    for i, s in enumerate(case.slots):
        k[s // bs, s % bs] = case.k_new[i].float()
        v[s // bs, s % bs] = case.v_new[i].float()
    return case, k, v


@pytest.mark.parametrize("seed,chunks,cached,hq,hkv", [
    (1, [5, 17], [0, 40], 8, 2),
    (2, [33], [100], 4, 4),
    (3, [1, 16, 31], [7, 0, 64], 16, 1),
])
def test_fp64_matches_per_row_decode(seed, chunks, cached, hq, hkv):
    case, k, v = _small_case(seed, chunks, cached, hq, hkv)
    q = case.q_prefill.float()
    ref, covered = paged_prefill_fp64(q.numpy(), k.numpy(), v.numpy(), case.prefill_tables, case.prefill_lens,
                                      case.q_start, 16, case.scale)
    assert covered.all()
    rows = paged_prefill_by_decode(q, k, v, case.prefill_tables, case.prefill_lens, case.q_start, 16, case.scale)
    assert len(rows) == q.shape[0]
    got = np.stack([rows[i].numpy() for i in range(q.shape[0])])
    assert np.abs(got - ref).max() < 1e-5


def test_no_cache_chunk_is_causal_self_attention():
    import torch.nn.functional as F  # noqa: N812

    case, k, v = _small_case(4, [37], [0], hq=4, hkv=4, d=32)
    q = case.q_prefill.float()
    ref, _ = paged_prefill_fp64(q.numpy(), k.numpy(), v.numpy(), case.prefill_tables, case.prefill_lens,
                                case.q_start, 16, case.scale)
    t = case.prefill_tables[0]
    n = 37
    ks = torch.cat([k[b] for b in t])[:n]  # [n, H, D]
    vs = torch.cat([v[b] for b in t])[:n]
    sd = F.scaled_dot_product_attention(q.transpose(0, 1).unsqueeze(0), ks.transpose(0, 1).unsqueeze(0),
                                        vs.transpose(0, 1).unsqueeze(0), is_causal=True, scale=case.scale)
    sd = sd.squeeze(0).transpose(0, 1).numpy()
    assert np.abs(sd - ref).max() < 1e-5


def test_strict_mask_mistake_is_caught():
    """A mask that drops the diagonal (row attends to [0, p) instead of
    [0, p]) must differ from the per-row decode reduction by far more than
    the tolerance."""
    case, k, v = _small_case(5, [9], [3], hq=2, hkv=2, d=16)
    q = case.q_prefill.float()
    good, _ = paged_prefill_fp64(q.numpy(), k.numpy(), v.numpy(), case.prefill_tables, case.prefill_lens,
                                 case.q_start, 16, case.scale)
    # planted mistake: every row loses its own token
    bad, _ = paged_prefill_fp64(q.numpy(), k.numpy(), v.numpy(), case.prefill_tables,
                                [n - 1 for n in case.prefill_lens], case.q_start, 16, case.scale)
    rows = paged_prefill_by_decode(q, k, v, case.prefill_tables, case.prefill_lens, case.q_start, 16, case.scale)
    got = np.stack([rows[i].numpy() for i in range(q.shape[0])])
    assert np.abs(got - good).max() < 1e-5
    assert np.abs(got[1:] - bad[1:]).max() > 1e-2


def test_gqa_equals_repeated_heads():
    case, k, v = _small_case(6, [20], [30], hq=8, hkv=2, d=16)
    q = case.q_prefill.float().numpy()
    ref, _ = paged_prefill_fp64(q, k.numpy(), v.numpy(), case.prefill_tables, case.prefill_lens, case.q_start,
                                16, case.scale)
    k_rep = k.repeat_interleave(4, dim=2).numpy()
    v_rep = v.repeat_interleave(4, dim=2).numpy()
    mha, _ = paged_prefill_fp64(q, k_rep, v_rep, case.prefill_tables, case.prefill_lens, case.q_start, 16,
                                case.scale)
    assert np.abs(ref - mha).max() < 1e-12


def test_chunk_rows_bookkeeping():
    # ordered, disjoint chunks
    assert chunk_rows([0, 3, 10], [5, 20], 10) == [(0, 3, 2), (3, 7, 13)]
    # overlapping chunk starts where the previous one ends
    assert chunk_rows([0, 6, 4, 9], [6, 4, 3], 12) == [(0, 6, 0), (6, 0, 4), (6, 3, 0)]
    # q_start clamped to [0, Tq]; empty and negative-position chunks
    assert chunk_rows([-5, 2, 2, 50], [1, 0, 10], 8) == [(0, 2, -1), (2, 0, 0), (2, 6, 4)]


def test_negative_positions_are_zero_and_uncovered_rows_nan():
    case, k, v = _small_case(7, [6], [0], hq=2, hkv=2, d=16)
    q = case.q_prefill.float().numpy()
    # seq_len 4 < chunk 6: rows 0, 1 sit at positions -2, -1
    qs = [1, 7]
    q_pad = np.concatenate([np.zeros((1,) + q.shape[1:], np.float32), q, np.zeros((1,) + q.shape[1:], np.float32)])
    out, covered = paged_prefill_fp64(q_pad, k.numpy(), v.numpy(), case.prefill_tables, [4], qs, 16, case.scale)
    assert covered.tolist() == [False] + [True] * 6 + [False]
    assert np.isnan(out[0]).all() and np.isnan(out[7]).all()
    assert (out[1:3] == 0).all()
    rows = paged_prefill_by_decode(torch.from_numpy(q_pad), k, v, case.prefill_tables, [4], qs, 16, case.scale)
    assert sorted(rows) == [3, 4, 5, 6]
    for r, o in rows.items():
        assert np.abs(o.numpy() - out[r]).max() < 1e-5


def test_fp8_cache_rows_match_decode():
    from oracle import fp8

    case, k, v = _small_case(8, [12, 5], [20, 3], hq=4, hkv=2, d=32)
    kc, ks = fp8.quantize_per_head(k.numpy())
    vc, vs = fp8.quantize_per_head(v.numpy())
    k8 = torch.from_numpy(kc).view(torch.float8_e4m3fn)
    v8 = torch.from_numpy(vc).view(torch.float8_e4m3fn)
    q = case.q_prefill.float()
    ref, _ = paged_prefill_fp64(q.numpy(), fp8.decode(kc), fp8.decode(vc), case.prefill_tables,
                                case.prefill_lens, case.q_start, 16, case.scale, ks, vs)
    rows = paged_prefill_by_decode(q, k8, v8, case.prefill_tables, case.prefill_lens, case.q_start, 16, case.scale,
                                   torch.from_numpy(ks), torch.from_numpy(vs))
    got = np.stack([rows[i].numpy() for i in range(q.shape[0])])
    assert np.abs(got - ref).max() < 1e-5


def test_mixed_case_shapes():
    case = workloads.make_mixed_case(seed=0, device="meta")
    assert len(case.prefill_tables) == 8 and len(case.decode_tables) == 248
    assert case.q_prefill.shape == (8 * 512, 32, 128)
    assert len(case.slots) == 8 * 512 + 248
    assert len(set(case.slots)) == len(case.slots)
    for t, n in zip(case.prefill_tables + case.decode_tables, case.prefill_lens + case.decode_lens):
        assert len(t) == math.ceil(n / 16)
    alg = workloads.mixed_algorithmic(case)
    # expected magnitudes (decode reads ~2.2 GB; prefill ~155 GFLOP)
    assert 1.5e9 < alg["decode_bytes"] < 3e9
    assert 0.5e11 < alg["prefill_flops"] < 3e11
