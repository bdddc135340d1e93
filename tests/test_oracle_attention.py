"""Pins the CPU attention oracle (oracle/paged_attention.py).

The torch-SDPA restatement of the reference's _paged_attention_cpu
(kernels/paged_attention.py:21-73) is checked against an independent
float64 brute force and against closed forms and invariants chosen so that
plausible mistakes fail: a dropped softmax denominator (mean-of-V case), a
wrong GQA head mapping (GQA vs repeated-MHA case), a wrong block order or
offset (permutation and shared-prefix cases), wrong truncation (seq_len
rules).  The reference's own TestPagedAttention cases
(python_runtime/hal/tests/test_triton_kernels.py:166-269) run on it too.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import workloads
from oracle.paged_attention import paged_attention_cpu, paged_attention_fp64


def _dicts(case):
    rids = [f"req_{i}" for i in range(case.batch)]
    return dict(zip(rids, case.block_tables)), dict(zip(rids, case.seq_lens))


def _stack(outs: dict) -> np.ndarray:
    return torch.stack(list(outs.values())).float().numpy()


def _cos(a, b):
    a, b = np.ravel(a).astype(np.float64), np.ravel(b).astype(np.float64)
    return float(a @ b / math.sqrt((a @ a) * (b @ b)))


@pytest.mark.parametrize("config,batch", [("c1_opt125m", None), ("c2_tinyllama", 3)])
def test_restatement_matches_fp64(config, batch):
    case = workloads.make_case(config, seed=11, batch=batch)
    bt, sl = _dicts(case)
    got = _stack(paged_attention_cpu(case.q, case.k, case.v, bt, sl, case.block_size, case.scale))
    ref = paged_attention_fp64(case.q.float().numpy(), case.k.float().numpy(), case.v.float().numpy(),
                               case.block_tables, case.seq_lens, case.block_size, case.scale)
    tol = 1e-5 if case.q.dtype == torch.float32 else 2e-2
    assert np.abs(got - ref).max() < tol


def test_fp8_restatement_matches_fp64():
    from oracle import fp8

    case = workloads.make_case("c3_llama3_8b", seed=2, batch=2)
    kc, ks = fp8.quantize_per_head(case.k.float().numpy())
    vc, vs = fp8.quantize_per_head(case.v.float().numpy())
    k8 = torch.from_numpy(kc).view(torch.float8_e4m3fn)
    v8 = torch.from_numpy(vc).view(torch.float8_e4m3fn)
    bt, sl = _dicts(case)
    got = _stack(paged_attention_cpu(case.q, k8, v8, bt, sl, 16, case.scale, torch.from_numpy(ks),
                                     torch.from_numpy(vs)))
    ref = paged_attention_fp64(case.q.float().numpy(), fp8.decode(kc), fp8.decode(vc), case.block_tables,
                               case.seq_lens, 16, case.scale, ks, vs)
    assert np.abs(got - ref).max() < 1e-4


def test_identical_keys_give_mean_of_values():
    """Equal scores -> uniform softmax -> output = mean of the V rows."""
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 1, 2, 8, generator=g).expand(4, 16, 2, 8).contiguous()
    v = torch.randn(4, 16, 2, 8, generator=g)
    q = torch.randn(1, 4, 8, generator=g)
    bt, sl = {"a": [2, 0, 3]}, {"a": 37}
    out = paged_attention_cpu(q, k, v, bt, sl, 16)["a"]
    rows = torch.cat([v[2], v[0], v[3]])[:37]  # [37, 2, 8]
    want = rows.mean(0).repeat_interleave(2, dim=0)
    assert torch.allclose(out, want, atol=1e-6)
    ref = paged_attention_fp64(q.numpy(), k.numpy(), v.numpy(), [[2, 0, 3]], [37], 16, 1 / math.sqrt(8))
    assert np.abs(ref[0] - want.numpy()).max() < 1e-6


def test_single_token_returns_its_value_row():
    g = torch.Generator().manual_seed(1)
    k, v = torch.randn(3, 16, 2, 8, generator=g), torch.randn(3, 16, 2, 8, generator=g)
    q = torch.randn(1, 2, 8, generator=g)
    out = paged_attention_cpu(q, k, v, {"a": [1]}, {"a": 1}, 16)["a"]
    assert torch.allclose(out, v[1, 0], atol=1e-6)


def test_block_permutation_invariance():
    case = workloads.make_case("c1_opt125m", seed=4)
    perm = torch.randperm(case.k.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    k2, v2 = case.k[perm], case.v[perm]  # block j of the new pool is old block perm[j]
    tables2 = [[int(inv[b]) for b in t] for t in case.block_tables]
    a = paged_attention_fp64(case.q.numpy(), case.k.numpy(), case.v.numpy(), case.block_tables, case.seq_lens, 16,
                             case.scale)
    b = paged_attention_fp64(case.q.numpy(), k2.numpy(), v2.numpy(), tables2, case.seq_lens, 16, case.scale)
    assert np.abs(a - b).max() < 1e-12


def test_gqa_equals_mha_with_repeated_heads():
    case = workloads.make_case("c2_tinyllama", seed=5, batch=2)
    bt, sl = _dicts(case)
    g = case.q.shape[1] // case.k.shape[2]
    k_rep = case.k.repeat_interleave(g, dim=2)
    v_rep = case.v.repeat_interleave(g, dim=2)
    a = _stack(paged_attention_cpu(case.q.float(), case.k.float(), case.v.float(), bt, sl, 16, case.scale))
    b = _stack(paged_attention_cpu(case.q.float(), k_rep.float(), v_rep.float(), bt, sl, 16, case.scale))
    assert np.abs(a - b).max() < 1e-6
    # and a wrong mapping (h % Hkv instead of h // G) would differ
    idx = torch.arange(case.q.shape[1]) % case.k.shape[2]
    c = _stack(paged_attention_cpu(case.q.float(), case.k.float()[:, :, idx], case.v.float()[:, :, idx], bt, sl,
                                   16, case.scale))
    assert np.abs(a - c).max() > 1e-2


def test_shared_prefix_equals_copied_prefix():
    case = workloads.make_case("c3_llama3_8b", seed=6, batch=4)
    pre = case.meta["shared_prefix_blocks"]
    shared = case.block_tables[0][:pre]
    assert case.block_tables[1][:pre] == shared
    nb = case.k.shape[0]
    k2 = torch.cat([case.k, case.k[shared]])
    v2 = torch.cat([case.v, case.v[shared]])
    tables2 = [list(t) for t in case.block_tables]
    tables2[1][:pre] = list(range(nb, nb + pre))
    q = case.q.float().numpy()
    a = paged_attention_fp64(q, case.k.float().numpy(), case.v.float().numpy(), case.block_tables, case.seq_lens,
                             16, case.scale)
    b = paged_attention_fp64(q, k2.float().numpy(), v2.float().numpy(), tables2, case.seq_lens, 16, case.scale)
    assert np.abs(a - b).max() == 0.0


def test_length_rules():
    g = torch.Generator().manual_seed(8)
    k, v = torch.randn(6, 16, 2, 8, generator=g), torch.randn(6, 16, 2, 8, generator=g)
    q = torch.randn(3, 2, 8, generator=g)
    bt = {"a": [4, 1], "b": [0, 5, 2], "c": [3]}
    # "a": missing length -> whole table; "b": 200 > capacity -> 48; "c": 5
    out = paged_attention_cpu(q, k, v, bt, {"b": 200, "c": 5}, 16)
    ref = paged_attention_fp64(q.numpy(), k.numpy(), v.numpy(), [[4, 1], [0, 5, 2], [3]], [32, 48, 5], 16,
                               1 / math.sqrt(8))
    assert np.abs(_stack(out) - ref).max() < 1e-5


# The reference's TestPagedAttention cases, run on the restatement.
def test_reference_single_request_case():
    torch.manual_seed(42)
    q = torch.randn(1, 4, 32)
    k, v = torch.randn(4, 16, 4, 32), torch.randn(4, 16, 4, 32)
    out = paged_attention_cpu(q, k, v, {"req_1": [0, 1]}, {"req_1": 30}, 16)
    assert out["req_1"].shape == (4, 32)


def test_reference_gqa_case():
    torch.manual_seed(42)
    q = torch.randn(1, 8, 32)
    k, v = torch.randn(4, 16, 2, 32), torch.randn(4, 16, 2, 32)
    out = paged_attention_cpu(q, k, v, {"req_1": [0, 1, 2]}, {"req_1": 40}, 16)
    assert out["req_1"].shape == (8, 32)


def test_reference_matches_manual_gather_case():
    torch.manual_seed(42)
    k, v = torch.randn(4, 16, 4, 32), torch.randn(4, 16, 4, 32)
    q = torch.randn(1, 4, 32)
    out = paged_attention_cpu(q, k, v, {"req_1": [0, 1]}, {"req_1": 20}, 16)
    ks = torch.cat([k[0][:16], k[1][:4]]).unsqueeze(0).transpose(1, 2)
    vs = torch.cat([v[0][:16], v[1][:4]]).unsqueeze(0).transpose(1, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(2), ks, vs).squeeze(2)
    assert _cos(out["req_1"].numpy(), ref[0].numpy()) >= 0.999


def test_reference_multiple_requests_case():
    torch.manual_seed(42)
    q = torch.randn(2, 4, 32)
    k, v = torch.randn(8, 16, 4, 32), torch.randn(8, 16, 4, 32)
    out = paged_attention_cpu(q, k, v, {"req_1": [0, 1], "req_2": [2, 3]}, {"req_1": 20, "req_2": 30}, 16)
    assert set(out) == {"req_1", "req_2"}
