"""GPU parity of decode with shared-prefix groups (radix-cache blocks).

A statement of which sequences share leading blocks changes only how the
MFMA decode reads them (once per group of up to 16/G sharers), never the
result: every case is checked against the float64 oracle on the exact
cache contents, and against the same call without the statement.
Tolerances as elsewhere: bf16 outputs cosine >= 0.9999 and each element
within 2e-2 of the exact value rounded to bf16.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import ops, workloads
from kernels.paged_attention import paged_attention, paged_attention_tensors
from tests.gpu_util import assert_close, metrics, oracle_decode

pytestmark = pytest.mark.gpu

BS = 16


def _radix_tables(groups, seed):
    """groups: list of (shared_tokens, [lengths]).  Members of a group share
    the blocks of their first `shared_tokens` tokens (whole blocks); a
    nested group is written as (outer, [(inner, [lengths]), ...]).  Returns
    (tables, lens, pool size)."""
    rng = np.random.default_rng(seed)
    tables, lens = [], []
    counter = [0]

    def fresh(n):
        ids = list(range(counter[0], counter[0] + n))
        counter[0] += n
        return ids

    def emit(prefix_blocks, members):
        for m in members:
            if isinstance(m, tuple):
                inner, sub = m
                nb = (inner + BS - 1) // BS
                emit(prefix_blocks + fresh(nb - len(prefix_blocks)), sub)
            else:
                need = (m + BS - 1) // BS
                own = prefix_blocks[:need]
                tables.append(own + fresh(need - len(own)))
                lens.append(m)

    for shared, members in groups:
        emit(fresh((shared + BS - 1) // BS) if shared else [], members)
    pool = counter[0]
    perm = rng.permutation(pool + 5).tolist()  # scatter physical ids
    return [[perm[b] for b in t] for t in tables], lens, pool + 5


GROUPS = [
    (1024, [1024 + 5, 2000, 1030, 4096, 1024, 3000, 1100, 1500, 1999]),  # 9 sharers: several groups of 16/G
    (512 + 7, [600, 519, 800]),  # shared length not a multiple of 32: whole tiles only
    (0, [333]),
    (96, [96, 97, 128, 96]),  # members whose tokens all lie in the prefix
    (40, [100, 200]),  # fewer than 2 shared tiles: no group
    (1024, [(2048, [2100, 2500, 3000]), 1100, (1536, [1600, 1700])]),  # nested prefixes
    (64, [64]),
]


def _case(gpu, hq, hkv, d, kv_dtype, seed, groups=GROUPS):
    tables, lens, nb = _radix_tables(groups, seed)
    g = torch.Generator(device=gpu).manual_seed(seed)
    b = len(tables)
    q = torch.randn(b, hq, d, generator=g, device=gpu).to(torch.bfloat16)
    ksrc = torch.randn(nb, BS, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    vsrc = torch.randn(nb, BS, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    return workloads.DecodeCase("radix", q, ksrc, vsrc, tables, lens, BS, 1 / math.sqrt(d), kv_dtype)


def _decode(case, kc, vc, ks, vs, gpu, shared=None, workspace=None):
    sh = None if shared is None else torch.tensor(shared, dtype=torch.int32, device=gpu)
    out = paged_attention_tensors(case.q, kc, vc, case.tables_tensor(gpu), case.seq_lens_tensor(gpu), BS,
                                  case.scale, k_scale=ks, v_scale=vs, shared_prefix_lens=sh, workspace=workspace)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 8, 128), (32, 4, 64), (64, 8, 128),
                                      (16, 1, 128)])
@pytest.mark.parametrize("kv_dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_radix_groups_match_oracle(gpu, hq, hkv, d, kv_dtype):
    print(f"[case] radix groups hq={hq} hkv={hkv} d={d} kv={kv_dtype}", flush=True)
    case = _case(gpu, hq, hkv, d, kv_dtype, seed=hq + hkv + d)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    shared = ops.shared_prefix_lens(case.block_tables, case.seq_lens, BS)
    assert sum(s >= 64 for s in shared) >= 10  # the groups above do share
    out = _decode(case, kc, vc, ks, vs, gpu, shared)
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, f"radix {hq}/{hkv}/{d}")
    plain = _decode(case, kc, vc, ks, vs, gpu)
    err, cos = metrics(out.float().cpu().numpy(), plain.float().cpu().numpy())
    assert err <= 2e-2 and cos >= 0.99999, (err, cos)


def test_understated_shares_are_still_exact(gpu):
    """Stating less sharing than the tables have (or none) changes nothing."""
    case = _case(gpu, 32, 8, 128, torch.float8_e4m3fn, seed=5)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    full = ops.shared_prefix_lens(case.block_tables, case.seq_lens, BS)
    ref = oracle_decode(case, kc, vc, ks, vs)
    for shared in ([s // 2 for s in full], [min(s, 100) for s in full], [0] * len(full), [-5] * len(full)):
        out = _decode(case, kc, vc, ks, vs, gpu, shared)
        assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "understated")


@pytest.mark.parametrize("kv_dtype", [torch.float8_e4m3fn, torch.bfloat16])
def test_long_shared_prefix_split_over_many_waves(gpu, kv_dtype):
    """A 30000-token prefix shared by 3 sequences: the prefix run and the
    own runs are split over many waves, the merge combines both kinds."""
    print(f"[case] long shared prefix kv={kv_dtype}", flush=True)
    case = _case(gpu, 32, 8, 128, kv_dtype, seed=8, groups=[(30000, [30000, 30100, 31000]), (0, [500])])
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _decode(case, kc, vc, ks, vs, gpu, ops.shared_prefix_lens(case.block_tables, case.seq_lens, BS))
    ref = oracle_decode(case, kc, vc, ks, vs)
    assert_close(out.float().cpu().numpy(), ref, torch.bfloat16, "long shared prefix")


def test_full_c3_with_shared_prefix_statement(gpu):
    """Headline config: the 32 sequences on the shared 1024-token prefix run
    in groups; results agree with the ungrouped call and the oracle."""
    print("[case] c3 full size, shared-prefix statement", flush=True)
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=0)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    shared = ops.shared_prefix_lens(case.block_tables, case.seq_lens, BS)
    assert shared[1:32] == [1024] * 31 and not any(shared[32:])
    out = _decode(case, kc, vc, ks, vs, gpu, shared)
    plain = _decode(case, kc, vc, ks, vs, gpu)
    err, cos = metrics(out.float().cpu().numpy(), plain.float().cpu().numpy())
    assert err <= 2e-2 and cos >= 0.99999, (err, cos)
    idx = [0, 1, 2, 3, 4, 5, 30, 31, 32, 63]
    sub = workloads.DecodeCase("c3_sample", case.q[idx], case.k, case.v, [case.block_tables[i] for i in idx],
                               [case.seq_lens[i] for i in idx], BS, case.scale, case.kv_dtype)
    ref = oracle_decode(sub, kc, vc, ks, vs)
    assert_close(out[idx].float().cpu().numpy(), ref, torch.bfloat16, "c3 sample (grouped)")


def test_dict_api_groups_shared_blocks(gpu):
    """The dict API states the sharing its tables have; results match the
    oracle with prefixes shared between neighbouring requests."""
    case = _case(gpu, 32, 8, 128, torch.float8_e4m3fn, seed=11)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    rids = [f"req{i}" for i in range(case.batch)]
    out = paged_attention(case.q, kc, vc, dict(zip(rids, case.block_tables)), dict(zip(rids, case.seq_lens)),
                          block_size=BS, k_scale=ks, v_scale=vs)
    got = torch.stack([out[r] for r in rids]).float().cpu().numpy()
    assert_close(got, oracle_decode(case, kc, vc, ks, vs), torch.bfloat16, "dict api grouped")


def test_workspace_reuse_between_grouped_and_plain_calls(gpu):
    """Merge descriptors are rewritten by every call: grouped, plain and
    smaller calls on one workspace stay exact."""
    case = _case(gpu, 32, 8, 128, torch.float8_e4m3fn, seed=12)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    tables, lens = case.tables_tensor(gpu), case.seq_lens_tensor(gpu)
    need = ops.decode_workspace_bytes(case.batch, 32, 8, 128, tables.shape[1], BS)
    ws = ops.new_workspace(need, gpu)
    shared = ops.shared_prefix_lens(case.block_tables, case.seq_lens, BS)
    ref = oracle_decode(case, kc, vc, ks, vs)
    sh = torch.tensor(shared, dtype=torch.int32, device=gpu)
    outs = []
    for i in range(3):
        outs.append(ops.paged_decode(case.q, kc, vc, tables, lens, case.scale, BS, ks, vs, workspace=ws,
                                     shared_prefix_lens=sh).clone())
        ops.paged_decode(case.q[:4], kc, vc, tables[:4], lens[:4], case.scale, BS, ks, vs, workspace=ws,
                         shared_prefix_lens=sh[:4])
        ops.paged_decode(case.q, kc, vc, tables, lens, case.scale, BS, ks, vs, workspace=ws)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert_close(outs[0].float().cpu().numpy(), ref, torch.bfloat16, "workspace reuse")


def test_batches_above_the_plan_limit(gpu):
    """2100 sequences (above the 2048 the in-LDS plan holds): the statement is
    ignored and the ungrouped walk runs."""
    print("[case] batch 2100", flush=True)
    rng = np.random.default_rng(4)
    b, hq, hkv, d = 2100, 8, 2, 64
    lens = rng.integers(1, 80, size=b).tolist()
    nb = sum((n + BS - 1) // BS for n in lens) + 2
    perm = rng.permutation(nb).tolist()
    tables, pos = [], 0
    for n in lens:
        k = (n + BS - 1) // BS
        tables.append(perm[pos:pos + k])
        pos += k
    g = torch.Generator(device=gpu).manual_seed(4)
    q = torch.randn(b, hq, d, generator=g, device=gpu).to(torch.bfloat16)
    ksrc = torch.randn(nb, BS, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    vsrc = torch.randn(nb, BS, hkv, d, generator=g, device=gpu).to(torch.bfloat16)
    case = workloads.DecodeCase("wide", q, ksrc, vsrc, tables, lens, BS, 1 / math.sqrt(d), torch.float8_e4m3fn)
    kc, vc, ks, vs = workloads.materialize(case, "native")
    out = _decode(case, kc, vc, ks, vs, gpu, [64] * b)
    assert_close(out.float().cpu().numpy(), oracle_decode(case, kc, vc, ks, vs), torch.bfloat16, "batch 2100")
