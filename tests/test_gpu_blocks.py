"""GPU side of the block pool: device-resident tables, block copies and a
copy-on-write decode step through BlockManager + RadixCache + CacheManager.

Tables and copies are bit-exact against the host pool and the source
blocks; attention against the float64 oracle (tests/gpu_util.py bar).
"""

from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

from cf_hip import ops
from compiler.cache_policy import CachePolicy
from gpu_util import assert_close, codes
from oracle import fp8 as ofp8
from oracle.paged_attention import paged_attention_fp64
from python_runtime.engine import CacheManager, _KVCacheMixin
from python_runtime.engine.block_manager import BlockManager
from python_runtime.engine.cache import RadixCache

pytestmark = pytest.mark.gpu


def test_device_tables_follow_the_pool(gpu):
    rows, cols, bs = 16, 40, 16
    bm = BlockManager(512, bs)
    bm.bind_device(rows, cols, gpu)
    rng = random.Random(3)
    live: dict[str, int] = {}
    for step in range(80):
        if rng.random() < 0.3 and len(live) < rows:
            rid = f"q{step}"
            n = rng.randint(1, 200)
            bm.allocate(rid, n)
            bm.set_len(rid, n)
            live[rid] = n
        if rng.random() < 0.1 and live:
            rid = rng.choice(list(live))
            bm.free(rid)
            live.pop(rid)
        writes = [(rid, n, rng.randint(1, 3)) for rid, n in live.items() if rng.random() < 0.8]
        bm.prepare_writes(writes)
        for rid, n, c in writes:
            live[rid] = n + c
        tables, lens = bm.sync_device()
        if step % 10 == 9:
            t, l_ = tables.cpu().numpy(), lens.cpu().numpy()
            for rid, n in live.items():
                r = bm.row_of(rid)
                blocks = bm.get_blocks(rid)
                assert l_[r] == n
                np.testing.assert_array_equal(t[r, : len(blocks)], blocks)
                assert (t[r, len(blocks):] == -1).all()
            used = {bm.row_of(rid) for rid in live}
            assert all(l_[r] == 0 for r in range(rows) if r not in used)
            sp = bm.shared_prefix_lens().cpu().numpy()
            want = ops.shared_prefix_lens([t[r][t[r] >= 0].tolist() for r in range(rows)], l_.tolist(), bs)
            assert sp.tolist() == [int(x) for x in want]


@pytest.mark.parametrize("dtype", ["float8_e4m3fn", "bfloat16", "float64"])
def test_copy_blocks_slabs(gpu, dtype):
    """Whole-block copies over CacheManager slabs (K and V layouts, all
    layers): destinations equal their sources bit for bit, other blocks stay."""
    policy = CachePolicy.for_llama(3, 4, 32).to_dict()
    for slab in policy["slabs"]:
        slab["dtype"] = dtype
    mgr = CacheManager(policy, num_blocks=12, device=gpu)
    gen = torch.Generator(device=gpu).manual_seed(1)
    for t in mgr.paged_slabs():
        raw = t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t
        if t.dtype == torch.float8_e4m3fn:
            raw.copy_(torch.randint(0, 126, raw.shape, device=gpu, generator=gen, dtype=torch.uint8))
        else:
            raw.copy_(torch.randn(raw.shape, device=gpu, generator=gen, dtype=torch.float32).to(t.dtype))
    before = [t.detach().clone() for t in mgr.paged_slabs()]
    pairs = np.array([[3, 7], [0, 11], [5, 2]], dtype=np.int32)
    BlockManager.copy_blocks(pairs, mgr.paged_slabs())
    torch.cuda.synchronize()
    for t, b in zip(mgr.paged_slabs(), before):
        want = b.clone()
        for s, d in pairs:
            want[d] = b[s]
        tb = t.contiguous().view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t
        wb = want.contiguous().view(torch.uint8) if t.dtype == torch.float8_e4m3fn else want
        assert torch.equal(tb, wb)


def test_copy_blocks_mixin_cache(gpu):
    class _E(_KVCacheMixin):
        pass

    kv = _E().prepare_kv_blocks(2, 2, 8, 4, 6, dtype=torch.float16, device=gpu)
    kv.copy_(torch.randn(kv.shape, device=gpu).to(torch.float16))
    before = kv.clone()
    ops.copy_blocks(kv, torch.tensor([[1, 4]], dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    want = before.clone()
    want[4] = before[1]
    assert torch.equal(kv, want)


def _dense(kv_rows: dict[str, np.ndarray], order: list[str]):
    """Dense per-sequence caches for the oracle: one block table per
    sequence over its own rows."""
    bs = 16
    blocks, tables, lens = [], [], []
    for rid in order:
        x = kv_rows[rid]
        n = x.shape[0]
        nb = -(-n // bs)
        pad = np.zeros((nb * bs,) + x.shape[1:], x.dtype)
        pad[:n] = x
        tables.append(list(range(len(blocks), len(blocks) + nb)))
        blocks += list(pad.reshape(nb, bs, *x.shape[1:]))
        lens.append(n)
    return np.stack(blocks), tables, lens


def test_copy_on_write_decode_step(gpu):
    """A radix hit that ends inside a block: B shares A's partial block, B's
    first decode write copies it (A's rows stay A's), and attention of both
    requests over device tables matches the oracle on their own tokens."""
    L, hkv, g, d, bs = 2, 2, 4, 64, 16
    policy = CachePolicy.for_llama(L, hkv, d, kv_dtype="float8_e4m3fn")
    mgr = CacheManager(policy, num_blocks=32, device=gpu)
    bm = BlockManager(32, bs)
    bm.bind_device(4, 8, gpu)
    cache = RadixCache(bm)
    gen = torch.Generator().manual_seed(4)
    rows = {}  # (rid, layer, name) -> bf16 rows written, in position order

    def write(rid, start, x_by_layer):
        slots, copies = bm.prepare_writes([(rid, start, next(iter(x_by_layer.values())).shape[0])])
        BlockManager.copy_blocks(copies, mgr.paged_slabs())
        for (layer, name), x in x_by_layer.items():
            mgr.write_slots(name, layer, x.to(gpu), slots)
            prev = rows.get((rid, layer, name))
            rows[(rid, layer, name)] = x if prev is None else torch.cat([prev, x])
        return copies

    def fresh(n):
        return {(layer, name): torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
                for layer in range(L) for name in ("k", "v")}

    prompt = list(range(100, 120))  # 20 tokens: block 1 half full
    bm.allocate("A", 0)
    assert len(write("A", 0, fresh(20))) == 0
    cache.insert(prompt, bm.get_blocks("A"))
    hit, n = cache.match_prefix(prompt + [7])
    assert n == 20 and len(hit) == 2
    bm.assign_cached_blocks("B", hit)
    bm.set_len("B", 20)
    for key in list(rows):
        if key[0] == "A":
            rows[("B",) + key[1:]] = rows[key].clone()
    copies = write("B", 20, fresh(1))  # B's first decode token
    assert len(copies) == 1 and copies[0][0] == hit[1]
    write("A", 20, fresh(1))  # A decodes too: its block 1 is held by the radix cache -> copied as well
    tables, lens = bm.sync_device()
    assert lens.cpu().tolist()[: 2] == [21, 21]
    q = torch.randn(4, hkv * g, d, generator=gen).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    order = sorted(["A", "B"], key=bm.row_of)
    for layer in range(L):
        got = mgr.attend_rows(q.to(gpu), layer, tables, lens, bm.shared_prefix_lens()).float().cpu().numpy()
        ks = mgr.kv_scales("k")[layer].cpu().numpy()
        vs = mgr.kv_scales("v")[layer].cpu().numpy()

        def quant(x, sc):
            return ofp8.decode(ofp8.encode(x.float().numpy() / sc.reshape(1, -1, 1)))

        kd = {r: quant(rows[(r, layer, "k")], ks) for r in order}
        vd = {r: quant(rows[(r, layer, "v")], vs) for r in order}
        kc, tabs, lns = _dense(kd, order)
        vc, _, _ = _dense(vd, order)
        want = paged_attention_fp64(q[: len(order)].float().numpy()[[bm.row_of(r) for r in order]], kc, vc, tabs,
                                    lns, bs, scale, ks, vs)
        for i, r in enumerate(order):
            assert_close(got[bm.row_of(r)], want[i], torch.bfloat16, f"COW decode {r} layer {layer}")
        assert np.abs(got[2:]).max() == 0.0  # empty rows
    # A's and B's token-20 rows differ, so the copy kept them apart
    kb = mgr.layer_view("k", 0)
    a_blk, b_blk = bm.get_blocks("A")[1], bm.get_blocks("B")[1]
    assert a_blk != b_blk and not np.array_equal(codes(kb[a_blk, 4]), codes(kb[b_blk, 4]))
    assert np.array_equal(codes(kb[a_blk, :4]), codes(kb[b_blk, :4]))  # the shared prefix rows were copied


@pytest.mark.parametrize("dtype", ["float8_e4m3fn", "bfloat16"])
def test_prefill_chunks_from_slabs(gpu, dtype):
    """A chunked-prefill step through the block pool and CacheManager: two
    requests with cached prefixes (one shared through the radix cache) write
    their chunk's K/V at pool slots and attend from the slabs; the float64
    oracle runs on the slab contents."""
    from oracle.paged_attention import paged_prefill_fp64

    L, hkv, g, d, bs = 2, 2, 4, 128, 16
    mgr = CacheManager(CachePolicy.for_llama(L, hkv, d, kv_dtype=dtype), num_blocks=64, device=gpu)
    bm = BlockManager(64, bs)
    gen = torch.Generator().manual_seed(8)
    if dtype == "float8_e4m3fn":
        for name in ("k", "v"):
            # |x| stays under ~12 (N(0, 2) rows): codes of x / scale stay finite (< 448)
            mgr.set_kv_scales(name, torch.rand(L, hkv, generator=gen) * 0.02 + 0.05)

    def rows(n):
        return {(layer, name): (torch.randn(n, hkv, d, generator=gen) * 2).to(torch.bfloat16)
                for layer in range(L) for name in ("k", "v")}

    def write(writes, data):
        slots, copies = bm.prepare_writes(writes)
        BlockManager.copy_blocks(copies, mgr.paged_slabs())
        for (layer, name), x in data.items():
            mgr.write_slots(name, layer, x.to(gpu), slots)

    # cached prefixes: A 37 tokens; B shares A's first 21 tokens (a partial block)
    bm.allocate("A", 0)
    write([("A", 0, 37)], rows(37))
    bm.assign_cached_blocks("B", bm.get_blocks("A")[:2])
    # this step's chunks: A +50 rows at 37.., B +70 rows at 21..
    chunk = {"A": (37, 50), "B": (21, 70)}
    write([(r, s, n) for r, (s, n) in chunk.items()], rows(120))
    order = ["A", "B"]
    tabs = [bm.get_blocks(r) for r in order]
    width = max(len(t) for t in tabs)
    tables = torch.tensor([t + [-1] * (width - len(t)) for t in tabs], dtype=torch.int32, device=gpu)
    lens = torch.tensor([chunk[r][0] + chunk[r][1] for r in order], dtype=torch.int32, device=gpu)
    q_start = torch.tensor([0, 50, 120], dtype=torch.int32, device=gpu)
    q = torch.randn(120, hkv * g, d, generator=gen).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    for layer in range(L):
        got = mgr.attend_chunks(q.to(gpu), layer, tables, lens, q_start).float().cpu().numpy()
        kc, vc = mgr.layer_view("k", layer).detach().cpu(), mgr.layer_view("v", layer).detach().cpu()
        if dtype == "float8_e4m3fn":
            kf, vf = ofp8.decode(codes(kc)), ofp8.decode(codes(vc))
            ks, vs = mgr.kv_scales("k")[layer].cpu().numpy(), mgr.kv_scales("v")[layer].cpu().numpy()
        else:
            kf, vf, ks, vs = kc.float().numpy(), vc.float().numpy(), None, None
        want, covered = paged_prefill_fp64(q.float().numpy(), kf, vf, tabs, lens.cpu().tolist(), [0, 50, 120], bs,
                                           scale, ks, vs)
        assert covered.all()
        assert_close(got, want, torch.bfloat16, f"prefill from slabs {dtype} layer {layer}")
