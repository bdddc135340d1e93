"""Block pool (native), copy-on-write, device-row deltas and RadixCache, on the CPU.

The oracle (oracle/block_manager.py) is pinned by the reference's own
BlockManager tests (runtime/src/cache/block.rs:478-610) and by allocation
orders worked out by hand from block.rs (free list = stack of 0..n-1); the
native pool is then checked against the oracle on random operation
sequences.  RadixCache runs the reference's own test cases
(python_runtime/engine/tests/test_radix_cache.py) on this build's pool.
"""

from __future__ import annotations

import random

import numpy as np
import pytest

from cf_hip import ops
from oracle.block_manager import BlockManagerRef, OutOfBlocks
from python_runtime.engine.block_manager import BlockManager, PyBlockManager
from python_runtime.engine.cache import RadixCache


@pytest.fixture(params=["product", "oracle"])
def make(request):
    return BlockManager if request.param == "product" else BlockManagerRef


# ── the reference's BlockManager tests (block.rs:478-610), both sides ─


def test_reference_unit_cases(make):
    bm = make(1000, 16)
    assert bm.num_free_blocks() == 1000
    assert len(bm.allocate("req_1", 32)) == 2 and bm.num_free_blocks() == 998
    assert len(bm.allocate("b", 16)) == 1 and len(bm.allocate("c", 1)) == 1
    bm.free("req_1")
    assert bm.num_free_blocks() == 998  # 1000 - 2 - 1 - 1 + 2
    bm.free("nonexistent")
    assert bm.num_free_blocks() == 998
    with pytest.raises((RuntimeError, OutOfBlocks)):
        make(10, 16).allocate("req_1", 200)
    with pytest.raises(ValueError):
        make(0, 16)
    with pytest.raises(ValueError):
        make(100, 0)
    bm = make(1000, 16)
    src = bm.allocate("src", 64)
    shared = bm.share_prefix("src", "dst", 32)
    assert shared == src[:2] and bm.get_blocks("dst") == shared
    bm = make(1000, 16)
    bm.allocate("src", 32)
    bm.share_prefix("src", "dst", 16)
    bm.free("src")
    assert bm.num_free_blocks() == 999
    bm.free("dst")
    assert bm.num_free_blocks() == 1000
    bm = make(1000, 16)
    blocks = bm.allocate("req_1", 32)
    bm.free_block(blocks[0])
    assert bm.num_free_blocks() == 999
    bm = make(1000, 16)
    bm.assign_cached_blocks("req_1", [0, 1])
    assert bm.get_blocks("req_1") == [0, 1]
    with pytest.raises(KeyError):
        make(10, 16).get_blocks("unknown")


def test_allocation_order_known_answer(make):
    """Stack order from block.rs:145-173 / 177-196: pops 999, 998, ...;
    freed blocks come back last-in first-out."""
    bm = make(1000, 16)
    assert bm.allocate("a", 40) == [999, 998, 997]
    assert bm.allocate("b", 1) == [996]
    bm.free("a")  # pushes 999, 998, 997
    assert bm.allocate("c", 33) == [997, 998, 999]
    bm.ensure_blocks("b", 40)
    assert bm.get_blocks("b") == [996, 995, 994]
    bm.ensure_blocks("b", 10)  # already covered
    assert bm.get_blocks("b") == [996, 995, 994]


def test_utilization_and_properties():
    bm = PyBlockManager(100, 16)
    assert bm.block_size == 16 and bm.num_blocks == 100
    assert abs(bm.utilization()) < 1e-9
    bm.allocate("req_1", 160)
    assert abs(bm.utilization() - 0.1) < 1e-9
    with pytest.raises(RuntimeError):
        bm.allocate("req_1", 16)  # duplicate id
    with pytest.raises(ValueError):
        bm.share_prefix("missing", "x", 16)
    with pytest.raises(ValueError):
        bm.share_prefix("req_1", "y", 16 * 11)


def test_copy_on_write_known_answer(make):
    """The shared-partial-block hazard: B takes A's 20-token prefix (block 1
    half full, shared); B's write at position 20 must not land in A's
    block: B gets a fresh copy of it, A keeps its table."""
    bm = make(8, 16)
    a = bm.allocate("A", 20)  # [7, 6]
    assert a == [7, 6]
    bm.assign_cached_blocks("B", a)  # radix hit: both blocks now shared
    slots, copies = bm.prepare_writes([("B", 20, 1)])
    assert [tuple(c) for c in copies] == [(6, 5)]
    assert list(slots) == [5 * 16 + 4]
    assert bm.get_blocks("A") == [7, 6] and bm.get_blocks("B") == [7, 5]
    # a second write into the now-private block copies nothing
    slots, copies = bm.prepare_writes([("B", 21, 12)])
    assert len(copies) == 0 and list(slots) == [5 * 16 + p for p in range(5, 16)] + [4 * 16]
    assert bm.get_blocks("B") == [7, 5, 4]


def test_prepare_writes_all_or_nothing(make):
    bm = make(4, 16)
    bm.allocate("A", 16)
    before = bm.num_free_blocks()
    with pytest.raises((RuntimeError, OutOfBlocks)):
        bm.prepare_writes([("A", 16, 16), ("B", 0, 40)])  # needs 1 + 3 > 3
    assert bm.num_free_blocks() == before and bm.get_blocks("A") == [3]


def _random_ops(seed: int):
    rng = random.Random(seed)
    ops_ = []
    live: list[str] = []
    for k in range(300):
        r = rng.random()
        if r < 0.25 or not live:
            rid = f"r{k}"
            ops_.append(("allocate", rid, rng.randint(0, 70)))
            live.append(rid)
        elif r < 0.35:
            rid = live.pop(rng.randrange(len(live)))
            ops_.append(("free", rid))
        elif r < 0.45:
            ops_.append(("share_prefix", rng.choice(live), f"s{k}", rng.randint(0, 40)))
            live.append(f"s{k}")
        elif r < 0.55:
            ops_.append(("ensure_blocks", rng.choice(live), rng.randint(0, 90)))
        elif r < 0.6:
            ops_.append(("increment_ref_count", rng.randrange(64)))
        elif r < 0.65:
            ops_.append(("free_block", rng.randrange(64)))
        elif r < 0.7:
            ops_.append(("assign_cached_blocks", rng.choice(live), [rng.randrange(64) for _ in range(rng.randint(0, 3))]))
        else:
            ws = []
            for rid in rng.sample(live, min(len(live), rng.randint(1, 4))):
                ws.append((rid, rng.randint(0, 60), rng.randint(0, 20)))
            ops_.append(("prepare_writes", ws))
    return ops_


@pytest.mark.parametrize("seed", range(8))
def test_native_pool_matches_oracle(seed):
    a, b = BlockManager(64, 8), BlockManagerRef(64, 8)
    for op in _random_ops(seed):
        name, args = op[0], op[1:]
        res = []
        for bm in (a, b):
            try:
                out = getattr(bm, name)(*args)
                if name == "prepare_writes":
                    out = (list(map(int, out[0])), [tuple(map(int, c)) for c in out[1]])
                res.append(("ok", out))
            except (RuntimeError, OutOfBlocks, ValueError, KeyError) as e:
                res.append(("err", type(e) if not isinstance(e, OutOfBlocks) else RuntimeError))
        if res[0][0] == "err" and res[1][0] == "err":
            continue
        assert res[0] == res[1], (seed, op)
        assert a.num_free_blocks() == b.num_free_blocks(), (seed, op)
    for rid in b.tables:
        assert a.get_blocks(rid) == b.tables[rid]
    assert [a.ref_count(i) for i in range(64)] == b.rc


# ── device rows (host side) ────────────────────────────────────────────


def _apply(deltas: np.ndarray, table: np.ndarray, lens: np.ndarray) -> None:
    for r, c, v, _ in deltas:
        if c < 0:
            lens[r] = v
        else:
            table[r, c] = v


def test_table_deltas_track_tables():
    rows, cols = 6, 24
    bm = BlockManager(128, 4)
    bm.bind_rows(rows, cols)
    table = np.full((rows, cols), -1, np.int32)
    lens = np.zeros(rows, np.int32)
    rng = random.Random(5)
    live: dict[str, int] = {}
    for step in range(60):
        if rng.random() < 0.2 and len(live) < rows:
            rid = f"q{step}"
            bm.allocate(rid, rng.randint(1, 9))
            bm.set_len(rid, 0)
            live[rid] = 0
        if rng.random() < 0.1 and live:
            rid = rng.choice(list(live))
            bm.free(rid)
            live.pop(rid)
        writes = []
        for rid in live:
            if rng.random() < 0.7:
                writes.append((rid, live[rid], 1))
                live[rid] += 1
        bm.prepare_writes(writes)
        d = bm.table_deltas()
        _apply(d, table, lens)
        for rid, n in live.items():
            r = bm.row_of(rid)
            t = bm.get_blocks(rid)
            assert 0 <= r < rows and lens[r] == n
            np.testing.assert_array_equal(table[r, : len(t)], t)
            assert (table[r, len(t):] == -1).all()
        used = {bm.row_of(rid) for rid in live}
        assert all(lens[r] == 0 for r in range(rows) if r not in used)
        assert len(bm.table_deltas()) == 0  # nothing changed since
        sp = bm.shared_prefix_lens_host(rows)
        tabs = [table[r][table[r] >= 0].tolist() for r in range(rows)]
        want = ops.shared_prefix_lens(tabs, lens.tolist(), 4)
        assert sp.tolist() == [int(x) for x in want]


def test_table_deltas_errors():
    bm = BlockManager(64, 4)
    with pytest.raises(ValueError):
        bm.table_deltas()
    bm.bind_rows(1, 2)
    bm.allocate("a", 4)
    bm.allocate("b", 4)
    with pytest.raises(ValueError, match="rows exhausted"):
        bm.table_deltas()
    bm.free("b")
    bm.ensure_blocks("a", 12)
    with pytest.raises(ValueError, match="device rows hold"):
        bm.table_deltas()


# ── RadixCache: the reference's test cases on this pool ─────────────────


def _setup(num_blocks=100, block_size=4):
    bm = PyBlockManager(num_blocks, block_size)
    return bm, RadixCache(bm)


_n = [0]


def _alloc(bm, n_tokens):
    _n[0] += 1
    rid = f"__test_{_n[0]}"
    return bm.allocate(rid, n_tokens), rid


def test_radix_match_cases():
    bm, cache = _setup()
    assert cache.match_prefix([1, 2, 3]) == ([], 0)
    bm, cache = _setup(block_size=4)
    blks, _ = _alloc(bm, 3)
    cache.insert([1, 2, 3], blks)
    assert cache.match_prefix([1, 2, 3]) == (blks, 3)
    bm, cache = _setup(block_size=4)
    blks, _ = _alloc(bm, 8)
    cache.insert([1, 2, 3, 4, 5, 6, 7, 8], blks)
    assert cache.match_prefix([1, 2, 3, 4, 5, 6]) == (blks, 6)
    assert cache.match_prefix([1, 2]) == (blks[:1], 2)
    assert cache.match_prefix([9, 2, 3]) == ([], 0)
    bm, cache = _setup(block_size=8)
    b1, _ = _alloc(bm, 3)
    cache.insert([1, 2, 3], b1)
    b2, _ = _alloc(bm, 3)
    cache.insert([1, 4, 5], b2)
    assert cache.match_prefix([1, 2, 3]) == (b1, 3)
    assert cache.match_prefix([1, 4, 5]) == ([b1[0], b2[0]], 3)


def test_radix_insert_cases():
    bm, cache = _setup(block_size=4)
    blks, _ = _alloc(bm, 8)
    cache.insert([1, 2, 3, 4, 5, 6, 7, 8], blks)
    child = cache.root.children[1]
    assert child.token_ids == (1, 2, 3, 4, 5, 6, 7, 8) and child.kv_blocks == blks and child.ref_count == 1
    bm, cache = _setup()
    cache.insert([], [0])
    assert not cache.root.children
    bm, cache = _setup(block_size=4)
    b1, _ = _alloc(bm, 8)
    cache.insert([1, 2, 3, 4, 5, 6, 7, 8], b1)
    b2, _ = _alloc(bm, 6)
    cache.insert([1, 2, 3, 4, 9, 0], b2)
    child = cache.root.children[1]
    assert child.token_ids == (1, 2, 3, 4) and child.kv_blocks == b1[:1] and len(child.children) == 2
    bm, cache = _setup()
    b1, _ = _alloc(bm, 3)
    cache.insert([1, 2, 3], b1)
    b2, _ = _alloc(bm, 3)
    cache.insert([7, 8, 9], b2)
    assert len(cache.root.children) == 2
    bm, cache = _setup(block_size=4)
    b1, _ = _alloc(bm, 3)
    cache.insert([1, 2, 3], b1)
    b2, _ = _alloc(bm, 5)
    cache.insert([1, 2, 3, 4, 5], b2)
    assert cache.match_prefix([1, 2, 3, 4, 5])[1] == 5
    bm, cache = _setup(block_size=4)
    blks, rid = _alloc(bm, 4)
    assert bm.num_free_blocks() == 99
    cache.insert([1, 2, 3, 4], blks)
    bm.free(rid)
    assert bm.num_free_blocks() == 99


def test_radix_evict_cases():
    bm, cache = _setup(block_size=4)
    blks, rid = _alloc(bm, 4)
    cache.insert([1, 2, 3, 4], blks)
    bm.free(rid)
    assert bm.num_free_blocks() == 99
    cache.root.children[1].ref_count = 0
    assert cache.evict(2) == 1 and bm.num_free_blocks() == 100
    bm, cache = _setup(block_size=4)
    blks, _ = _alloc(bm, 4)
    cache.insert([1, 2, 3, 4], blks)
    assert cache.evict(2) == 0 and bm.num_free_blocks() == 99
    assert _setup()[1].evict(0) == 0
    bm, cache = _setup(block_size=4)
    b1, _ = _alloc(bm, 4)
    cache.insert([1, 2, 3, 4], b1)
    b2, _ = _alloc(bm, 4)
    cache.insert([5, 6, 7, 8], b2)
    cache.root.children[1].ref_count = 0
    assert cache.evict(10) == 1 and 1 not in cache.root.children and 5 in cache.root.children


def test_radix_block_manager_integration():
    bm, cache = _setup(block_size=8)
    blks, _ = _alloc(bm, 12)
    cache.insert([1, 2, 3, 4, 5, 6, 7, 8, 9, 0, 1, 2], blks)
    assert cache.match_prefix([1, 2, 3, 4]) == (blks[:1], 4)
    bm, cache = _setup(block_size=4)
    b1, _ = _alloc(bm, 8)
    cache.insert([1, 2, 3, 4, 5, 6, 7, 8], b1)
    b2, _ = _alloc(bm, 8)
    cache.insert([1, 2, 3, 4, 9, 0, 1, 2], b2)
    assert cache.root.children[1].kv_blocks == b1[:1] and len(cache.root.children[1].children) == 2
    bm = PyBlockManager(10, 4)
    blks = bm.allocate("req_a", 8)
    assert bm.num_free_blocks() == 8
    bm.free_block(blks[0])
    assert bm.num_free_blocks() == 9
    bm.free_block(blks[1])
    assert bm.num_free_blocks() == 10


def test_radix_partial_block_hit_is_copied_on_write():
    """A radix hit ending inside a block shares that partial block; the
    hitting request's first write copies it instead of writing into it."""
    bm, cache = _setup(num_blocks=16, block_size=4)
    a, rid_a = _alloc(bm, 6)  # tokens 0..5: block a[1] half full
    cache.insert([10, 11, 12, 13, 14, 15], a)
    blocks, n = cache.match_prefix([10, 11, 12, 13, 14, 15, 99])
    assert (blocks, n) == (a, 6)
    bm.assign_cached_blocks("B", blocks)
    slots, copies = bm.prepare_writes([("B", 6, 1)])
    assert [tuple(c) for c in copies] == [(a[1], bm.get_blocks("B")[1])]
    assert bm.get_blocks(rid_a) == a and bm.get_blocks("B")[0] == a[0]
    assert slots[0] == bm.get_blocks("B")[1] * 4 + 2


def test_prepare_writes_batch_equals_list_form():
    a, b = BlockManager(256, 8), BlockManager(256, 8)
    from python_runtime.engine.block_manager import RequestBatch

    for bm in (a, b):
        bm.allocate("x", 20)
        bm.allocate("y", 3)
        bm.share_prefix("x", "z", 12)
    writes = [("x", 20, 5), ("z", 12, 9), ("y", 3, 0), ("w", 0, 17)]
    s1, c1 = a.prepare_writes(writes)
    s2, c2 = b.prepare_writes_batch(RequestBatch([w[0] for w in writes]), np.array([w[1] for w in writes]),
                                    np.array([w[2] for w in writes]))
    assert s1.tolist() == s2.tolist() and c1.tolist() == c2.tolist()
    with pytest.raises(ValueError, match="listed twice"):
        a.prepare_writes([("x", 30, 1), ("x", 31, 1)])
    with pytest.raises(ValueError, match="listed twice"):
        a.prepare_writes([("new", 0, 1), ("new", 1, 1)])
    with pytest.raises(KeyError):
        a.set_len("nobody", 3)
