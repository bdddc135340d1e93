"""Host logic of the engine-side KV cache (CacheManager, _KVCacheMixin) on the CPU.

Pins the oracle of the reference's paged write/read semantics
(oracle/cache_manager.py) with known answers worked out by hand from the
reference's code and its own tests (python_runtime/engine/tests/
test_cache_manager.py:106-183, test_mlir_executor.py:74-110), then checks
the product's host-side addressing (slot resolution, sorted tables,
operand normalization, policy parsing, slab shapes) against that oracle.
No kernel runs here: I/O on a CPU slab must raise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cache_manager as ocm
from oracle import fp8 as ofp8
from python_runtime.engine import CacheManager, _dict_to_proto_cache_policy, _KVCacheMixin, _normalize_kv_for_cache
from python_runtime.engine.cache_manager import (
    first_cover_table,
    normalize_kv,
    resolve_slots,
    slots_for_positions,
    sorted_table_matrix,
)


def _policy(layers=4, heads=8, dim=64, dtype="float32", block_size=16):
    return {
        "slabs": [
            {"slab_id": "k", "storage": "paged", "dims": {"layers": layers, "heads": heads, "dim": dim},
             "layout": "BNLD", "dtype": dtype},
            {"slab_id": "v", "storage": "paged", "dims": {"layers": layers, "heads": heads, "dim": dim},
             "layout": "BNLD", "dtype": dtype},
        ],
        "intercepts": [
            {"slab_id": "k", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[1]", "layer": "sequential", "func_index": 3, "output_index": 1},
            {"slab_id": "v", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[2]", "layer": "sequential"},
        ],
        "block_size": block_size,
        "max_requests": 256,
    }


# ── oracle pins (known answers) ───────────────────────────────────────


def test_oracle_roundtrip_single_request():
    """Reference test_write_read_roundtrip / test_block_boundary: positions
    0..n-1 of one request read back unchanged."""
    rng = np.random.default_rng(0)
    slab = np.zeros((16, 4, 16, 8, 64), np.float32)
    data = rng.standard_normal((32, 8, 64)).astype(np.float32)
    ocm.write_paged(slab, 0, data, list(range(32)), {"r0": [0, 1]})
    got = ocm.read_paged(slab, 0, 32, {"r0": [0, 1]})
    assert got.shape == (1, 32, 8, 64)
    np.testing.assert_array_equal(got[0], data)
    np.testing.assert_array_equal(slab[0, 0], data[:16])
    np.testing.assert_array_equal(slab[1, 0], data[16:])


def test_oracle_layer_isolation():
    """Reference test_layer_isolation."""
    slab = np.zeros((16, 4, 16, 8, 64), np.float32)
    ocm.write_paged(slab, 0, np.ones((1, 8, 64)), [0], {"r0": [0]})
    ocm.write_paged(slab, 1, 2 * np.ones((1, 8, 64)), [0], {"r0": [0]})
    np.testing.assert_array_equal(ocm.read_paged(slab, 0, 1, {"r0": [0]}), np.ones((1, 1, 8, 64)))
    np.testing.assert_array_equal(ocm.read_paged(slab, 1, 1, {"r0": [0]}), 2 * np.ones((1, 1, 8, 64)))


def test_oracle_multi_request_first_cover_rule():
    """Reference test_multi_request, with every cell's answer: positions go to
    the first table covering their block (r0 for blocks 0 and 1), so r1's
    block (physical 2) stays zero and r1 reads zeros past its table."""
    rng = np.random.default_rng(1)
    slab = np.zeros((16, 1, 16, 2, 4), np.float32)
    bt = {"r0": [0, 1], "r1": [2]}
    k0 = rng.standard_normal((16, 2, 4)).astype(np.float32)
    k1 = rng.standard_normal((1, 2, 4)).astype(np.float32)
    ocm.write_paged(slab, 0, k0, list(range(16)), bt)
    ocm.write_paged(slab, 0, k1, [16], bt)
    got = ocm.read_paged(slab, 0, 17, bt)
    np.testing.assert_array_equal(got[0, :16], k0)
    np.testing.assert_array_equal(got[0, 16], k1[0])
    np.testing.assert_array_equal(got[1], 0.0)
    np.testing.assert_array_equal(slab[2], 0.0)
    np.testing.assert_array_equal(slab[1, 0, 0], k1[0])


def test_oracle_cover_order_and_read_order():
    """Iteration order picks the writer, sorted ids pick the read order:
    tables {"b": [5], "a": [7, 8]} send block 0 to b's 5 and block 1 to a's
    8; a reads first."""
    assert ocm.write_slots({"b": [5], "a": [7, 8]}, [3, 20, 40], 16, 10) == [5 * 16 + 3, 8 * 16 + 4, -1]
    slab = np.zeros((10, 1, 16, 1, 1), np.float32)
    slab[5, 0, :, 0, 0] = 1.0
    slab[7, 0, :, 0, 0] = 2.0
    got = ocm.read_paged(slab, 0, 16, {"b": [5], "a": [7, 8]})
    np.testing.assert_array_equal(got[:, :, 0, 0], [[2.0] * 16, [1.0] * 16])


def test_oracle_negative_ids_wrap_and_bad_ids_raise():
    assert ocm.write_slots({"r": [-1]}, [2], 4, 6) == [5 * 4 + 2]
    with pytest.raises(IndexError):
        ocm.write_slots({"r": [6]}, [0], 4, 6)


def test_oracle_read_truncates_and_pads():
    """max_seq_len shorter than the table stops mid-block; longer pads zeros."""
    slab = np.arange(4 * 1 * 4 * 1 * 1, dtype=np.float32).reshape(4, 1, 4, 1, 1) + 1
    got = ocm.read_paged(slab, 0, 6, {"r": [2, 0]})[0, :, 0, 0]
    np.testing.assert_array_equal(got, [9, 10, 11, 12, 1, 2])
    got = ocm.read_paged(slab, 0, 10, {"r": [3]})[0, :, 0, 0]
    np.testing.assert_array_equal(got, [13, 14, 15, 16, 0, 0, 0, 0, 0, 0])


def test_oracle_fp8_slab_is_quantizer_roundtrip():
    """FP8 slab rows equal FP8KVCacheQuantizer's quantize -> dequantize per
    head (the pinned fp8 oracle), not a re-derivation."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((5, 3, 16)) * 5).astype(np.float32)
    scale = np.array([0.05, 0.5, 2.0], np.float32)
    slab = np.zeros((4, 1, 8, 3, 16), np.uint8)
    ocm.write_paged(slab, 0, x, list(range(5)), {"r": [1]}, scale=scale)
    got = ocm.read_paged(slab, 0, 5, {"r": [1]}, scale=scale)[0]
    for h in range(3):
        want = ofp8.dequantize(ofp8.quantize(x[:, h], float(scale[h])), float(scale[h]))
        np.testing.assert_array_equal(got[:, h], want)


def test_oracle_later_row_wins():
    slab = np.zeros((2, 1, 4, 1, 1), np.float32)
    ocm.write_paged(slab, 0, np.array([1.0, 2.0]).reshape(2, 1, 1), [1, 1], {"r": [0]})
    assert slab[0, 0, 1, 0, 0] == 2.0


# ── product host logic vs the oracle ──────────────────────────────────


def _random_tables(rng, n_req, nb, max_blocks):
    ids = rng.permutation(nb)
    tables, at = {}, 0
    for r in range(n_req):
        n = int(rng.integers(0, max_blocks + 1))
        tables[f"req{rng.integers(1000):03d}_{r}"] = [int(x) for x in ids[at: at + n]]
        at += n
    return tables


@pytest.mark.parametrize("seed", range(6))
def test_slots_match_oracle(seed):
    rng = np.random.default_rng(seed)
    nb, bs = 64, 16
    bt = _random_tables(rng, int(rng.integers(1, 6)), nb, 8)
    if seed % 2:  # overlapping tables: shared prefix blocks, as a radix cache gives
        first = next(iter(bt.values()), [])
        for k in list(bt)[1:]:
            bt[k] = first[:2] + bt[k]
    pos = rng.integers(0, 9 * bs, size=40)
    cover = first_cover_table(bt, nb)
    got = slots_for_positions(cover, pos, bs)
    want = ocm.write_slots(bt, [int(p) for p in pos], bs, nb)
    np.testing.assert_array_equal(got, want)


def test_resolve_slots_dedups_and_rejects_negative():
    bt = {"r": [3, 1]}
    cover = first_cover_table(bt, 4)
    s = resolve_slots(bt, cover, torch.tensor([0, 5, 0, 40]), 4, torch.device("cpu"))
    assert s.tolist()[1:] == [1 * 4 + 1, 3 * 4 + 0, -1] and s[0] < 0
    with pytest.raises(ValueError):
        resolve_slots(bt, cover, torch.tensor([-1]), 4, torch.device("cpu"))


def test_first_cover_table_checks_ids():
    with pytest.raises(IndexError):
        first_cover_table({"r": [0, 9]}, 8)
    np.testing.assert_array_equal(first_cover_table({"a": [1], "b": [2, -1]}, 8), [1, 7])


def test_sorted_table_matrix():
    ids, mat = sorted_table_matrix({"b": [4, 5, 6], "a": [-2], "c": []}, 8)
    assert ids == ["a", "b", "c"]
    np.testing.assert_array_equal(mat, [[6, -1, -1], [4, 5, 6], [-1, -1, -1]])
    assert mat.dtype == np.int32


@pytest.mark.parametrize(
    "shape", [(1, 8, 4, 64), (1, 4, 8, 64), (4, 8, 64), (8, 4, 64), (4, 512), (1, 4, 512)]
)
def test_normalize_kv_formats(shape):
    """The reference's accepted SDPA operand formats (test_cache_manager.py:57-94)."""
    x = torch.randn(*shape, dtype=torch.bfloat16)
    y = normalize_kv(x, 8, 64)
    assert y.shape == (4, 8, 64) and y.dtype == torch.bfloat16
    if shape == (1, 8, 4, 64):
        assert torch.equal(y, x[0].permute(1, 0, 2))
    k, v = _normalize_kv_for_cache(x, x, 8, 64)
    assert torch.equal(k, y) and torch.equal(v, y)


def test_policy_from_dict():
    pol = _dict_to_proto_cache_policy(_policy(dtype="float8_e4m3fn", block_size=16))
    assert pol.block_size == 16 and pol.max_requests == 256
    assert [s.name for s in pol.slabs] == ["k", "v"]
    assert pol.slabs[0].num_layers == 4 and pol.slabs[0].num_heads == 8 and pol.slabs[0].head_dim == 64
    assert list(pol.intercepts[0].param_indices) == [3, 1] and list(pol.intercepts[1].param_indices) == []
    assert pol.intercepts[1].source == "operand[2]"


def test_manager_slab_shapes_and_layouts_cpu():
    """Logical shapes are the reference's (test_slab_shape); storage is
    head-major for keys and channel-major for values."""
    mgr = CacheManager(_policy(4, 8, 64), num_blocks=10, device="cpu")
    k, v = mgr._slabs["k"], mgr._slabs["v"]
    assert k.shape == (10, 4, 16, 8, 64) and v.shape == (10, 4, 16, 8, 64)
    kl, vl = mgr.layer_view("k", 1), mgr.layer_view("v", 1)
    assert kl.shape == (10, 16, 8, 64) and kl.stride()[1:] == (64, 16 * 64, 1)
    assert vl.stride()[1:] == (1, 64 * 16, 16)
    fixed = CacheManager(
        {"slabs": [{"slab_id": "state", "storage": "fixed", "dims": {"layers": 4, "dim": 1024}}],
         "intercepts": [], "max_requests": 256},
        num_blocks=1, device="cpu",
    )
    assert fixed._slabs["state"].shape == (256, 4, 1024)
    data = torch.randn(1024)
    fixed.write_fixed("state", 0, 0, data)
    assert torch.equal(fixed.read_fixed("state", 0, 0), data)
    assert not fixed.has_paged_cache and mgr.has_paged_cache
    assert (mgr.configured_kv_heads(), mgr.configured_head_dim(), mgr.configured_num_layers()) == (8, 64, 4)


def test_manager_fp8_scales_cpu():
    mgr = CacheManager(_policy(2, 4, 16, dtype="float8_e4m3fn"), num_blocks=4, device="cpu")
    assert mgr._slabs["k"].dtype == torch.float8_e4m3fn
    assert torch.equal(mgr.kv_scales("k"), torch.ones(2, 4))
    mgr.set_kv_scales("k", torch.tensor([0.5, 1.0, 2.0, 4.0]), layer_idx=1)
    assert mgr.kv_scales("k")[1].tolist() == [0.5, 1.0, 2.0, 4.0] and mgr.kv_scales("k")[0].tolist() == [1.0] * 4
    with pytest.raises(ValueError):
        mgr.set_kv_scales("k", torch.tensor(0.0))


def test_manager_layer_counters_cpu():
    """Reference test_begin_step_resets_layers."""
    mgr = CacheManager(_policy(), num_blocks=16, device="cpu")
    mgr.begin_step({})
    assert mgr._layer_counters["k"] == 0
    mgr.resolve_layer("k")
    mgr.resolve_layer("k")
    assert mgr._layer_counters["k"] == 2
    mgr.begin_step({})
    assert mgr._layer_counters["k"] == 0


def test_io_on_cpu_slab_raises():
    """No CPU path: kernels need device tensors."""
    mgr = CacheManager(_policy(), num_blocks=16, device="cpu")
    mgr.begin_step({"r0": [0, 1]})
    with pytest.raises(ValueError, match="ROCm device"):
        mgr.write_paged("k", 0, torch.randn(6, 8, 64), torch.arange(6))
    with pytest.raises(ValueError, match="ROCm device"):
        mgr.read_paged("k", 0, 6)
    mgr.begin_step({})
    mgr.write_paged("k", 0, torch.randn(6, 8, 64), torch.arange(6))  # no tables: nothing to write
    with pytest.raises(RuntimeError):
        mgr.read_paged("k", 0, 6)


class _Exec(_KVCacheMixin):
    def __init__(self):
        self._kv_cache = None
        self._block_tables = {}
        self._block_size = 16
        self._num_kv_heads = 0
        self._head_dim = 0


def test_mixin_shapes_cpu():
    ex = _Exec()
    kv = ex.prepare_kv_blocks(num_layers=32, num_kv_heads=8, head_dim=128, block_size=16, num_blocks=10,
                              device="cpu")
    assert kv.shape == (10, 32, 2, 16, 8, 128) and kv.dtype == torch.float16
    assert kv[:, 3, 1].stride()[1:] == (128, 16 * 128, 1)
    ex.set_kv_cache(kv, block_tables={"r0": [0, 1]}, num_kv_heads=8, head_dim=128, block_size=16)
    assert ex._max_seq_from_tables({"a": [1, 2], "b": [3]}) == 32
    with pytest.raises(ValueError, match="ROCm device"):
        ex.write_kv_to_cache(torch.randn(4, 8, 128), torch.randn(4, 8, 128), torch.arange(4), {"r0": [0]})
    with pytest.raises(RuntimeError):
        ex.gather_kv_from_cache({}, 4)
