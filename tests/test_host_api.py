"""Host-side behaviour that needs no GPU: the reference-shaped Python API
refuses CPU tensors (there is no CPU fallback), the FP8 quantizer's
configuration rules, the HAL registry and HipBackend dispatch, KV layouts
and the seeded workloads."""

from __future__ import annotations

import pytest
import torch

from cf_hip import layout as L
from cf_hip import workloads
from kernels.paged_attention import paged_attention, paged_attention_tensors
from kernels.quantize import FP8KVCacheQuantizer
from python_runtime.hal import registry
from python_runtime.hal.hip_backend import HipBackend
from python_runtime.hal.interface import OpExecutor


def test_cpu_tensors_are_refused():
    q = torch.randn(1, 4, 32)
    k = torch.randn(4, 16, 4, 32)
    with pytest.raises(ValueError, match="ROCm"):
        paged_attention(q, k, k, {"r": [0]}, {"r": 5})
    with pytest.raises(ValueError, match="ROCm"):
        paged_attention_tensors(q, k, k, torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="ROCm"):
        FP8KVCacheQuantizer().quantize_block(k)


def test_quantizer_configuration():
    with pytest.raises(ValueError, match="block_size"):
        FP8KVCacheQuantizer(block_size=0)
    q = FP8KVCacheQuantizer(block_size=8)
    assert q.block_size == 8 and q.fp8_max == 448.0 and q._has_fp8_dtype()
    assert q.check_hardware_support("NVIDIA H100") and q.check_hardware_support("AMD MI300")
    assert q.check_hardware_support("AMD Instinct MI355X")
    assert not q.check_hardware_support("NVIDIA A100") and not q.check_hardware_support("CPU")
    for hw in ("H100", "H200", "RTX_4090", "RTX_6000_ADA", "MI300"):
        assert hw in q.SUPPORTED_HARDWARE


def test_compiler_quantize_reexport():
    from compiler.quantize import FP8KVCacheQuantizer as A
    from compiler.quantize.fp8_kv_cache import FP8KVCacheQuantizer as B

    assert A is FP8KVCacheQuantizer and B is FP8KVCacheQuantizer


class _Recorder(OpExecutor):
    def __init__(self):
        self.calls = []

    def execute(self, op_name, inputs, **kwargs):
        self.calls.append((op_name, len(inputs), kwargs))
        return torch.zeros(1)


def test_registry_semantics():
    name = "test_backend_xyz"
    registry.register(name, lambda **kw: _Recorder())
    with pytest.raises(ValueError, match="already registered"):
        registry.register(name, lambda **kw: _Recorder())
    assert isinstance(registry.create(name), _Recorder)
    assert name in registry.list_backends()
    with pytest.raises(KeyError):
        registry.create("no_such_backend")
    with pytest.raises(KeyError):
        registry.get("no_such_backend")


def test_hip_backend_dispatch_and_errors():
    fb = _Recorder()
    be = HipBackend(fallback=fb)
    be.execute("silu", [torch.zeros(2)], alpha=1)
    assert fb.calls == [("silu", 1, {"alpha": 1})]
    with pytest.raises(ValueError, match="Unknown op"):
        HipBackend().execute("silu", [torch.zeros(2)])
    with pytest.raises(ValueError, match="at least 4"):
        be.execute("paged_attention", [torch.zeros(1)])
    with pytest.raises(ValueError, match="at most 5"):
        be.execute("paged_attention", [torch.zeros(1)] * 6)
    with pytest.raises(NotImplementedError):
        be.async_copy(None, None, 0)
    with pytest.raises(NotImplementedError):
        be.memory_retrieve(None, None)
    with pytest.raises(NotImplementedError):
        be.send_kv_cache(None, "x")
    assert "paged_attention" in HipBackend.supported_ops()
    assert {"cache_read", "cache_write"} <= set(HipBackend.supported_ops())
    with pytest.raises(ValueError, match="at least 5"):
        be.execute("cache_write", [torch.zeros(1)] * 4)
    with pytest.raises(ValueError, match="ROCm device"):
        be.execute("cache_read", [torch.zeros(2, 16, 1, 8), torch.zeros(2, 16, 1, 8),
                                  torch.zeros(1, 1, dtype=torch.int32)])


def test_hip_backend_sdpa_routing_on_the_host():
    """scaled_dot_product_attention takes 3-4 inputs (the reference's
    registration); calls the HIP kernels do not run -- CPU tensors, a mask,
    dropout, a query longer than one token, head counts torch would reject --
    go to the fallback with their inputs and kwargs unchanged, and without a
    fallback raise ValueError."""
    fb = _Recorder()
    be = HipBackend(fallback=fb)
    q, k, v = torch.zeros(2, 4, 1, 8), torch.zeros(2, 4, 5, 8), torch.zeros(2, 4, 5, 8)
    mask = torch.zeros(2, 1, 1, 5)
    be.execute("scaled_dot_product_attention", [q, k, v])
    be.execute("scaled_dot_product_attention", [q, k, v, mask], is_causal=False)
    be.execute("scaled_dot_product_attention", [torch.zeros(2, 4, 3, 8), k, v], scale=0.5)
    assert fb.calls == [("scaled_dot_product_attention", 3, {}),
                        ("scaled_dot_product_attention", 4, {"is_causal": False}),
                        ("scaled_dot_product_attention", 3, {"scale": 0.5})]
    with pytest.raises(ValueError, match="at least 3"):
        be.execute("scaled_dot_product_attention", [q, k])
    with pytest.raises(ValueError, match="at most 4"):
        be.execute("scaled_dot_product_attention", [q, k, v, mask, mask])
    with pytest.raises(ValueError, match="no fallback"):
        HipBackend().execute("scaled_dot_product_attention", [q, k, v])
    assert "scaled_dot_product_attention" in HipBackend.supported_ops()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
def test_layouts(dtype):
    k, v = L.alloc_kv_cache(5, 16, 4, 32, dtype, "cpu", "native")
    assert k.shape == v.shape == (5, 16, 4, 32)
    assert k.stride() == (4 * 16 * 32, 32, 16 * 32, 1)
    assert v.stride() == (4 * 32 * 16, 1, 32 * 16, 16)
    assert L.layout_of(k, False) == "native" and L.layout_of(v, True) == "native"
    src = torch.randn(5, 16, 4, 32)
    for lay in ("native", "token_major"):
        for is_v in (False, True):
            t = L.to_layout(src, lay, is_v)
            assert torch.equal(t, src) and L.layout_of(t, is_v) == lay
    # paired: one allocation, (block, head) = K tile [bs][D] then V tile [D][bs]
    kp, vp = L.alloc_kv_cache(5, 16, 4, 32, dtype, "cpu", "paired")
    assert kp.stride() == (4 * 2 * 16 * 32, 32, 2 * 16 * 32, 1)
    assert vp.stride() == (4 * 2 * 16 * 32, 1, 2 * 16 * 32, 16)
    assert vp.data_ptr() - kp.data_ptr() == 16 * 32 * kp.element_size()
    assert L.layout_of(kp, False) == "paired" and L.layout_of(vp, True) == "paired"
    vsrc = torch.randn(5, 16, 4, 32)
    kp, vp = L.to_paired(src.to(dtype), vsrc.to(dtype))
    assert torch.equal(kp.float(), src.to(dtype).float()) and torch.equal(vp.float(), vsrc.to(dtype).float())
    # block 2, head 3, token 5, channel 7 of K and of V, read from the raw storage
    raw = kp.as_strided((5 * 4 * 2 * 16 * 32,), (1,), kp.storage_offset()).view(5, 4, 2, 16 * 32)
    assert torch.equal(raw[2, 3, 0, 5 * 32 + 7].float(), kp[2, 5, 3, 7].float())
    assert torch.equal(raw[2, 3, 1, 7 * 16 + 5].float(), vp[2, 5, 3, 7].float())
    with pytest.raises(ValueError):
        L.to_layout(src, "paired", False)
    with pytest.raises(ValueError):
        L.alloc_kv_cache(1, 16, 1, 8, torch.float32, "cpu", "bogus")


def test_workloads_are_seeded_and_shaped():
    a = workloads.make_case("c3_llama3_8b", seed=1, batch=4)
    b = workloads.make_case("c3_llama3_8b", seed=1, batch=4)
    assert a.block_tables == b.block_tables and a.seq_lens == b.seq_lens and torch.equal(a.k, b.k)
    pre = a.meta["shared_prefix_blocks"]
    assert pre == 64 and a.block_tables[0][:pre] == a.block_tables[1][:pre]
    assert not set(a.block_tables[2]) & set(a.block_tables[0])
    assert all(1024 <= n <= 8192 for n in a.seq_lens)
    assert a.q.shape == (4, 32, 128) and a.k.shape[1:] == (16, 8, 128) and a.kv_dtype == torch.float8_e4m3fn
    c4 = workloads.make_case("c4_llama3_70b", seed=1, batch=16)
    assert all(512 <= n <= 32768 for n in c4.seq_lens) and c4.q.shape[1] == 64
    c1 = workloads.make_case("c1_opt125m", seed=1)
    flat = [b for t in c1.block_tables for b in t]
    assert len(flat) == len(set(flat)) and all(0 <= x < 256 for x in flat)
    with pytest.raises(ValueError):
        workloads.make_case("nope")


def test_algorithmic_bytes():
    q = torch.zeros(2, 4, 8, dtype=torch.bfloat16)
    k = torch.zeros(4, 16, 2, 8, dtype=torch.bfloat16)
    case = workloads.DecodeCase("t", q, k, k, [[0, 1], [0, 2]], [20, 30], 16, 0.1, torch.float8_e4m3fn)
    ab = workloads.algorithmic_bytes(case)
    per_tok = 2 * 2 * 8 * 1
    # block 0: 16 rows (shared), block 1: 4 rows, block 2: 14 rows
    assert ab["unique_kv"] == (16 + 4 + 14) * per_tok
    assert ab["logical"] - ab["unique"] == (50 - 34) * per_tok
    assert ab["tokens"] == 50


def test_shared_prefix_lens_matches_token_level_definition():
    """ops.shared_prefix_lens against a token-by-token statement of sharing:
    the longest t such that every token x < t of both sequences lies in the
    same physical block at the same table position."""
    import random

    from cf_hip.ops import shared_prefix_lens

    rng = random.Random(3)
    bs = 16
    for _ in range(300):
        n = rng.randint(1, 9)
        pool = iter(range(10**6))
        tables, lens = [], []
        prev = []
        for _b in range(n):
            keep = rng.randint(0, len(prev)) if prev and rng.random() < 0.7 else 0
            nblk = rng.randint(max(keep, 1), keep + 6)
            t = prev[:keep] + [next(pool) for _ in range(nblk - keep)]
            tables.append(t)
            lens.append(rng.randint(1, nblk * bs))
            prev = t
        got = shared_prefix_lens(tables, lens, bs)
        assert got[0] == 0
        for b in range(1, n):
            t = 0
            while (t < min(lens[b - 1], lens[b]) and tables[b - 1][t // bs] == tables[b][t // bs]):
                t += 1
            assert got[b] == t, (tables[b - 1], tables[b], lens[b - 1], lens[b], got[b], t)
