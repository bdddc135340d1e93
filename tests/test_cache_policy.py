"""Cache policy contract: dict form, proto wire format, FP8 slab dtype and scales.

The reference's own cases (compiler/tests/test_cache_policy_metadata.py,
test_cache_policy_binding.py) run against this build's CachePolicy; the
proto encoding is pinned by bytes worked out by hand from the field numbers
of include/sfa_abi.proto:256-286 and the protobuf wire format (tag =
field << 3 | wire type, varints little-endian base 128, repeated scalars
packed), so a wrong field number or type fails.
"""

from __future__ import annotations

import struct

import pytest
import torch

from compiler.cache_policy import (
    CachePolicy,
    _InterceptSpec,
    _SlabSpec,
    bind_cache_policy,
    parse_cache_policy,
    serialize_cache_policy,
)
from compiler.sfa_cache_proto import SfaCachePolicy
from python_runtime.engine import CacheManager

BINDINGS = [(0, 1, "k"), (0, 2, "v"), (2, 1, "k"), (2, 2, "v")]


def _llama(num_layers: int = 2) -> CachePolicy:
    return CachePolicy.for_llama(num_layers=num_layers, num_kv_heads=12, head_dim=64)


def test_for_llama_dict_matches_reference_shape():
    """test_cache_policy_in_metadata's field checks and dict round trip."""
    policy = CachePolicy.for_llama(num_layers=1, num_kv_heads=2, head_dim=8)
    d = policy.to_dict()
    assert d == {
        "slabs": [
            {"slab_id": "k", "storage": "paged", "dims": {"layers": 1, "heads": 2, "dim": 8}, "layout": "BNLD",
             "dtype": "float32"},
            {"slab_id": "v", "storage": "paged", "dims": {"layers": 1, "heads": 2, "dim": 8}, "layout": "BNLD",
             "dtype": "float32"},
        ],
        "intercepts": [
            {"slab_id": "k", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[1]", "layer": "sequential"},
            {"slab_id": "v", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[2]", "layer": "sequential"},
        ],
        "block_size": 16,
        "max_requests": 256,
    }
    assert CachePolicy.from_dict(d).to_dict() == d
    empty = CachePolicy()
    assert empty.is_empty and CachePolicy.none().to_dict() == {"slabs": [], "intercepts": [], "block_size": 16,
                                                               "max_requests": 256}
    assert CachePolicy.from_dict(None).is_empty


def test_for_config_llama3_8b():
    cfg = {"num_hidden_layers": 32, "num_attention_heads": 32, "num_key_value_heads": 8, "hidden_size": 4096}
    p = CachePolicy.for_config(cfg)
    assert [s.dims for s in p.slabs] == [{"layers": 32, "heads": 8, "dim": 128}] * 2
    nested = CachePolicy.for_config({"text_config": dict(cfg, head_dim=96)}, block_size=32, kv_dtype="float8_e4m3fn")
    assert nested.block_size == 32 and nested.slabs[0].dims["dim"] == 96
    assert [s.dtype for s in nested.slabs] == ["float8_e4m3fn"] * 2

    class Obj:
        num_hidden_layers, num_attention_heads, hidden_size = 4, 8, 512
        num_key_value_heads = None

    assert CachePolicy.for_config(Obj()).slabs[0].dims == {"layers": 4, "heads": 8, "dim": 64}


@pytest.mark.parametrize("cfg,msg", [
    ({"num_attention_heads": 8, "hidden_size": 64}, "missing attention fields"),
    ({"num_hidden_layers": 2, "num_attention_heads": 8}, "head_dim and hidden_size"),
    ({"num_hidden_layers": 2, "num_attention_heads": 8, "hidden_size": 60}, "not divisible"),
    ({"num_hidden_layers": 2, "num_attention_heads": 8, "hidden_size": 64, "layer_types": ["full_attention"]},
     "layer_types length"),
])
def test_for_config_errors(cfg, msg):
    with pytest.raises(ValueError, match=msg):
        CachePolicy.for_config(cfg)


def test_for_config_mixed_linear():
    cfg = {"num_hidden_layers": 4, "num_attention_heads": 16, "num_key_value_heads": 2, "head_dim": 256,
           "layer_types": ["linear_attention", "linear_attention", "linear_attention", "full_attention"],
           "linear_num_key_heads": 16, "linear_num_value_heads": 32, "linear_key_head_dim": 128,
           "linear_value_head_dim": 128}
    p = CachePolicy.for_config(cfg)
    assert [s.slab_id for s in p.slabs] == ["k", "v", "recurrent_state", "conv_state"]
    assert p.slabs[0].dims == {"layers": 1, "heads": 2, "dim": 256}
    assert p.slabs[2].dims == {"layers": 3, "heads": 32, "key_dim": 128, "value_dim": 128}
    # 2 * 16 * 128 + 32 * 128 channels, default kernel 4
    assert p.slabs[3].dims == {"layers": 3, "channels": 8192, "kernel": 4}
    assert [(i.op_name, i.source) for i in p.intercepts[2:]] == [("linear_attn", "recurrent_state"),
                                                               ("linear_attn", "conv_state")]


def test_for_rwkv():
    p = CachePolicy.for_rwkv(num_layers=4, state_dim=1024, max_requests=8)
    assert p.slabs[0].to_dict() == {"slab_id": "state", "storage": "fixed", "dims": {"layers": 4, "dim": 1024},
                                    "layout": "RLD", "dtype": "float32"}
    assert p.max_requests == 8 and p.intercepts[0].source == "output"


def test_kv_dtype_checked():
    with pytest.raises(ValueError, match="kv_dtype"):
        CachePolicy.for_llama(2, 2, 8, kv_dtype="int8")


def test_bind_cache_policy_reference_cases():
    policy = bind_cache_policy(_llama(2), BINDINGS)
    assert len(policy.intercepts) == 4
    for (fi, oi, slab_id), ic in zip(BINDINGS, policy.intercepts):
        assert (ic.slab_id, ic.func_index, ic.output_index) == (slab_id, fi, oi)
        assert ic.source == ("operand[1]" if slab_id == "k" else "operand[2]")
    assert bind_cache_policy(_llama(2), []).intercepts == _llama(2).intercepts
    rwkv = bind_cache_policy(CachePolicy.for_rwkv(num_layers=2, state_dim=64), BINDINGS)
    state = [i for i in rwkv.intercepts if i.op_name == "state_evolve"]
    assert len(state) == 1 and state[0].func_index is None
    original = _llama(2)
    bind_cache_policy(original, BINDINGS)
    assert all(i.func_index is None for i in original.intercepts)


def test_serialize_reference_roundtrip():
    """test_roundtrip_param_indices, parsed with this build's messages."""
    blob = serialize_cache_policy(bind_cache_policy(_llama(2), BINDINGS))
    proto = SfaCachePolicy()
    proto.ParseFromString(blob)
    assert [s.name for s in proto.slabs] == ["k", "v"]
    s0 = proto.slabs[0]
    assert (s0.num_layers, s0.num_heads, s0.head_dim, s0.block_size) == (2, 12, 64, 16)
    assert [list(ip.param_indices) for ip in proto.intercepts] == [[fi, oi] for fi, oi, _ in BINDINGS]
    assert (proto.block_size, proto.max_requests) == (16, 256)
    back = parse_cache_policy(blob)
    assert [(i.func_index, i.output_index) for i in back.intercepts] == [(fi, oi) for fi, oi, _ in BINDINGS]
    assert back.slabs[0].dims == {"layers": 2, "heads": 12, "dim": 64}


def _varint(n: int) -> bytes:
    out = b""
    while True:
        b, n = n & 0x7F, n >> 7
        out += bytes([b | (0x80 if n else 0)])
        if not n:
            return out


def _tag(field: int, wire: int) -> bytes:
    return _varint(field << 3 | wire)


def test_wire_format_known_bytes():
    """Hand-assembled encoding: policy block_size 16 / max_requests 256, one
    FP8 slab "k" (1 layer, 2 heads, dim 8, scales 0.5 / 2.0) and one
    intercept with param_indices [3, 1]."""
    assert _tag(222, 0) == bytes([0xF0, 0x0D]) and _varint(256) == bytes([0x80, 0x02])
    slab = (
        _tag(200, 2) + b"\x01k" + _tag(201, 2) + b"\x05paged" + _tag(202, 2) + b"\x04BNLD"
        + _tag(203, 2) + b"\x0dfloat8_e4m3fn" + _tag(205, 0) + b"\x10" + _tag(206, 0) + b"\x01"
        + _tag(207, 0) + b"\x02" + _tag(208, 0) + b"\x08"
        + _tag(209, 2) + b"\x08" + struct.pack("<2f", 0.5, 2.0)
    )
    ic = (_tag(210, 2) + b"\x01k" + _tag(211, 2) + b"\x04sdpa" + _tag(212, 2) + b"\x0aread_write"
          + _tag(213, 2) + b"\x0aoperand[1]" + _tag(214, 2) + b"\x0asequential" + _tag(215, 2) + b"\x02\x03\x01")
    want = (_tag(220, 2) + _varint(len(slab)) + slab + _tag(221, 2) + _varint(len(ic)) + ic
            + _tag(222, 0) + b"\x10" + _tag(223, 0) + _varint(256))
    policy = CachePolicy(
        slabs=[_SlabSpec("k", "paged", {"layers": 1, "heads": 2, "dim": 8}, "BNLD", "float8_e4m3fn",
                         scales=[[0.5, 2.0]])],
        intercepts=[_InterceptSpec("k", "sdpa", "read_write", "operand[1]", func_index=3, output_index=1)],
    )
    assert serialize_cache_policy(policy) == want
    back = parse_cache_policy(want)
    assert back.slabs[0].scales == [[0.5, 2.0]] and back.slabs[0].dtype == "float8_e4m3fn"
    assert back.intercepts[0].func_index == 3 and back.intercepts[0].output_index == 1


def test_fp8_scales_in_policy():
    p = CachePolicy.for_llama(2, 3, 16, kv_dtype="float8_e4m3fn")
    p.set_kv_scales("k", torch.tensor([[0.5, 1.0, 2.0], [0.25, 0.125, 4.0]]))
    assert p.to_dict()["slabs"][0]["scales"] == [[0.5, 1.0, 2.0], [0.25, 0.125, 4.0]]
    assert "scales" not in p.to_dict()["slabs"][1]
    assert CachePolicy.from_dict(p.to_dict()).to_dict() == p.to_dict()
    assert parse_cache_policy(serialize_cache_policy(p)).slabs[0].scales == [[0.5, 1.0, 2.0], [0.25, 0.125, 4.0]]
    with pytest.raises(ValueError):
        p.set_kv_scales("k", [[1.0, 1.0]])
    with pytest.raises(ValueError):
        p.set_kv_scales("k", [[1.0, 0.0, 1.0], [1.0, 1.0, 1.0]])
    with pytest.raises(ValueError):
        CachePolicy.for_llama(2, 3, 16).set_kv_scales("k", [[1.0] * 3] * 2)
    bad = SfaCachePolicy()
    s = bad.slabs.add(name="k", slab_type="paged", dtype="float8_e4m3fn", num_layers=2, num_heads=3, head_dim=16)
    s.scales.extend([1.0, 2.0])
    with pytest.raises(ValueError):
        parse_cache_policy(bad.SerializeToString())


@pytest.mark.parametrize("form", ["policy", "dict", "bytes", "proto"])
def test_manager_takes_every_policy_form(form):
    """CacheManager reads slabs and FP8 scales from each policy form (CPU
    slabs: allocation only)."""
    p = CachePolicy.for_llama(2, 3, 16, kv_dtype="float8_e4m3fn")
    p.set_kv_scales("v", [[0.5, 1.0, 2.0], [0.25, 0.125, 4.0]])
    arg = {"policy": p, "dict": p.to_dict(), "bytes": serialize_cache_policy(p),
           "proto": SfaCachePolicy.FromString(serialize_cache_policy(p))}[form]
    mgr = CacheManager(arg, num_blocks=5, device="cpu")
    assert mgr._slabs["k"].shape == (5, 2, 16, 3, 16) and mgr._slabs["k"].dtype == torch.float8_e4m3fn
    assert torch.equal(mgr.kv_scales("k"), torch.ones(2, 3))
    assert mgr.kv_scales("v").tolist() == [[0.5, 1.0, 2.0], [0.25, 0.125, 4.0]]
    assert mgr._roles == {"k": "k", "v": "v"}
