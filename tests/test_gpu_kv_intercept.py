"""The executor's cache-policy intercept on the GPU (PagedKVIntercept).

The first four tests restate the reference's own intercept cases
(python_runtime/engine/tests/test_kv_intercept.py:158-255: contract
filtering and layer isolation, the exact-not-block-multiple decode gather,
prefill leaving the SDPA inputs alone) with the reference's policy shape;
the rest check the outputs that replace the gather + dense SDPA against the
float64 oracle and against the reference's own path (gather + dense SDPA):
decode from the slabs (fp32, bf16 and e4m3 slabs; one request and a
multi-request batch with mixed table lengths), the default prefill (the
reference's dense SDPA over the op's own K and V), and the opt-in
chunked-prefill from the slabs (bf16 queries over e4m3 slabs, a first chunk
and a later one that also sees the cached prefix).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F  # noqa: N812

from oracle import fp8 as ofp8
from oracle.paged_attention import paged_attention_fp64, paged_prefill_fp64
from python_runtime.engine.kv_intercept import PagedKVIntercept
from python_runtime.hal.interface import OpExecutor
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu

_NH, _HD = 2, 4


@dataclass
class Op:
    op_name: str
    operands: list[str]
    results: list[str]
    attributes: dict = field(default_factory=dict)


def _policy_dict(num_layers: int = 2, heads: int = _NH, dim: int = _HD, dtype: str = "float32") -> dict:
    """The reference test's policy: K and V slabs, one read_write intercept
    per (layer, slab) keyed by the producer's (func_index, output_index)."""
    slabs = [{"slab_id": s, "storage": "paged", "dims": {"layers": num_layers, "heads": heads, "dim": dim},
              "layout": "BNLD", "dtype": dtype} for s in ("k", "v")]
    intercepts = []
    for layer in range(num_layers):
        fi = 1 + layer * 2
        for slab, oi in (("k", 0), ("v", 1)):
            intercepts.append({"slab_id": slab, "op_name": "scaled_dot_product_attention", "direction": "read_write",
                               "source": f"operand[{1 if slab == 'k' else 2}]", "layer": "sequential",
                               "func_index": fi, "output_index": oi})
    return {"slabs": slabs, "intercepts": intercepts, "block_size": 16, "max_requests": 256}


def _module(num_layers: int = 2, **kw) -> SimpleNamespace:
    """Function outputs as the reference's split module lays them out:
    0 main_0 -> %q0; 1 + 2l main_(l)a -> %k(l) @ 0, %v(l) @ 1; 2 + 2l SDPA."""
    funcs = [SimpleNamespace(outputs=[("%q0", "t", False)])]
    for layer in range(num_layers):
        funcs.append(SimpleNamespace(outputs=[(f"%k{layer}", "t", True), (f"%v{layer}", "t", True)]))
        funcs.append(SimpleNamespace(outputs=[(f"%out{layer}", "t", False)]))
    return SimpleNamespace(functions=funcs, metadata={"cache_policy": _policy_dict(num_layers, **kw),
                                                      "num_blocks": 64})


def _sdpa_op(layer: int) -> Op:
    return Op("scaled_dot_product_attention", [f"%q{layer}", f"%k{layer}", f"%v{layer}", "%attn_mask"],
              [f"%out{layer}"])


def _kv(seq: int, base: float, dev) -> torch.Tensor:
    return torch.full((1, _NH, seq, _HD), base, device=dev)


class _DenseSdpa(OpExecutor):
    """What the reference's PyTorchBackend runs for the op without a mask
    (pytorch_backend/_ops_attention.py:13-53), counting its calls."""

    def __init__(self):
        self.calls = 0

    def execute(self, op_name, inputs, **kwargs):
        assert op_name == "scaled_dot_product_attention"
        self.calls += 1
        q, k, v = inputs[0], inputs[1], inputs[2]
        return F.scaled_dot_product_attention(q.float(), k.float(), v.float(), scale=kwargs.get("scale"),
                                              is_causal=bool(kwargs.get("is_causal", False))).to(q.dtype)


def test_each_layer_writes_its_own_slab_layer(gpu):
    ic = PagedKVIntercept.from_module(_module(2), device=gpu)
    ic.begin_step({"r0": [0, 1]}, positions=torch.tensor([0, 1, 2]))
    ssa: dict[str, torch.Tensor] = {}
    for layer, base in ((0, 1.0), (1, 2.0)):
        ssa[f"%k{layer}"] = _kv(3, base, gpu)
        ssa[f"%v{layer}"] = _kv(3, base + 10, gpu)
        ic.handle(_sdpa_op(layer), ssa)
    for layer, base in ((0, 1.0), (1, 2.0)):
        k = ic.cache_mgr.read_paged("k", layer, max_seq_len=3)
        v = ic.cache_mgr.read_paged("v", layer, max_seq_len=3)
        assert torch.equal(k, torch.full((1, 3, _NH, _HD), base, device=gpu)), f"layer {layer} K"
        assert torch.equal(v, torch.full((1, 3, _NH, _HD), base + 10, device=gpu)), f"layer {layer} V"


def test_intercept_ignores_foreign_producer(gpu):
    ic = PagedKVIntercept.from_module(_module(1), device=gpu)
    ic.begin_step({"r0": [0]}, positions=torch.tensor([0]))
    ssa = {"%k_foreign": _kv(1, 7.0, gpu), "%v_foreign": _kv(1, 8.0, gpu)}
    op = Op("scaled_dot_product_attention", ["%q0", "%k_foreign", "%v_foreign", "%attn_mask"], ["%out0"])
    ic.handle(op, ssa)
    assert torch.all(ic.cache_mgr.read_paged("k", 0, max_seq_len=1) == 0.0)
    hal = _DenseSdpa()
    ic.run_sdpa(op, [torch.zeros(1, _NH, 1, _HD, device=gpu), ssa["%k_foreign"], ssa["%v_foreign"]], hal)
    assert hal.calls == 1  # nothing was intercepted: the op runs as the reference runs it


def test_decode_gather_is_exact_not_block_multiple(gpu):
    """replace_inputs=True: the reference's decode (gather + substitute)."""
    ic = PagedKVIntercept.from_module(_module(1), device=gpu, replace_inputs=True)
    tables = {"r0": [0, 1]}
    ic.begin_step(tables, positions=torch.tensor([0, 1, 2, 3, 4, 5, 6]), is_decode=False)
    ic.handle(_sdpa_op(0), {"%k0": _kv(7, 1.0, gpu), "%v0": _kv(7, 11.0, gpu)})
    ic.begin_step(tables, positions=torch.tensor([7]), is_decode=True)
    ssa = {"%k0": torch.full((1, _NH, 1, _HD), 99.0, device=gpu), "%v0": torch.full((1, _NH, 1, _HD), 109.0,
                                                                                     device=gpu)}
    ic.handle(_sdpa_op(0), ssa)
    k = ssa["%k0"]
    assert k.shape == (1, _NH, 8, _HD)
    assert torch.equal(k[0, :, :7], torch.full((_NH, 7, _HD), 1.0, device=gpu))
    assert torch.equal(k[0, :, 7:8], torch.full((_NH, 1, _HD), 99.0, device=gpu))
    assert torch.equal(ssa["%v0"][0, :, 7:8], torch.full((_NH, 1, _HD), 109.0, device=gpu))


@pytest.mark.parametrize("replace_inputs", [False, True])
def test_prefill_does_not_replace_sdpa_inputs(gpu, replace_inputs):
    ic = PagedKVIntercept.from_module(_module(1), device=gpu, replace_inputs=replace_inputs)
    ic.begin_step({"r0": [0]}, positions=torch.tensor([0, 1]), is_decode=False)
    k, v = _kv(2, 3.0, gpu), _kv(2, 4.0, gpu)
    ssa = {"%k0": k, "%v0": v}
    ic.handle(_sdpa_op(0), ssa)
    assert ssa["%k0"] is k and ssa["%v0"] is v
    hal = _DenseSdpa()
    ic.run_sdpa(_sdpa_op(0), [torch.zeros(1, _NH, 2, _HD, device=gpu), k, v], hal)
    assert hal.calls == 1  # fp32 slabs: the chunk kernel does not apply, the op runs densely


def test_decode_attends_from_the_slabs(gpu):
    """Prefill 0..6 then decode at 7 (the reference's gather case with random
    rows): the paged output equals the float64 oracle over exactly rows
    0..7, and the reference's own path (gather + dense SDPA); no dense call
    is made, nothing is gathered."""
    g = torch.Generator(device=gpu).manual_seed(5)
    rows_k = torch.randn(8, _NH, _HD, generator=g, device=gpu)
    rows_v = torch.randn(8, _NH, _HD, generator=g, device=gpu)
    q = torch.randn(1, _NH, 1, _HD, generator=g, device=gpu)
    outs = {}
    for replace in (False, True):
        ic = PagedKVIntercept.from_module(_module(1), device=gpu, replace_inputs=replace)
        tables = {"r0": [3, 5]}
        ic.begin_step(tables, positions=torch.arange(7), is_decode=False)
        ssa = {"%k0": rows_k[:7].permute(1, 0, 2).unsqueeze(0), "%v0": rows_v[:7].permute(1, 0, 2).unsqueeze(0)}
        ic.handle(_sdpa_op(0), ssa)
        ic.begin_step(tables, positions=torch.tensor([7]), is_decode=True)
        ssa = {"%k0": rows_k[7:].permute(1, 0, 2).unsqueeze(0), "%v0": rows_v[7:].permute(1, 0, 2).unsqueeze(0)}
        ic.handle(_sdpa_op(0), ssa)
        hal = _DenseSdpa()
        outs[replace] = ic.run_sdpa(_sdpa_op(0), [q, ssa["%k0"], ssa["%v0"]], hal)
        assert hal.calls == (1 if replace else 0)
    torch.cuda.synchronize()
    kc = rows_k.cpu().numpy()[:, None]  # [8 blocks of one token, 1, H, D]
    vc = rows_v.cpu().numpy()[:, None]
    ref = paged_attention_fp64(q[:, :, 0].cpu().numpy(), kc, vc, [list(range(8))], [8], 1, 1 / math.sqrt(_HD))
    assert_close(outs[False][:, :, 0].cpu().numpy(), ref, torch.float32, "intercept decode from slabs")
    assert_close(outs[True][:, :, 0].cpu().numpy(), ref, torch.float32, "reference path (gather + dense)")


def _e4m3_rows(ic: PagedKVIntercept, slab: str, layer: int, table: list[int], n: int) -> np.ndarray:
    """Rows 0..n-1 of a request as the slab holds them (codes decoded by the
    oracle, times the slab's per-head scale): [n, H, D] float."""
    view = ic.cache_mgr.layer_view(slab, layer)
    codes = view.contiguous().view(torch.uint8).cpu().numpy()
    vals = ofp8.decode(codes) * ic.cache_mgr.kv_scales(slab)[layer].cpu().numpy()[None, None, :, None]
    tok = np.arange(n)
    return vals[np.asarray(table)[tok // 16], tok % 16]


@pytest.mark.parametrize("act", [torch.bfloat16, torch.float16])
def test_llama_shaped_prefill_then_decode_from_fp8_slabs(gpu, act):
    """Llama-3-8B attention shape, e4m3 slabs, bf16 or fp16 activations, one
    request: a 300-token chunk at 0..299, a second chunk at 300..599 (sees
    the cached prefix), then a decode at 600 -- every output from the slabs
    on the HIP kernels (no dense fallback), against the float64 oracle on the
    codes the slabs hold."""
    hq, hkv, d, layers = 32, 8, 128, 2
    ic = PagedKVIntercept.from_module(_module(layers, heads=hkv, dim=d, dtype="float8_e4m3fn"), device=gpu,
                                      prefill_from_slabs=True)
    for s in ("k", "v"):
        ic.cache_mgr.set_kv_scales(s, torch.full((layers, hkv), 0.02))
    g = torch.Generator(device=gpu).manual_seed(11)
    table = [int(x) for x in torch.randperm(64, generator=torch.Generator().manual_seed(2))[:40]]
    tables = {"req": table}
    hal = _DenseSdpa()
    layer = 1  # the second layer's op (the first consumes layer 0's counters)
    for start, n, decode in ((0, 300, False), (300, 300, False), (600, 1, True)):
        print(f"[case] intercept llama {act} chunk start={start} rows={n} decode={decode}", flush=True)
        ic.begin_step(tables, positions=torch.arange(start, start + n), is_decode=decode)
        q = torch.randn(1, hq, n, d, generator=g, device=gpu).to(act)
        results = []
        for lay in range(layers):
            k = torch.randn(1, hkv, n, d, generator=g, device=gpu).to(act)
            v = torch.randn(1, hkv, n, d, generator=g, device=gpu).to(act)
            ssa = {f"%k{lay}": k, f"%v{lay}": v}
            ic.handle(_sdpa_op(lay), ssa)
            assert ssa[f"%k{lay}"] is k  # never substituted
            attrs = {} if decode else {"is_causal": True}
            results.append(ic.run_sdpa(_sdpa_op(lay), [q, k, v], hal, **attrs))
        torch.cuda.synchronize()
        assert hal.calls == 0
        out = results[layer]
        assert out.shape == (1, hq, n, d) and out.dtype == act
        kk = _e4m3_rows(ic, "k", layer, table, start + n)
        vv = _e4m3_rows(ic, "v", layer, table, start + n)
        kc, vc = kk[:, None], vv[:, None]  # one-token blocks
        qrows = q[0].permute(1, 0, 2).float().cpu().numpy()  # [n, Hq, D]
        ref, _ = paged_prefill_fp64(qrows, kc, vc, [list(range(start + n))], [start + n], [0, n], 1,
                                    1 / math.sqrt(d))
        got = out[0].permute(1, 0, 2).float().cpu().numpy()
        assert_close(got, ref, act, f"intercept llama {act} start={start} n={n}")


def test_default_prefill_is_the_reference_dense_sdpa(gpu):
    """Prefill chunks at 0..255 and 256..511 over e4m3 slabs, bf16
    activations: by default the op's output is the HAL's dense causal SDPA
    over the op's own (unquantized) K and V -- the reference's call, bitwise
    -- and the rows still land in the slabs.  Opting in to prefill from the
    slabs at position 0 over bf16 slabs gives the same attention within the
    bf16 tolerance (the slabs hold the op's K and V exactly there)."""
    hq, hkv, d = 8, 2, 64
    g = torch.Generator(device=gpu).manual_seed(3)
    table = list(range(20, 52))  # 32 blocks of the 64-block pool: 512 tokens
    for dtype, opt_in in (("float8_e4m3fn", False), ("bfloat16", False), ("bfloat16", True)):
        ic = PagedKVIntercept.from_module(_module(1, heads=hkv, dim=d, dtype=dtype), device=gpu,
                                          prefill_from_slabs=opt_in)
        if dtype == "float8_e4m3fn":
            for s in ("k", "v"):
                ic.cache_mgr.set_kv_scales(s, torch.full((1, hkv), 0.02))
        for start in ((0,) if opt_in else (0, 256)):
            n = 256
            print(f"[case] default prefill dtype={dtype} opt_in={opt_in} start={start}", flush=True)
            ic.begin_step({"r0": table}, positions=torch.arange(start, start + n), is_decode=False)
            q = torch.randn(1, hq, n, d, generator=g, device=gpu).to(torch.bfloat16)
            k = torch.randn(1, hkv, n, d, generator=g, device=gpu).to(torch.bfloat16)
            v = torch.randn(1, hkv, n, d, generator=g, device=gpu).to(torch.bfloat16)
            ssa = {"%k0": k, "%v0": v}
            ic.handle(_sdpa_op(0), ssa)
            assert ssa["%k0"] is k and ssa["%v0"] is v
            hal = _DenseSdpa()
            kr = k.repeat_interleave(hq // hkv, dim=1)
            vr = v.repeat_interleave(hq // hkv, dim=1)
            out = ic.run_sdpa(_sdpa_op(0), [q, kr, vr], hal, is_causal=True)
            want = _DenseSdpa().execute("scaled_dot_product_attention", [q, kr, vr], is_causal=True)
            torch.cuda.synchronize()
            if opt_in:
                assert hal.calls == 0
                assert_close(out.float().cpu().numpy(), want.float().cpu().numpy(), torch.bfloat16,
                             "prefill from bf16 slabs at position 0 vs dense causal SDPA")
            else:
                assert hal.calls == 1 and torch.equal(out, want)
            back = ic.cache_mgr.read_paged("k", 0, start + n)[0, start:start + n].permute(1, 0, 2)
            if dtype == "bfloat16":
                assert torch.equal(back.to(torch.bfloat16), k[0]), "rows written to the slab"


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_multi_request_decode_matches_the_reference_gather(gpu, dtype):
    """Three requests (sorted ids differ from insertion order), GQA 8/2
    heads, tables of 3, 2 and 4 blocks.  A decode step whose position every
    table covers is answered from the slabs and equals the reference's path
    (gather + dense SDPA, replace_inputs=True); a step past the shortest
    table -- where the reference's gather adds zero rows to that request's
    softmax -- gathers as the reference does, so both paths agree there
    too, bitwise."""
    hq, hkv, d = 8, 2, 64
    tdt = {"float32": torch.float32, "bfloat16": torch.bfloat16}[dtype]
    g = torch.Generator(device=gpu).manual_seed(9)
    tables = {"rb": [7, 3, 11], "ra": [0, 5], "rc": [20, 21, 22, 23]}
    rows = {rid: torch.randn(len(t) * 16, hkv, d, generator=g, device=gpu).to(tdt) for rid, t in tables.items()}
    outs = {}
    for replace in (False, True):
        ic = PagedKVIntercept.from_module(_module(1, heads=hkv, dim=d, dtype=dtype), device=gpu,
                                          replace_inputs=replace)
        for rid, t in tables.items():  # fill every request's blocks through its own table
            ic.begin_step({rid: t}, positions=torch.arange(len(t) * 16), is_decode=False)
            kv = rows[rid].permute(1, 0, 2).unsqueeze(0)
            ic.handle(_sdpa_op(0), {"%k0": kv, "%v0": kv * 0.5})
        for pos in (20, 40):
            print(f"[case] multi-request decode dtype={dtype} replace={replace} pos={pos}", flush=True)
            ic.begin_step(tables, positions=torch.tensor([pos]), is_decode=True)
            knew = torch.randn(1, hkv, 1, d, generator=torch.Generator(device=gpu).manual_seed(pos),
                               device=gpu).to(tdt)
            ssa = {"%k0": knew, "%v0": knew * 0.5}
            ic.handle(_sdpa_op(0), ssa)
            q = torch.randn(3, hq, 1, d, generator=torch.Generator(device=gpu).manual_seed(100 + pos),
                            device=gpu).to(tdt)
            hal = _DenseSdpa()
            k_in, v_in = ssa["%k0"], ssa["%v0"]
            if k_in.shape[1] == hkv and k_in.shape[2] > 1:  # gathered operands: GQA for the dense HAL
                k_in = k_in.repeat_interleave(hq // hkv, dim=1)
                v_in = v_in.repeat_interleave(hq // hkv, dim=1)
            outs[(replace, pos)] = (ic.run_sdpa(_sdpa_op(0), [q, k_in, v_in], hal).float().cpu(), hal.calls)
    torch.cuda.synchronize()
    # position 20: every table covers 21 tokens -> kernel vs the reference's dense path
    assert outs[(False, 20)][1] == 0 and outs[(True, 20)][1] == 1
    assert_close(outs[(False, 20)][0].numpy(), outs[(True, 20)][0].numpy(), tdt, "multi-request decode")
    # position 40: "ra" holds 32 tokens -> both gather, zero rows included
    assert outs[(False, 40)][1] == 1 and outs[(True, 40)][1] == 1
    assert torch.equal(outs[(False, 40)][0], outs[(True, 40)][0])
