"""PagedKVIntercept's intercept rules on the host, over a recording stand-in
for the CacheManager (no device work): the (func_index, output_index)
contract (reference python_runtime/engine/mlir_executor.py:375-393),
sequential layer resolution once per step, write placement at the step's
positions, and which ops `run_sdpa` answers from the slabs."""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from compiler.sfa_cache_proto import SfaInterceptSpec
from python_runtime.engine.kv_intercept import PagedKVIntercept


@dataclass
class Op:
    op_name: str
    operands: list[str]
    results: list[str]
    attributes: dict = field(default_factory=dict)


class _Mgr:
    """Records the CacheManager calls the intercept makes."""

    def __init__(self):
        self.calls = []
        self.counters: dict[str, int] = {}
        self._block_size = 16

    def begin_step(self, tables):
        self.calls.append(("begin", sorted(tables)))
        self.counters = {}

    def resolve_layer(self, slab):
        n = self.counters.get(slab, 0)
        self.counters[slab] = n + 1
        return n

    def write_paged(self, slab, layer, data, positions):
        self.calls.append(("write", slab, layer, tuple(data.shape), positions.tolist()))

    def read_paged(self, slab, layer, n):
        self.calls.append(("read", slab, layer, n))
        return torch.zeros(1, n, 2, 4)

    def layer_view(self, slab, layer):
        return torch.zeros(1, 16, 2, 4)  # a float32 slab: no chunk kernel for it

    def attend(self, q, layer, lens, k_slab="k", v_slab="v", scale=None):
        self.calls.append(("attend", k_slab, v_slab, layer, list(lens), round(scale, 6)))
        return torch.zeros(q.shape)


class _Hal:
    def __init__(self):
        self.calls = 0

    def execute(self, op_name, inputs, **kw):
        self.calls += 1
        return torch.ones(1)


def _intercepts(num_layers: int) -> list:
    out = []
    for layer in range(num_layers):
        for slab, oi in (("k", 0), ("v", 1)):
            spec = SfaInterceptSpec()
            spec.slab_id = slab
            spec.op_name_pattern = "scaled_dot_product_attention"
            spec.intercept_type = "read_write"
            spec.source = f"operand[{1 if slab == 'k' else 2}]"
            spec.layer = "sequential"
            spec.param_indices.extend([1 + 2 * layer, oi])
            out.append(spec)
    return out


def _producers(num_layers: int) -> dict:
    p = {}
    for layer in range(num_layers):
        for name, oi in ((f"%k{layer}", 0), (f"%v{layer}", 1)):
            p[name] = (1 + 2 * layer, oi)
            p[name.lstrip("%")] = (1 + 2 * layer, oi)
    return p


def _op(layer: int, k: str | None = None, v: str | None = None) -> Op:
    return Op("scaled_dot_product_attention", [f"%q{layer}", k or f"%k{layer}", v or f"%v{layer}", "%mask"],
              [f"%out{layer}"])


def test_contract_filter_and_sequential_layers():
    mgr = _Mgr()
    ic = PagedKVIntercept(mgr, _intercepts(2), _producers(2))
    ic.begin_step({"r1": [4], "r0": [2]}, positions=torch.tensor([[5, 6]]), is_decode=False)
    kv = torch.zeros(1, 2, 2, 4)
    ssa = {"%k0": kv, "%v0": kv, "%k1": kv, "%v1": kv, "%kx": kv, "%vx": kv}
    ic.handle(_op(0), ssa)
    ic.handle(_op(0, "%kx", "%vx"), ssa)  # a foreign producer: no intercept applies
    ic.handle(_op(1), ssa)
    writes = [c for c in mgr.calls if c[0] == "write"]
    # per-slab counters run 0, 1 over the step: layer 0's op writes slab layer
    # 0, layer 1's op slab layer 1; the foreign op writes nothing
    assert writes == [("write", "k", 0, (1, 2, 2, 4), [5, 6]), ("write", "v", 0, (1, 2, 2, 4), [5, 6]),
                      ("write", "k", 1, (1, 2, 2, 4), [5, 6]), ("write", "v", 1, (1, 2, 2, 4), [5, 6])]
    assert mgr.calls[0] == ("begin", ["r0", "r1"])


def test_decode_answers_from_the_slabs_and_prefill_goes_to_the_hal():
    mgr = _Mgr()
    ic = PagedKVIntercept(mgr, _intercepts(1), _producers(1))
    hal = _Hal()
    q = torch.zeros(1, 8, 1, 4)
    # prefill, fp32 activations: written, then the op runs through the HAL as is
    ic.begin_step({"r0": [0]}, positions=torch.arange(3), is_decode=False)
    ic.handle(_op(0), {"%k0": torch.zeros(1, 2, 3, 4), "%v0": torch.zeros(1, 2, 3, 4)})
    ic.run_sdpa(_op(0), [torch.zeros(1, 8, 3, 4)], hal)
    assert hal.calls == 1
    # decode at position 20 with a two-block table: attention over 21 tokens, no gather
    ic.begin_step({"r0": [0, 1]}, positions=torch.tensor([20]), is_decode=True)
    ic.handle(_op(0), {"%k0": torch.zeros(1, 2, 1, 4), "%v0": torch.zeros(1, 2, 1, 4)})
    out = ic.run_sdpa(_op(0), [q], hal, scale=0.25)
    assert hal.calls == 1 and out.shape == q.shape
    assert ("attend", "k", "v", 0, [21], 0.25) in mgr.calls
    assert not any(c[0] == "read" for c in mgr.calls)
    # a position past the table: the reference's gather pads with zero rows
    # that enter its softmax, so this step gathers and the op runs on the HAL
    ic.begin_step({"r0": [0]}, positions=torch.tensor([20]), is_decode=True)
    ssa = {"%k0": torch.zeros(1, 2, 1, 4), "%v0": torch.zeros(1, 2, 1, 4)}
    n_attend = sum(c[0] == "attend" for c in mgr.calls)
    ic.handle(_op(0), ssa)
    assert ("read", "k", 0, 21) in mgr.calls and ("read", "v", 0, 21) in mgr.calls
    assert ssa["%k0"].shape == (1, 2, 21, 4)
    ic.run_sdpa(_op(0), [q, ssa["%k0"], ssa["%v0"]], hal)
    assert hal.calls == 2 and sum(c[0] == "attend" for c in mgr.calls) == n_attend
    # several requests, every table long enough: one attend over all of them
    ic.begin_step({"r1": [2, 3], "r0": [0, 1]}, positions=torch.tensor([17]), is_decode=True)
    ic.handle(_op(0), {"%k0": torch.zeros(1, 2, 1, 4), "%v0": torch.zeros(1, 2, 1, 4)})
    ic.run_sdpa(_op(0), [torch.zeros(2, 8, 1, 4)], hal)
    assert mgr.calls[-1][:5] == ("attend", "k", "v", 0, [18, 18]) and hal.calls == 2
    # a decode op the reference would mask (is_causal, or a boolean mask):
    # the reference's gathered operands go to the HAL
    ic.begin_step({"r0": [0, 1]}, positions=torch.tensor([20]), is_decode=True)
    ic.handle(_op(0), {"%k0": torch.zeros(1, 2, 1, 4), "%v0": torch.zeros(1, 2, 1, 4)})
    ic.run_sdpa(_op(0), [q, torch.zeros(1, 2, 1, 4), torch.zeros(1, 2, 1, 4)], hal, is_causal=True)
    assert hal.calls == 3 and mgr.calls[-1] == ("read", "v", 0, 21)
    # an op no intercept matched runs through the HAL
    ic.run_sdpa(_op(0, "%kx", "%vx"), [q], hal)
    assert hal.calls == 4


def test_prefill_from_slabs_is_opt_in_and_causal_only():
    mgr = _Mgr()
    hal = _Hal()
    for opt_in in (False, True):
        ic = PagedKVIntercept(mgr, _intercepts(1), _producers(1), prefill_from_slabs=opt_in)
        ic.begin_step({"r0": [0]}, positions=torch.arange(3), is_decode=False)
        ic.handle(_op(0), {"%k0": torch.zeros(1, 2, 3, 4), "%v0": torch.zeros(1, 2, 3, 4)})
        assert bool(ic._pending) == opt_in
        # fp32 slabs here: even when opted in, the chunk kernel does not apply
        ic.run_sdpa(_op(0), [torch.zeros(1, 8, 3, 4)], hal, is_causal=True)
    assert hal.calls == 2


def test_replace_inputs_gathers_like_the_reference():
    mgr = _Mgr()
    ic = PagedKVIntercept(mgr, _intercepts(1), _producers(1), replace_inputs=True)
    ic.begin_step({"r0": [0]}, positions=torch.tensor([7]), is_decode=True)
    ssa = {"%k0": torch.zeros(1, 2, 1, 4, dtype=torch.float16), "%v0": torch.zeros(1, 2, 1, 4)}
    ic.handle(_op(0), ssa)
    assert ("read", "k", 0, 8) in mgr.calls and ("read", "v", 0, 8) in mgr.calls
    assert ssa["%k0"].shape == (1, 2, 8, 4) and ssa["%k0"].dtype == torch.float16
    hal = _Hal()
    ic.run_sdpa(_op(0), [torch.zeros(1, 2, 1, 4)], hal)
    assert hal.calls == 1
