"""The executor's cache-policy intercept, with attention read from the slabs.

Drop-in for the reference's MlirExecutor._handle_cache_intercept and the
dense SDPA call that follows it (python_runtime/engine/mlir_executor.py
:369-419 and :358).  The reference, at each intercepted SDPA op:
  1. writes the op's K and V operands into the paged slabs at this step's
     positions (CacheManager.write_paged, one Python loop per token);
  2. on a decode step, gathers each slab's rows [0, max_position] back into
     dense [requests, heads, seq, dim] tensors (read_paged: requests in
     sorted id order, rows past a request's table left zero) and
     substitutes them for the SDPA's K and V operands;
  3. runs the SDPA op densely through the HAL (hal.execute).

PagedKVIntercept keeps the intercept's rules -- which intercepts apply
(the (func_index, output_index) contract on the op's source operand),
sequential layer resolution, the write placement -- and replaces the data
path:
  - the writes are one cf_paged_write launch per slab;
  - decode: when every request's table covers max_position + 1 tokens,
    nothing is gathered; `run_sdpa` computes the op's output with the paged
    decode kernel straight from the slabs (CacheManager.attend), each
    request over exactly the prefix through the fed token, which is what
    the reference's gathered operands hold.  When some table is shorter,
    the reference's gather pads that request with zero rows that take part
    in its softmax; such a step gathers and substitutes the operands as the
    reference does and the op runs on the HAL, so its output is the
    reference's in every case;
  - prefill: the SDPA inputs stay untouched and the op runs on the HAL, as
    in the reference (dense attention over the op's own K and V with its
    positional mask).  With prefill_from_slabs=True, a single request's
    causal chunk with bf16 queries over bf16 / e4m3 slabs (or fp16 queries
    over fp16 / e4m3 slabs) runs
    chunked-prefill attention from the slabs instead (CacheManager
    .attend_chunks: the row at position p sees positions [0, p]).  That is
    a different operation, not a faster route to the same one: it reads K
    and V back from the slabs (on e4m3 slabs, the quantized values) and a
    chunk after the first also sees the cached prefix, which the
    reference's call never does.
With replace_inputs=True every decode step gathers (one cf_paged_gather
launch per slab) and substitutes the SDPA operands, and `run_sdpa` passes
the op to the HAL.

An op is any object with `op_name`, `operands`, `results` and (optionally)
`attributes`, as the reference's compiler.artifact.MlirOp.
"""

from __future__ import annotations

import math
from typing import Any

import torch

from python_runtime.engine.cache_manager import CacheManager, _as_policy

_DEFAULT_NUM_BLOCKS = 1024


def _source_index(idef: Any) -> int | None:
    src = str(idef.source)
    if src.startswith("operand[") and src.endswith("]"):
        try:
            return int(src[len("operand["):-1])
        except ValueError:
            return None
    return None


class PagedKVIntercept:
    """Cache-policy intercepts of SDPA ops over a device-resident CacheManager.

    Args:
        cache_mgr: the CacheManager holding the policy's slabs.
        intercepts: the policy's intercept specs (SfaInterceptSpec-like:
            slab_id, op_name_pattern, intercept_type, source, param_indices).
        ssa_producer: SSA value name -> (producer function index, output
            index), the executor's map of function outputs
            (mlir_executor.py:105-109).
        replace_inputs: decode as the reference does (gather + substitute
            the SDPA operands) instead of attending from the slabs.
        prefill_from_slabs: answer causal single-request prefill chunks
            with chunked-prefill attention over the slabs (which sees the
            cached prefix and the slabs' quantized values) instead of the
            reference's dense SDPA over the op's own K and V.
    """

    def __init__(self, cache_mgr: CacheManager, intercepts: list[Any], ssa_producer: dict[str, tuple[int, int]],
                 replace_inputs: bool = False, prefill_from_slabs: bool = False) -> None:
        self.cache_mgr = cache_mgr
        self.replace_inputs = replace_inputs
        self.prefill_from_slabs = prefill_from_slabs
        self._by_op: dict[str, list[Any]] = {}
        for idef in intercepts:
            self._by_op.setdefault(idef.op_name_pattern, []).append(idef)
        self._producer = dict(ssa_producer)
        self.block_tables: dict[str, list[int]] = {}
        self.positions: torch.Tensor | None = None
        self.is_decode = False
        # op results[0] (or id) -> {operand index: (slab id, layer)} for run_sdpa
        self._pending: dict[Any, dict[int, tuple[str, int]]] = {}

    @classmethod
    def from_module(cls, module: Any, device: torch.device | str | None = None,
                    replace_inputs: bool = False, prefill_from_slabs: bool = False) -> "PagedKVIntercept | None":
        """Built from a compiled module the way the reference executor sets
        up its cache manager (mlir_executor.py:105-123): the metadata's
        cache_policy and num_blocks, the functions' outputs as producers.
        None when the module has no paged policy."""
        raw = (getattr(module, "metadata", None) or {}).get("cache_policy")
        if not raw:
            return None
        policy = _as_policy(raw)
        if len(policy.slabs) == 0:
            return None
        producer: dict[str, tuple[int, int]] = {}
        for fi, func in enumerate(module.functions):
            for oi, out in enumerate(func.outputs):
                name = out[0]
                producer[name] = (fi, oi)
                producer[name.lstrip("%")] = (fi, oi)
        num_blocks = int(module.metadata.get("num_blocks", _DEFAULT_NUM_BLOCKS))
        mgr = CacheManager(policy, num_blocks=num_blocks, device=device)
        return cls(mgr, list(policy.intercepts), producer, replace_inputs, prefill_from_slabs)

    # ── per-step state (the executor's _block_tables / _current_*) ───────

    def begin_step(self, block_tables: dict[str, list[int]], positions: torch.Tensor | None = None,
                   is_decode: bool = False) -> None:
        """Once per forward: this step's tables, positions and phase; resets
        the sequential layer counters (mlir_executor.py:186-191, 300-303)."""
        self.block_tables = block_tables or {}
        self.positions = positions
        self.is_decode = bool(is_decode)
        self._pending.clear()
        self.cache_mgr.begin_step(self.block_tables)

    def intercepted_ops(self) -> set[str]:
        return set(self._by_op)

    # ── the intercept ────────────────────────────────────────────────────

    @staticmethod
    def _op_key(op: Any) -> Any:
        results = getattr(op, "results", None)
        return results[0] if results else id(op)

    def handle(self, op: Any, ssa_values: dict[str, torch.Tensor]) -> None:
        """The intercept at `op` (reference _handle_cache_intercept): write
        the op's K/V operands into the slabs and, on decode, either record
        the paged attention `run_sdpa` performs or (replace_inputs) gather
        and substitute the operands."""
        for idef in self._by_op.get(op.op_name, []):
            if idef.intercept_type not in ("write", "read_write"):
                continue
            src_idx = _source_index(idef)
            if len(idef.param_indices) >= 2:
                # only the op whose source operand is exactly this producer output
                contract = (int(idef.param_indices[0]), int(idef.param_indices[1]))
                if src_idx is None or src_idx >= len(op.operands):
                    continue
                name = op.operands[src_idx]
                if self._producer.get(name, self._producer.get(name.lstrip("%"))) != contract:
                    continue
            data = self._source(idef, op, ssa_values)
            if data is None:
                continue
            layer = self.cache_mgr.resolve_layer(idef.slab_id)
            positions = self.positions
            if positions is not None:
                flat = positions.squeeze(0) if positions.dim() >= 2 else positions
                self.cache_mgr.write_paged(idef.slab_id, layer, data, flat)
            if idef.intercept_type != "read_write" or not self.block_tables or src_idx is None:
                continue
            if positions is None or positions.numel() == 0:
                continue
            if not self.is_decode:
                if self.prefill_from_slabs:
                    self._pending.setdefault(self._op_key(op), {})[src_idx] = (idef.slab_id, layer)
                continue
            seq_len = int(positions.max().item()) + 1
            if self.replace_inputs or not self._tables_cover(seq_len):
                gathered = self.cache_mgr.read_paged(idef.slab_id, layer, seq_len)
                key = op.operands[src_idx]
                key = key if key in ssa_values else key.lstrip("%")
                if key in ssa_values:
                    dtype = ssa_values[key].dtype
                    if gathered.dim() == 4:
                        gathered = gathered.permute(0, 2, 1, 3)
                    ssa_values[key] = gathered.to(dtype)
                continue
            self._pending.setdefault(self._op_key(op), {})[src_idx] = (idef.slab_id, layer)

    def _tables_cover(self, seq_len: int) -> bool:
        """Whether every request's table holds seq_len tokens, i.e. the
        reference's gather would add no zero rows."""
        bs = self.cache_mgr._block_size
        return all(len(t) * bs >= seq_len for t in self.block_tables.values())

    @staticmethod
    def _source(idef: Any, op: Any, ssa_values: dict[str, torch.Tensor]) -> torch.Tensor | None:
        src_idx = _source_index(idef)
        if src_idx is not None:
            if src_idx < len(op.operands):
                name = op.operands[src_idx]
                return ssa_values.get(name, ssa_values.get(name.lstrip("%")))
            return None
        if idef.source == "output" and getattr(op, "results", None):
            name = op.results[0]
            return ssa_values.get(name, ssa_values.get(name.lstrip("%")))
        return None

    # ── the SDPA call ────────────────────────────────────────────────────

    def run_sdpa(self, op: Any, inputs: list[torch.Tensor], hal: Any, **attrs: Any) -> torch.Tensor:
        """The op's output: attention from the slabs when `handle` recorded
        both K (operand 1) and V (operand 2) for it and the call is one the
        kernels compute exactly as the reference's dense SDPA would, else
        hal.execute(...) as the reference does -- on a decode step over the
        operands the reference's gather would substitute."""
        pending = self._pending.pop(self._op_key(op), None)
        if pending is not None and 1 in pending and 2 in pending and inputs and inputs[0].dim() == 4:
            (k_slab, k_layer), (v_slab, v_layer) = pending[1], pending[2]
            if k_layer == v_layer:
                if self.is_decode:
                    out = self._decode(inputs, k_slab, v_slab, k_layer, attrs)
                    if out is None:
                        inputs = self._gathered(inputs, pending)
                else:
                    out = self._prefill(inputs, k_slab, v_slab, k_layer, attrs)
                if out is not None:
                    return out
        return hal.execute(op.op_name, inputs, **attrs)

    def _gathered(self, inputs: list[torch.Tensor], pending: dict[int, tuple[str, int]]) -> list[torch.Tensor]:
        """`inputs` with K and V replaced as the reference's decode intercept
        replaces them: rows [0, max_position] of every request (sorted ids)
        gathered from the slabs, zero past a request's table."""
        seq_len = int(self.positions.max().item()) + 1
        out = list(inputs)
        for idx in (1, 2):
            slab, layer = pending[idx]
            g = self.cache_mgr.read_paged(slab, layer, seq_len)
            if g.dim() == 4:
                g = g.permute(0, 2, 1, 3)
            out[idx] = g.to(inputs[idx].dtype)
        return out

    @staticmethod
    def _mask_of(inputs: list[torch.Tensor], attrs: dict) -> torch.Tensor | None:
        mask = attrs.get("attn_mask")
        if mask is None and len(inputs) > 3:
            mask = inputs[3]
        return mask

    @classmethod
    def _decode_unmasked(cls, inputs: list[torch.Tensor], attrs: dict) -> bool:
        """Whether the reference's SDPA leaves a single-query decode row
        unmasked: no dropout, is_causal unset, and no mask or a positional
        [.., 1, 1] mask (which its conversion turns into zeros)."""
        if attrs.get("dropout_p") or attrs.get("is_causal"):
            return False
        mask = cls._mask_of(inputs, attrs)
        if mask is None:
            return True
        return bool(mask.dtype.is_floating_point and mask.shape[-1] == 1 and mask.shape[-2] == 1)

    def _decode(self, inputs: list[torch.Tensor], k_slab: str, v_slab: str, layer: int,
                attrs: dict) -> torch.Tensor | None:
        """q [R, Hq, 1, D] (sorted request order, as the reference's gather)
        -> [R, Hq, 1, D] over positions [0, max_position] of every request
        (`handle` records the op only when each table covers them)."""
        mgr = self.cache_mgr
        tables = self.block_tables
        q = inputs[0]
        if q.shape[2] != 1 or q.shape[0] != len(tables) or self.positions is None:
            return None
        if not self._decode_unmasked(inputs, attrs):
            return None
        seq_len = int(self.positions.max().item()) + 1
        if not self._tables_cover(seq_len):
            return None
        lens = [seq_len] * len(tables)
        scale = attrs.get("scale")
        scale = float(scale) if scale is not None else 1.0 / math.sqrt(q.shape[-1])
        out = mgr.attend(q[:, :, 0, :], layer, lens, k_slab=k_slab, v_slab=v_slab, scale=scale)
        return out.unsqueeze(2)

    def _prefill(self, inputs: list[torch.Tensor], k_slab: str, v_slab: str, layer: int,
                 attrs: dict) -> torch.Tensor | None:
        """One request's causal chunk q [1, Hq, L, D] at this step's
        positions -> [1, Hq, L, D]: chunked-prefill attention from the slabs
        (only with prefill_from_slabs)."""
        mgr = self.cache_mgr
        q = inputs[0]
        if q.shape[0] != 1 or len(self.block_tables) != 1 or self.positions is None or attrs.get("dropout_p"):
            return None
        # causal by position: is_causal, or the reference's positional mask
        mask = self._mask_of(inputs, attrs)
        if not (attrs.get("is_causal") or (mask is not None and mask.dtype.is_floating_point)):
            return None
        pos = self.positions.reshape(-1)
        L = q.shape[2]
        if pos.numel() != L or L == 0:
            return None
        kv, vv = mgr.layer_view(k_slab, layer), mgr.layer_view(v_slab, layer)
        kernel_dtypes = {torch.bfloat16: (torch.bfloat16, torch.float8_e4m3fn),
                         torch.float16: (torch.float16, torch.float8_e4m3fn)}
        if kv.dtype not in kernel_dtypes.get(q.dtype, ()) or mgr._block_size != 16:
            return None
        p0 = int(pos[0].item())
        if not bool(torch.equal(pos.cpu(), torch.arange(p0, p0 + L))):
            return None  # the chunk kernel takes consecutive positions
        table = next(iter(self.block_tables.values()))
        dev = kv.device
        tables = torch.tensor([list(table)], dtype=torch.int32).to(dev)
        seq_lens = torch.tensor([p0 + L], dtype=torch.int32).to(dev)
        q_start = torch.tensor([0, L], dtype=torch.int32).to(dev)
        scale = attrs.get("scale")
        scale = float(scale) if scale is not None else 1.0 / math.sqrt(q.shape[-1])
        rows = q[0].permute(1, 0, 2)  # [L, Hq, D]
        try:
            out = mgr.attend_chunks(rows, layer, tables, seq_lens, q_start, k_slab=k_slab, v_slab=v_slab,
                                    scale=scale)
        except NotImplementedError:
            return None  # a layout or shape the chunk kernel does not take
        return out.permute(1, 0, 2).unsqueeze(0)


__all__ = ["PagedKVIntercept"]
