"""CacheManager: device-resident KV slabs with paged write / read / attend.

Drop-in for the reference's CacheManager
(python_runtime/engine/cache_manager.py:79-267): same constructor, policy
formats (an SfaCachePolicy message or the JSON dict of metadata.json,
converted by `_dict_to_proto_cache_policy`, :30-66; also the serialized
blob and compiler.cache_policy.CachePolicy), slab shapes, per-step state
and read/write semantics.  What differs is where the bytes live and
what moves them:

- Slabs live in HBM (the device given, default the current GPU).  A paged
  slab keeps the reference's logical shape [num_blocks, layers, block_size,
  heads, dim] (`_slabs[name]`), but its storage is laid out for the kernels
  that read it: a slab bound to SDPA operand 1 (keys) stores each (block,
  layer) as [heads, block_size, dim] and one bound to operand 2 (values) as
  [heads, dim, block_size].  Each layer's view is then the decode /
  chunked-prefill kernels' native layout and attention reads the slab in
  place, with no gather.
- write_paged resolves token positions to slots (the reference's rule: the
  first request, in block-table order, whose table covers the position's
  block; uncovered positions are skipped with a warning, :139-171) and
  writes all rows in one kernel launch (cf_paged_write).
- read_paged gathers the requests' blocks, in sorted request-id order with
  zeros past each table (:173-197), in one launch (cf_paged_gather).
- Slabs may be "float8_e4m3fn": rows are quantized on write with per-(layer,
  head) scales (from the policy, else 1.0, settable) and dequantized on read
  (float32 result); attention reads the codes directly.
- attend() (no reference counterpart) runs decode attention for one query
  row per request straight from the slabs.

Every I/O method runs on the GPU through libcf_hip.so and raises if the
slab is not on a GPU or the library is missing; there is no CPU path.
"""

from __future__ import annotations

import logging
import math
from typing import Any

import numpy as np
import torch

from cf_hip import ops as _ops
from compiler.sfa_cache_proto import SfaCachePolicy, SfaInterceptSpec, SfaSlabSpec

_logger = logging.getLogger(__name__)

_ROLE_KEY, _ROLE_VALUE, _ROLE_PLAIN = "k", "v", "plain"


# Cache policy types (the reference's proto-backed dataclasses).


def _dict_to_proto_cache_policy(raw: dict[str, Any]) -> SfaCachePolicy:
    """JSON cache_policy dict (metadata.json) -> SfaCachePolicy message, with
    the reference's field mapping and defaults (cache_manager.py:30-66);
    an FP8 slab's "scales" [layers][heads] go to SlabSpec.scales."""
    block_size = int(raw.get("block_size", 16))
    policy = SfaCachePolicy()
    policy.block_size = block_size
    policy.max_requests = int(raw.get("max_requests", 256))
    for s in raw.get("slabs", []):
        dims = s["dims"]
        slab = policy.slabs.add()
        slab.name = s["slab_id"]
        slab.slab_type = s["storage"]
        slab.layout = s.get("layout", "")
        slab.dtype = s.get("dtype", "float32")
        slab.block_size = block_size
        slab.num_layers = int(dims.get("layers", 0))
        slab.num_heads = int(dims.get("heads", 0))
        slab.head_dim = int(dims.get("dim", 0))
        if s.get("scales") is not None:
            slab.scales.extend(float(x) for row in s["scales"] for x in row)
    for i in raw.get("intercepts", []):
        spec = policy.intercepts.add()
        spec.slab_id = i["slab_id"]
        spec.op_name_pattern = i["op_name"]
        spec.intercept_type = i["direction"]
        spec.source = i.get("source", "")
        spec.layer = i.get("layer", "sequential")
        for key in ("func_index", "output_index"):
            if i.get(key) is not None:
                spec.param_indices.append(int(i[key]))
    return policy


def _as_policy(policy: Any) -> Any:
    """Accepted policy forms: an SfaCachePolicy message (this package's or
    protoc-generated), its serialized bytes, the metadata.json dict, or a
    compiler.cache_policy.CachePolicy."""
    if isinstance(policy, (bytes, bytearray, memoryview)):
        msg = SfaCachePolicy()
        msg.ParseFromString(bytes(policy))
        return msg
    if isinstance(policy, dict):
        return _dict_to_proto_cache_policy(policy)
    if hasattr(policy, "to_dict") and not hasattr(policy, "SerializeToString"):
        return _dict_to_proto_cache_policy(policy.to_dict())
    return policy


def _dtype_from_str(name: str) -> torch.dtype:
    """Slab dtype by name; unknown names give float32 as in the reference
    (cache_manager.py:69-76).  "float8_e4m3fn" / "fp8_e4m3" add FP8 slabs."""
    mapping: dict[str, torch.dtype] = {
        "float32": torch.float32,
        "float16": torch.float16,
        "bfloat16": torch.bfloat16,
        "float64": torch.float64,
        "float8_e4m3fn": torch.float8_e4m3fn,
        "fp8_e4m3": torch.float8_e4m3fn,
    }
    return mapping.get(name, torch.float32)


# Host-side addressing: pure functions, no device work.


def first_cover_table(block_tables: dict[str, list[int]], num_blocks: int) -> np.ndarray:
    """Physical block of each logical block index under the reference's
    write rule: index j goes to the first table (in iteration order) longer
    than j (cache_manager.py:157-162).  Ids are checked against the slab
    and negative ids wrap as torch indexing does; out-of-range ids raise
    IndexError like the reference's slab assignment."""
    longest = max((len(b) for b in block_tables.values()), default=0)
    out = np.empty(longest, dtype=np.int64)
    covered = 0
    for blocks in block_tables.values():
        n = len(blocks)
        if n > covered:
            ids = np.asarray(blocks[covered:n], dtype=np.int64)
            bad = (ids < -num_blocks) | (ids >= num_blocks)
            if bad.any():
                raise IndexError(f"block id {int(ids[bad][0])} out of range for {num_blocks} blocks")
            out[covered:n] = ids % num_blocks
            covered = n
    return out


def slots_for_positions(cover: np.ndarray, positions: np.ndarray, block_size: int) -> np.ndarray:
    """Slot block * block_size + offset per position; -1 where no table covers it."""
    pos = np.asarray(positions, dtype=np.int64).reshape(-1)
    bidx = pos // block_size
    ok = (pos >= 0) & (bidx < cover.shape[0])
    slots = np.full(pos.shape, -1, dtype=np.int64)
    slots[ok] = cover[bidx[ok]] * block_size + pos[ok] % block_size
    return slots


def resolve_slots(
    block_tables: dict[str, list[int]], cover: np.ndarray, positions: torch.Tensor, block_size: int,
    device: torch.device,
) -> torch.Tensor:
    """int64 slots on `device` for token `positions` ([T]) under `cover`
    (first_cover_table of `block_tables`); a negative slot marks a skipped
    position.

    Host positions resolve on the host: negative ones raise ValueError,
    uncovered ones are logged as skipped (the reference's warning,
    cache_manager.py:163-171), and of several rows bound for one slot only
    the last is written.  Device positions resolve on their device without a
    sync: negative or uncovered ones are skipped silently, and which of
    several rows bound for one slot lands is unspecified."""
    bs = block_size
    if positions.device.type == "cpu":
        pos_np = positions.to(torch.int64).numpy()
        if (pos_np < 0).any():
            raise ValueError("write: positions must be non-negative")
        slots_np = slots_for_positions(cover, pos_np, bs)
        # Rows landing on one slot: the last one wins, as in the reference's
        # sequential loop (the kernel writes rows in no fixed order).
        live = np.nonzero(slots_np >= 0)[0]
        if live.size > 1:
            rev = live[::-1]
            _, first_in_rev = np.unique(slots_np[rev], return_index=True)
            drop = np.setdiff1d(live, rev[first_in_rev])
            slots_np[drop] = -2
        for i in np.nonzero(slots_np == -1)[0]:
            pos = int(pos_np[i])
            _logger.warning(
                "KV write skipped: position %d (block_idx=%d) not covered by any request's block table "
                "(table lengths: %s).",
                pos, pos // bs, [len(b) for b in block_tables.values()],
            )
        return torch.from_numpy(slots_np).to(device)
    cov = torch.from_numpy(np.append(cover, -1)).to(positions.device)
    pos = positions.to(torch.int64)
    bidx = torch.where(pos >= 0, pos // bs, cover.shape[0]).clamp(max=cover.shape[0])
    blk = cov[bidx]
    return torch.where(blk >= 0, blk * bs + pos % bs, torch.full_like(pos, -1)).to(device)


def sorted_table_matrix(block_tables: dict[str, list[int]], num_blocks: int) -> tuple[list[str], np.ndarray]:
    """Requests in sorted id order and their tables as an int32 [R, Mb]
    matrix padded with -1 (read order of cache_manager.py:190)."""
    items = sorted(block_tables.items())
    width = max((len(b) for _, b in items), default=0)
    mat = np.full((len(items), max(width, 1)), -1, dtype=np.int32)
    for r, (_, blocks) in enumerate(items):
        if blocks:
            ids = np.asarray(blocks, dtype=np.int64)
            bad = (ids < -num_blocks) | (ids >= num_blocks)
            if bad.any():
                raise IndexError(f"block id {int(ids[bad][0])} out of range for {num_blocks} blocks")
            mat[r, : len(blocks)] = ids % num_blocks
    return [k for k, _ in items], mat


def normalize_kv(t: torch.Tensor, num_heads: int, head_dim: int) -> torch.Tensor:
    """SDPA K/V operand -> [seq, heads, dim] (the reference's accepted
    formats, cache_manager.py:222-237): [1, H, S, D] / [1, S, H, D] squeeze
    the batch, [H, S, D] permutes, [S, H*D] and [., H*D] reshape."""
    if t.dim() >= 4 and t.shape[0] == 1:
        t = t.squeeze(0)
    if t.dim() == 3 and t.shape[0] == num_heads and t.shape[-1] == head_dim:
        t = t.permute(1, 0, 2)
    elif t.dim() == 3 and t.shape[1] == num_heads and t.shape[-1] == head_dim:
        pass
    elif t.dim() in (2, 3) and t.shape[-1] == num_heads * head_dim:
        t = t.reshape(-1, num_heads, head_dim)
    return t


def _slab_role(spec: Any, intercepts: list[Any]) -> str:
    """Keys (SDPA operand 1) or values (operand 2), from the slab's
    intercepts, else from its name."""
    for i in intercepts:
        if i.slab_id == spec.name:
            if i.source == "operand[1]":
                return _ROLE_KEY
            if i.source == "operand[2]":
                return _ROLE_VALUE
    name = spec.name.lower()
    if name in ("k", "key", "keys", "k_cache", "key_cache"):
        return _ROLE_KEY
    if name in ("v", "value", "values", "v_cache", "value_cache"):
        return _ROLE_VALUE
    return _ROLE_PLAIN


# The slab owner.


class CacheManager:
    """Manages cache slabs and positional I/O at runtime (device-resident).

    Args:
        policy: SfaCachePolicy message, its serialized bytes, the
            metadata.json dict or a compiler.cache_policy.CachePolicy;
            FP8 slabs take their scales from it (1.0 where absent).
        num_blocks: physical blocks per paged slab.
        device: where the slabs live (default: the current GPU).
    """

    def __init__(self, policy: Any, num_blocks: int, device: torch.device | str | None = None) -> None:
        policy = _as_policy(policy)
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("CacheManager needs a GPU (no device given and none is visible)")
            device = torch.device("cuda", torch.cuda.current_device())
        self._policy = policy
        self._num_blocks = int(num_blocks)
        self._block_size = int(policy.block_size)
        self._max_requests = int(policy.max_requests)
        self._device = torch.device(device)

        self._slabs: dict[str, torch.Tensor] = {}
        self._specs: dict[str, Any] = {}
        self._roles: dict[str, str] = {}
        self._scales: dict[str, torch.Tensor] = {}
        self._layer_counters: dict[str, int] = {}
        self._block_tables: dict[str, list[int]] = {}
        self._cover: np.ndarray | None = None
        self._sorted: tuple[list[str], torch.Tensor, list[int]] | None = None
        self._attend_meta: tuple[tuple[int, ...], torch.Tensor, torch.Tensor | None] | None = None

        intercepts = list(getattr(policy, "intercepts", []))
        for spec in policy.slabs:
            self._specs[spec.name] = spec
            self._roles[spec.name] = _slab_role(spec, intercepts)
            self._slabs[spec.name] = self._allocate_slab(spec)
            self._layer_counters[spec.name] = 0
            if self._slabs[spec.name].dtype == torch.float8_e4m3fn:
                shape = (max(spec.num_layers, 1), max(spec.num_heads, 1))
                stored = list(getattr(spec, "scales", []))
                if stored:
                    if len(stored) != shape[0] * shape[1]:
                        raise ValueError(f"slab {spec.name!r}: {len(stored)} scales for {shape[0]} x {shape[1]}")
                    sc = torch.tensor(stored, dtype=torch.float32).reshape(shape)
                    if not bool(torch.all(torch.isfinite(sc) & (sc > 0))):
                        raise ValueError(f"slab {spec.name!r}: FP8 scales must be finite and positive")
                else:
                    sc = torch.ones(shape, dtype=torch.float32)
                self._scales[spec.name] = sc.to(self._device)

    def _allocate_slab(self, spec: Any) -> torch.Tensor:
        dtype = _dtype_from_str(spec.dtype)
        nb, L, bs, H, D = self._num_blocks, spec.num_layers, self._block_size, spec.num_heads, spec.head_dim
        if spec.slab_type == "paged":
            role = self._roles[spec.name]
            if role == _ROLE_KEY:
                # storage [NB, L, H, bs, D] -> logical [NB, L, bs, H, D]
                return torch.zeros(nb, L, H, bs, D, dtype=dtype, device=self._device).permute(0, 1, 3, 2, 4)
            if role == _ROLE_VALUE:
                # storage [NB, L, H, D, bs] -> logical [NB, L, bs, H, D]
                return torch.zeros(nb, L, H, D, bs, dtype=dtype, device=self._device).permute(0, 1, 4, 2, 3)
            return torch.zeros(nb, L, bs, H, D, dtype=dtype, device=self._device)
        if spec.slab_type == "fixed":
            return torch.zeros(self._max_requests, L, D, dtype=dtype, device=self._device)
        raise ValueError(f"Unknown storage type: {spec.slab_type}")

    # Step bookkeeping: the active request and its positions.

    def begin_step(self, block_tables: dict[str, list[int]]) -> None:
        """Sets this step's block tables and resets the layer counters."""
        self._block_tables = block_tables
        self._cover = None
        self._sorted = None
        self._attend_meta = None
        for key in self._layer_counters:
            self._layer_counters[key] = 0

    def resolve_layer(self, slab_id: str) -> int:
        """Return and increment the sequential layer counter for *slab_id*."""
        layer = self._layer_counters[slab_id]
        self._layer_counters[slab_id] += 1
        return layer

    def _cover_table(self) -> np.ndarray:
        if self._cover is None:
            self._cover = first_cover_table(self._block_tables, self._num_blocks)
        return self._cover

    def _sorted_tables(self) -> tuple[list[str], torch.Tensor, list[int]]:
        """(sorted request ids, device int32 [R, Mb] tables, table lengths)."""
        if self._sorted is None:
            ids, mat = sorted_table_matrix(self._block_tables, self._num_blocks)
            lens = [len(self._block_tables[k]) for k in ids]
            self._sorted = (ids, torch.from_numpy(mat).to(self._device), lens)
        return self._sorted

    # Per-(layer, KV head) FP8 dequant scales of the paged slabs.

    def kv_scales(self, slab_id: str) -> torch.Tensor:
        """Per-(layer, head) float32 dequant scales [L, H] of an FP8 slab."""
        if slab_id not in self._scales:
            raise ValueError(f"slab {slab_id!r} is not an FP8 slab")
        return self._scales[slab_id]

    def set_kv_scales(self, slab_id: str, scales: torch.Tensor, layer_idx: int | None = None) -> None:
        """Sets an FP8 slab's scales ([L, H], or [H] / scalar for one layer).
        Rows already written keep the codes of the old scales."""
        dst = self.kv_scales(slab_id)
        src = torch.as_tensor(scales, dtype=torch.float32).to(self._device)
        if not bool(torch.all(torch.isfinite(src) & (src > 0))):
            raise ValueError("FP8 scales must be finite and positive")
        if layer_idx is None:
            dst.copy_(src.expand_as(dst))
        else:
            dst[layer_idx].copy_(src.reshape(-1).expand_as(dst[layer_idx]))

    def calibrate_kv_scales(self, slab_id: str, layer_idx: int, sample: torch.Tensor) -> torch.Tensor:
        """Sets layer `layer_idx`'s scales to amax / 448 per head of `sample`
        ([T, H, D] or any format write_paged accepts), on the GPU
        (FP8KVCacheQuantizer.compute_scale, compiler/quantize/fp8_kv_cache.py:77-83)."""
        spec = self._specs[slab_id]
        x = normalize_kv(sample, spec.num_heads, spec.head_dim)
        sc = _ops.fp8_amax_scale(x)
        self.kv_scales(slab_id)[layer_idx].copy_(sc.reshape(-1))
        return sc

    # Writing and reading K/V rows through block tables.

    def layer_view(self, slab_id: str, layer_idx: int) -> torch.Tensor:
        """Layer `layer_idx` of a paged slab as [num_blocks, block_size, heads, dim]."""
        return self._slabs[slab_id][:, layer_idx]

    def write_paged(self, slab_id: str, layer_idx: int, data: torch.Tensor, positions: torch.Tensor) -> None:
        """Writes token rows `data` at `positions` of this step's requests.

        Positions on the host are resolved to slots on the host, and
        positions no table covers are skipped with a warning (negative
        positions raise ValueError); positions already on the GPU are
        resolved there, and uncovered or negative ones are skipped without a
        warning, which would need a device sync."""
        slab = self._slabs[slab_id]
        bt = self._block_tables
        if not bt or slab is None:
            return
        spec = self._specs[slab_id]
        rows = normalize_kv(data, spec.num_heads, spec.head_dim)
        if rows.dim() != 3:
            raise ValueError(f"write_paged: cannot read {tuple(data.shape)} as [seq, {spec.num_heads}, {spec.head_dim}]")
        if positions.dim() == 0:
            positions = positions.reshape(1)
        positions = positions.reshape(-1)
        if positions.numel() != rows.shape[0]:
            raise ValueError(f"write_paged: {positions.numel()} positions for {rows.shape[0]} rows")
        bs = self._block_size
        slots = resolve_slots(bt, self._cover_table(), positions, bs, self._device)
        if rows.device != self._device:
            rows = rows.to(self._device)
        view = self.layer_view(slab_id, layer_idx)
        if view.dtype == torch.float64:
            keep = slots >= 0
            s = slots[keep]
            view[s // bs, s % bs] = rows[keep].to(torch.float64)
            return
        sc = self._scales[slab_id][layer_idx] if slab_id in self._scales else None
        _ops.paged_write(rows, slots, view, sc)

    def read_paged(self, slab_id: str, layer_idx: int, max_seq_len: int) -> torch.Tensor:
        """Dense [requests, max_seq_len, heads, dim] rows of this step's
        requests (sorted request-id order, zeros past a table), in the slab
        dtype (float32 for an FP8 slab)."""
        slab = self._slabs[slab_id]
        if slab is None or not self._block_tables:
            raise RuntimeError("Paged slab read requested without active block tables")
        _, tables, _ = self._sorted_tables()
        view = self.layer_view(slab_id, layer_idx)
        if view.dtype == torch.float64:
            # No float64 kernel: the same gather with torch indexing on the device.
            bs = self._block_size
            s = torch.arange(int(max_seq_len), device=self._device)
            ids = tables[:, (s // bs).clamp(max=tables.shape[1] - 1)].long()
            valid = (ids >= 0) & (s // bs < tables.shape[1])
            rows = view[ids.clamp(min=0), (s % bs).expand_as(ids)]
            return torch.where(valid[..., None, None], rows, torch.zeros((), dtype=rows.dtype, device=rows.device))
        sc = self._scales[slab_id][layer_idx] if slab_id in self._scales else None
        return _ops.paged_gather(view, tables, int(max_seq_len), scale=sc)

    # Decode and chunked-prefill attention straight over the slabs.

    def attend(
        self,
        q: torch.Tensor,
        layer_idx: int,
        seq_lens: list[int] | torch.Tensor | None = None,
        k_slab: str = "k",
        v_slab: str = "v",
        scale: float | None = None,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Decode attention of one query row per request, read straight
        from the paged slabs (no gather).

        q: [requests, q_heads, dim] in sorted request-id order (the order
        of read_paged).  seq_lens: tokens per request (default: every table
        full, len(table) * block_size).  scale: softmax scale (default
        1/sqrt(dim)).  Returns [requests, q_heads, dim] in q's dtype.
        """
        if not self._block_tables:
            raise RuntimeError("attend requested without active block tables")
        ids, tables, lens = self._sorted_tables()
        bs = self._block_size
        if seq_lens is None:
            seq_list = [n * bs for n in lens]
        elif isinstance(seq_lens, torch.Tensor):
            seq_list = [int(x) for x in seq_lens.reshape(-1).tolist()]
        else:
            seq_list = [int(x) for x in seq_lens]
        if len(seq_list) != len(ids) or q.shape[0] != len(ids):
            raise ValueError(f"attend: {len(ids)} requests, {q.shape[0]} query rows, {len(seq_list)} lengths")
        for n, s in zip(lens, seq_list):
            if s < 0 or s > n * bs:
                raise ValueError(f"attend: sequence length {s} outside the table's {n * bs} slots")
        kv = self.layer_view(k_slab, layer_idx)
        vv = self.layer_view(v_slab, layer_idx)
        ks = self._scales[k_slab][layer_idx] if k_slab in self._scales else None
        vs = self._scales[v_slab][layer_idx] if v_slab in self._scales else None
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        dev = self._device
        key = tuple(seq_list)
        if self._attend_meta is None or self._attend_meta[0] != key:
            # Lengths and the shared-prefix statement are per step, not per layer.
            host_tables = [[t % self._num_blocks for t in self._block_tables[k]] for k in ids]
            sp = _ops.shared_prefix_lens(host_tables, seq_list, bs)
            seq_t = torch.tensor(seq_list, dtype=torch.int32).to(dev)
            sp_t = torch.tensor(sp, dtype=torch.int32).to(dev) if any(sp) else None
            self._attend_meta = (key, seq_t, sp_t)
        _, seq_t, sp_t = self._attend_meta
        if q.device != dev:
            q = q.to(dev)
        return _ops.paged_decode(
            q, kv, vv, tables, seq_t, float(scale), bs, k_scale=ks, v_scale=vs, out=out, shared_prefix_lens=sp_t
        )

    def write_slots(self, slab_id: str, layer_idx: int, data: torch.Tensor, slots: torch.Tensor | np.ndarray) -> None:
        """Writes token rows at explicit slots (block * block_size + offset),
        e.g. those BlockManager.prepare_writes returns; negative slots are
        skipped."""
        spec = self._specs[slab_id]
        rows = normalize_kv(data, spec.num_heads, spec.head_dim)
        if rows.dim() != 3:
            raise ValueError(f"write_slots: cannot read {tuple(data.shape)} as [seq, {spec.num_heads}, {spec.head_dim}]")
        slots = torch.as_tensor(slots).reshape(-1).to(self._device)
        if slots.numel() != rows.shape[0]:
            raise ValueError(f"write_slots: {slots.numel()} slots for {rows.shape[0]} rows")
        if rows.device != self._device:
            rows = rows.to(self._device)
        view = self.layer_view(slab_id, layer_idx)
        if view.dtype == torch.float64:
            bs = self._block_size
            keep = slots >= 0
            s = slots[keep]
            view[s // bs, s % bs] = rows[keep].to(torch.float64)
            return
        sc = self._scales[slab_id][layer_idx] if slab_id in self._scales else None
        _ops.paged_write(rows, slots, view, sc)

    def attend_rows(
        self,
        q: torch.Tensor,
        layer_idx: int,
        block_tables: torch.Tensor,
        seq_lens: torch.Tensor,
        shared_prefix_lens: torch.Tensor | None = None,
        k_slab: str = "k",
        v_slab: str = "v",
        scale: float | None = None,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Decode attention from the slabs with device-resident tables (e.g.
        BlockManager.sync_device): q [rows, q_heads, dim], block_tables int32
        [rows, cols], seq_lens int32 [rows] (rows of length 0 give zeros)."""
        kv = self.layer_view(k_slab, layer_idx)
        vv = self.layer_view(v_slab, layer_idx)
        ks = self._scales[k_slab][layer_idx] if k_slab in self._scales else None
        vs = self._scales[v_slab][layer_idx] if v_slab in self._scales else None
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        return _ops.paged_decode(q, kv, vv, block_tables, seq_lens, float(scale), self._block_size, k_scale=ks,
                                 v_scale=vs, out=out, shared_prefix_lens=shared_prefix_lens)

    def attend_chunks(
        self,
        q: torch.Tensor,
        layer_idx: int,
        block_tables: torch.Tensor,
        seq_lens: torch.Tensor,
        q_start: torch.Tensor,
        k_slab: str = "k",
        v_slab: str = "v",
        scale: float | None = None,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Chunked-prefill attention from the slabs: q [Tq, q_heads, dim]
        holds the rows of N chunks (chunk n owns rows [q_start[n],
        q_start[n+1])), whose K/V are already written; row i of a chunk of L
        rows sits at position seq_lens[n] - L + i and sees positions up to
        it.  block_tables int32 [N, cols]; seq_lens int32 [N]."""
        kv = self.layer_view(k_slab, layer_idx)
        vv = self.layer_view(v_slab, layer_idx)
        ks = self._scales[k_slab][layer_idx] if k_slab in self._scales else None
        vs = self._scales[v_slab][layer_idx] if v_slab in self._scales else None
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        return _ops.prefill_chunk(q, kv, vv, block_tables, seq_lens, q_start, float(scale), self._block_size,
                                  k_scale=ks, v_scale=vs, out=out)

    def paged_slabs(self) -> list[torch.Tensor]:
        """Every paged slab (all layers), e.g. for BlockManager.copy_blocks."""
        return [t for name, t in self._slabs.items() if self._specs[name].slab_type == "paged"]

    # Fixed-size (per-slot) state slabs: [slots, layers, ...] rows.

    def write_fixed(self, slab_id: str, slot: int, layer_idx: int, data: torch.Tensor) -> None:
        slab = self._slabs[slab_id]
        slab[slot, layer_idx] = data.float().to(slab.device)

    def read_fixed(self, slab_id: str, slot: int, layer_idx: int) -> torch.Tensor:
        return self._slabs[slab_id][slot, layer_idx]

    def _normalize_kv(self, data: torch.Tensor, slab_id: str) -> torch.Tensor:
        spec = self._specs[slab_id]
        return normalize_kv(data, spec.num_heads, spec.head_dim)

    @staticmethod
    def _pos_to_list(positions: torch.Tensor) -> list[int]:
        """Token positions as Python ints, in order (a 0-d tensor gives one)."""
        return [int(v) for v in positions.reshape(-1).tolist()]

    # Policy-derived geometry (reference cache_manager.py:241-267): the
    # first positive value among the policy's slabs, paged slabs only for
    # the head geometry; 0 when no slab states it.

    def _policy_value(self, field: str, paged_only: bool) -> int:
        values = (int(getattr(spec, field)) for spec in self._policy.slabs
                  if not paged_only or spec.slab_type == "paged")
        return next((v for v in values if v > 0), 0)

    @property
    def has_paged_cache(self) -> bool:
        """Whether the policy declares at least one paged (block-table) slab."""
        return any(spec.slab_type == "paged" for spec in self._policy.slabs)

    def configured_kv_heads(self) -> int:
        return self._policy_value("num_heads", paged_only=True)

    def configured_head_dim(self) -> int:
        return self._policy_value("head_dim", paged_only=True)

    def configured_num_layers(self) -> int:
        return self._policy_value("num_layers", paged_only=False)


__all__ = [
    "CacheManager",
    "SfaCachePolicy",
    "SfaInterceptSpec",
    "SfaSlabSpec",
    "_dict_to_proto_cache_policy",
    "first_cover_table",
    "normalize_kv",
    "resolve_slots",
    "slots_for_positions",
    "sorted_table_matrix",
]
