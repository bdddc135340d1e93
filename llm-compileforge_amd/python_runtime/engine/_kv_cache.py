"""Paged KV cache mixin for executors, on the GPU.

Drop-in for the reference's _KVCacheMixin and _normalize_kv_for_cache
(python_runtime/engine/_kv_cache.py:23-186): same attributes, method
names, arguments and semantics.  The combined cache keeps the reference's
logical shape [num_blocks, layers, 2, block_size, kv_heads, head_dim]
(index 0 of dim 2 = keys, 1 = values); prepare_kv_blocks allocates it in
HBM with each (block, layer, K|V) stored head-major ([kv_heads, block_size,
head_dim]), the layout the attention kernels read keys in.  Any other
strides (for example a contiguous tensor of the reference's layout) work
too.

write_kv_to_cache writes a layer's keys and values in two kernel launches
(cf_paged_write) with the reference's placement rule (first table, in
iteration order, that covers the position's block; :68-104);
gather_kv_from_cache gathers them in sorted request order with zeros past
each table (:106-132; cf_paged_gather).  FP8 caches (dtype
torch.float8_e4m3fn, an addition) quantize with per-(layer, K|V, head)
scales, `_kv_scales` [layers, 2, kv_heads], and gather as float32.
attend() (an addition) runs decode attention straight from the cache.
Everything runs on the GPU; a cache that is not on one raises.
"""

from __future__ import annotations

import math

import torch

from cf_hip import ops as _ops
from python_runtime.engine.cache_manager import first_cover_table, normalize_kv, resolve_slots, sorted_table_matrix


class _KVCacheMixin:
    """Paged KV cache read/write methods.

    Requires these attributes on the inheriting class:
        _kv_cache, _block_tables, _block_size, _num_kv_heads, _head_dim
    """

    _kv_cache: torch.Tensor | None
    _block_tables: dict[str, list[int]]
    _block_size: int
    _num_kv_heads: int
    _head_dim: int

    def set_kv_cache(
        self,
        kv_cache: torch.Tensor | None,
        block_tables: dict[str, list[int]] | None = None,
        block_size: int = 16,
        num_kv_heads: int = 0,
        head_dim: int = 0,
    ) -> None:
        self._kv_cache = kv_cache
        self._block_tables = block_tables or {}
        self._block_size = block_size
        self._num_kv_heads = num_kv_heads
        self._head_dim = head_dim

    def prepare_kv_blocks(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int,
        num_blocks: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str | None = None,
    ) -> torch.Tensor:
        """Zeroed cache [num_blocks, num_layers, 2, block_size, num_kv_heads,
        head_dim] on `device` (default the current GPU), stored head-major."""
        if device is None:
            if not torch.cuda.is_available():
                raise RuntimeError("prepare_kv_blocks needs a GPU (no device given and none is visible)")
            device = torch.device("cuda", torch.cuda.current_device())
        storage = torch.zeros(num_blocks, num_layers, 2, num_kv_heads, block_size, head_dim, dtype=dtype,
                              device=device)
        return storage.permute(0, 1, 2, 4, 3, 5)

    def _max_seq_from_tables(self, block_tables: dict[str, list[int]]) -> int:
        total = 0
        for blocks in block_tables.values():
            total = max(total, len(blocks))
        return total * self._block_size

    def _fp8_scales(self) -> torch.Tensor:
        """Per-(layer, K|V, head) scales of an FP8 cache, ones until set."""
        cache = self._kv_cache
        assert cache is not None
        want = (cache.shape[1], 2, cache.shape[4])
        sc = getattr(self, "_kv_scales", None)
        if sc is None or tuple(sc.shape) != want or sc.device != cache.device:
            sc = torch.ones(want, dtype=torch.float32, device=cache.device)
            self._kv_scales = sc
        return sc

    def set_kv_scales(self, scales: torch.Tensor) -> None:
        """Sets an FP8 cache's dequant scales, [layers, 2, kv_heads] (or
        anything that broadcasts to it); rows already written keep their
        codes."""
        dst = self._fp8_scales()
        src = torch.as_tensor(scales, dtype=torch.float32).to(dst.device)
        if not bool(torch.all(torch.isfinite(src) & (src > 0))):
            raise ValueError("FP8 scales must be finite and positive")
        dst.copy_(src.expand_as(dst))

    def _scale_of(self, layer_idx: int, kv: int) -> torch.Tensor | None:
        if self._kv_cache is None or self._kv_cache.dtype != torch.float8_e4m3fn:
            return None
        return self._fp8_scales()[layer_idx, kv]

    def _rows(self, t: torch.Tensor) -> torch.Tensor:
        cache = self._kv_cache
        assert cache is not None
        h, d = cache.shape[4], cache.shape[5]
        t = normalize_kv(t, h, d)
        if t.dim() != 3 or t.shape[1:] != (h, d):
            raise ValueError(f"KV rows {tuple(t.shape)} do not match the cache's ({h}, {d}) heads x dim")
        return t if t.device == cache.device else t.to(cache.device)

    def _write_kv_flat(
        self,
        key: torch.Tensor,
        value: torch.Tensor,
        positions: torch.Tensor,
        block_tables: dict[str, list[int]],
        layer_idx: int,
    ) -> None:
        cache = self._kv_cache
        if cache is None or not block_tables:
            return
        if positions.dim() == 0:
            positions = positions.reshape(1)
        positions = positions.reshape(-1)
        k, v = self._rows(key), self._rows(value)
        if k.shape[0] != positions.numel() or v.shape[0] != positions.numel():
            raise ValueError(f"{positions.numel()} positions for {k.shape[0]} key / {v.shape[0]} value rows")
        cover = first_cover_table(block_tables, cache.shape[0])
        slots = resolve_slots(block_tables, cover, positions, self._block_size, cache.device)
        _ops.paged_write(k, slots, cache[:, layer_idx, 0], self._scale_of(layer_idx, 0))
        _ops.paged_write(v, slots, cache[:, layer_idx, 1], self._scale_of(layer_idx, 1))

    def _gather_kv_flat(
        self,
        block_tables: dict[str, list[int]],
        max_seq_len: int,
        layer_idx: int,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        cache = self._kv_cache
        if cache is None or not block_tables:
            raise RuntimeError("KV cache not initialized")
        _, mat = sorted_table_matrix(block_tables, cache.shape[0])
        tables = torch.from_numpy(mat).to(cache.device)
        key = _ops.paged_gather(cache[:, layer_idx, 0], tables, int(max_seq_len), scale=self._scale_of(layer_idx, 0))
        value = _ops.paged_gather(cache[:, layer_idx, 1], tables, int(max_seq_len),
                                  scale=self._scale_of(layer_idx, 1))
        return key, value

    def write_kv_to_cache(
        self,
        key: torch.Tensor,
        value: torch.Tensor,
        positions: torch.Tensor,
        block_tables: dict[str, list[int]],
        layer_idx: int = 0,
    ) -> None:
        self._write_kv_flat(key, value, positions, block_tables, layer_idx)

    def gather_kv_from_cache(
        self,
        block_tables: dict[str, list[int]],
        max_seq_len: int,
        layer_idx: int = 0,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        return self._gather_kv_flat(block_tables, max_seq_len, layer_idx)

    def attend(
        self,
        q: torch.Tensor,
        block_tables: dict[str, list[int]],
        seq_lens: list[int],
        layer_idx: int = 0,
        scale: float | None = None,
    ) -> torch.Tensor:
        """Decode attention of one query row per request ([requests, q_heads,
        dim], sorted request-id order) over the cached layer; seq_lens in
        the same order."""
        cache = self._kv_cache
        if cache is None or not block_tables:
            raise RuntimeError("KV cache not initialized")
        ids, mat = sorted_table_matrix(block_tables, cache.shape[0])
        if len(seq_lens) != len(ids):
            raise ValueError(f"{len(seq_lens)} lengths for {len(ids)} requests")
        for k, s in zip(ids, seq_lens):
            if s < 0 or s > len(block_tables[k]) * self._block_size:
                raise ValueError(f"sequence length {s} outside request {k!r}'s table")
        dev = cache.device
        tables = torch.from_numpy(mat).to(dev)
        seq_t = torch.tensor([int(s) for s in seq_lens], dtype=torch.int32).to(dev)
        if scale is None:
            scale = 1.0 / math.sqrt(q.shape[-1])
        return _ops.paged_decode(
            q.to(dev), cache[:, layer_idx, 0], cache[:, layer_idx, 1], tables, seq_t, float(scale),
            self._block_size, k_scale=self._scale_of(layer_idx, 0), v_scale=self._scale_of(layer_idx, 1),
        )


def _normalize_kv_for_cache(
    k: torch.Tensor,
    v: torch.Tensor,
    num_kv_heads: int,
    head_dim: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """K/V operands -> [seq, heads, head_dim] (the reference's accepted
    formats, _kv_cache.py:154-186)."""
    return normalize_kv(k, num_kv_heads, head_dim), normalize_kv(v, num_kv_heads, head_dim)


__all__ = ["_KVCacheMixin", "_normalize_kv_for_cache"]
