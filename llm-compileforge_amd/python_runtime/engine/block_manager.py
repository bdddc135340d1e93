"""Paged KV block manager over the native block pool (libcf_hip.so).

`BlockManager` (alias `PyBlockManager`) is a drop-in for the reference's
PyBlockManager (runtime/src/lib.rs:82-168, over BlockManager,
runtime/src/cache/block.rs:78-352): the same constructor, methods,
properties, block-id allocation order and exceptions (allocate /
ensure_blocks: RuntimeError when the pool is exhausted; share_prefix:
ValueError; get_blocks: KeyError), so the reference's RadixCache and
scheduler logic run on it unchanged.  The bookkeeping lives in C++
(csrc/block_pool.hip); Python only marshals.

Additions for the GPU path (no reference counterparts):

- `prepare_writes([(request_id, start, count), ...])` makes the blocks a
  step writes exclusively owned, replacing shared ones (refcount > 1: a
  radix-shared prefix, possibly a partial last block) by fresh blocks, and
  returns the new tokens' slots plus the (old, new) copy-on-write pairs.
  `copy_blocks(pairs, caches)` performs those copies on the device for every
  cache tensor (each layer's K and V, or CacheManager slabs).
- `bind_device(rows, cols)` keeps an int32 block table [rows, cols] and
  lengths [rows] on the GPU; `sync_device()` uploads only the cells that
  changed since the last sync (one small copy and one scatter kernel)
  instead of rebuilding and uploading every table each step;
  `shared_prefix_lens()` gives the decode kernel's shared-prefix statement
  for the rows.
"""

from __future__ import annotations

import ctypes
from typing import Iterable

import numpy as np
import torch

from cf_hip import ops as _ops
from cf_hip._abi import check, lib


def _b(s: str) -> bytes:
    return s.encode("utf-8")


class BlockManager:
    """Reference-counted paged block pool with per-request block tables.

    Args:
        num_blocks: physical blocks in the pool (> 0).
        block_size: tokens per block (> 0).
    """

    def __init__(self, num_blocks: int, block_size: int) -> None:
        h = ctypes.c_void_p()
        check(lib().cf_bp_create(int(num_blocks), int(block_size), ctypes.byref(h)), "BlockManager")  # ValueError
        self._h = h
        self._num_blocks = int(num_blocks)
        self._block_size = int(block_size)
        self._table: torch.Tensor | None = None
        self._lens: torch.Tensor | None = None
        # two pinned staging buffers for the deltas, each reused once its copy has run
        self._stage: list[torch.Tensor | None] = [None, None]
        self._stage_done: list[torch.cuda.Event | None] = [None, None]
        self._stage_k = 0
        self._delta_buf = np.empty((4096, 4), dtype=np.int32)

    def __del__(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                lib().cf_bp_destroy(h)
            except Exception:
                pass
            self._h = ctypes.c_void_p()

    # ── reference API (PyBlockManager) ─────────────────────

    @property
    def block_size(self) -> int:
        return self._block_size

    @property
    def num_blocks(self) -> int:
        return self._num_blocks

    def _ids_out(self, n: int) -> tuple[np.ndarray, ctypes.c_int64]:
        return np.empty(max(n, 1), dtype=np.int32), ctypes.c_int64(0)

    def allocate(self, request_id: str, num_tokens: int) -> list[int]:
        """Blocks for a new request's first num_tokens tokens
        (block.rs:145-173); RuntimeError when the pool is exhausted or the
        id already has blocks."""
        if num_tokens < 0:
            raise OverflowError("num_tokens must be non-negative")
        need = -(-int(num_tokens) // self._block_size)
        buf, n = self._ids_out(need)
        rc = lib().cf_bp_allocate(self._h, _b(request_id), int(num_tokens), buf.ctypes.data, buf.size,
                                  ctypes.byref(n))
        check(rc, "allocate")
        return buf[: n.value].tolist()

    def free(self, request_id: str) -> None:
        """Releases a request's blocks (shared ones only lose a reference)."""
        check(lib().cf_bp_free(self._h, _b(request_id)), "free")

    def free_block(self, block_id: int) -> None:
        """Releases one reference to one block (radix-cache eviction)."""
        check(lib().cf_bp_free_block(self._h, int(block_id)), "free_block")

    def get_blocks(self, request_id: str) -> list[int]:
        """A request's block table; KeyError for an unknown id."""
        n = ctypes.c_int64(0)
        check(lib().cf_bp_get_blocks(self._h, _b(request_id), None, 0, ctypes.byref(n)), "get_blocks")
        buf, n2 = self._ids_out(n.value)
        check(lib().cf_bp_get_blocks(self._h, _b(request_id), buf.ctypes.data, buf.size, ctypes.byref(n2)),
              "get_blocks")
        return buf[: n2.value].tolist()

    def assign_cached_blocks(self, request_id: str, block_ids: list[int]) -> None:
        """Prepends prefix-cache blocks to a request's table, one reference each."""
        ids = np.asarray(list(block_ids), dtype=np.int32)
        check(lib().cf_bp_assign_cached_blocks(self._h, _b(request_id), ids.ctypes.data if ids.size else None,
                                               int(ids.size)), "assign_cached_blocks")

    def ensure_blocks(self, request_id: str, target_tokens: int) -> None:
        """Grows a request's table to cover target_tokens tokens."""
        check(lib().cf_bp_ensure_blocks(self._h, _b(request_id), int(target_tokens)), "ensure_blocks")

    def share_prefix(self, src_request_id: str, dst_request_id: str, prefix_len: int) -> list[int]:
        """Gives dst the blocks holding src's first prefix_len tokens; ValueError on misuse."""
        need = -(-int(prefix_len) // self._block_size)
        buf, n = self._ids_out(need)
        rc = lib().cf_bp_share_prefix(self._h, _b(src_request_id), _b(dst_request_id), int(prefix_len),
                                      buf.ctypes.data, buf.size, ctypes.byref(n))
        if rc != 0:
            try:
                check(rc, "share_prefix")
            except (KeyError, RuntimeError) as e:
                raise ValueError(str(e.args[0] if e.args else e)) from None
        return buf[: n.value].tolist()

    def num_free_blocks(self) -> int:
        out = ctypes.c_int64(0)
        check(lib().cf_bp_num_free(self._h, ctypes.byref(out)), "num_free_blocks")
        return int(out.value)

    def num_allocated_blocks(self) -> int:
        return self._num_blocks - self.num_free_blocks()

    def utilization(self) -> float:
        return self.num_allocated_blocks() / self._num_blocks

    def increment_ref_count(self, block_id: int) -> None:
        check(lib().cf_bp_increment_ref_count(self._h, int(block_id)), "increment_ref_count")

    def ref_count(self, block_id: int) -> int:
        out = ctypes.c_int64(0)
        check(lib().cf_bp_ref_count(self._h, int(block_id), ctypes.byref(out)), "ref_count")
        return int(out.value)

    # ── writes with copy-on-write ──────────────────────────

    def prepare_writes(self, writes: Iterable[tuple[str, int, int]]) -> tuple[np.ndarray, np.ndarray]:
        """For writes [(request_id, start, count), ...]: grows tables, makes
        every touched block exclusively owned (copy-on-write of shared
        blocks) and returns (slots int64 [sum(count)], copies int32 [n, 2]
        of (old, new) blocks).  All-or-nothing: RuntimeError when the pool
        cannot cover every write."""
        ws = list(writes)
        batch = RequestBatch([w[0] for w in ws])
        start = np.fromiter((w[1] for w in ws), dtype=np.int64, count=len(ws))
        count = np.fromiter((w[2] for w in ws), dtype=np.int64, count=len(ws))
        return self.prepare_writes_batch(batch, start, count)

    def prepare_writes_batch(self, batch: "RequestBatch", start: np.ndarray,
                             count: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """prepare_writes for a fixed list of requests (encoded once, reused
        every step): start / count int64 [len(batch)]."""
        n = len(batch)
        start = np.ascontiguousarray(start, dtype=np.int64)
        count = np.ascontiguousarray(count, dtype=np.int64)
        if start.shape != (n,) or count.shape != (n,):
            raise ValueError(f"start and count must have {n} entries")
        total = int(count.sum())
        bs = self._block_size
        live = count > 0
        # at most one copy per block a write touches
        cap = int(((start + count - 1) // bs - start // bs + 1)[live].sum()) if n else 0
        slots = np.empty(max(total, 1), dtype=np.int64)
        copies = np.empty((max(cap, 1), 2), dtype=np.int32)
        nc = ctypes.c_int64(0)
        rc = lib().cf_bp_prepare_writes(self._h, n, batch.c_ids, start.ctypes.data, count.ctypes.data,
                                        slots.ctypes.data, copies.ctypes.data, copies.shape[0], ctypes.byref(nc))
        check(rc, "prepare_writes")
        return slots[:total], copies[: nc.value]

    def set_len(self, request_id: str, tokens: int) -> None:
        """Sets a request's token count (its device row length)."""
        check(lib().cf_bp_set_len(self._h, _b(request_id), int(tokens)), "set_len")

    @staticmethod
    def copy_blocks(copies: np.ndarray | torch.Tensor, caches: Iterable[torch.Tensor]) -> None:
        """Device copies of copy-on-write pairs into every cache tensor whose
        dim 0 is the block (per-layer K/V caches, CacheManager slabs, the
        combined [NB, L, 2, ...] cache)."""
        caches = list(caches)
        if len(copies) == 0 or not caches:
            return
        dev = caches[0].device
        pairs = torch.as_tensor(np.asarray(copies, dtype=np.int32)).to(dev)
        for c in caches:
            _ops.copy_blocks(c, pairs)

    # ── device-resident tables ─────────────────────────────

    def bind_rows(self, rows: int, cols: int) -> None:
        """Starts tracking device rows [rows, cols] (host side only; see bind_device)."""
        check(lib().cf_bp_bind_rows(self._h, int(rows), int(cols)), "bind_rows")

    def bind_device(self, rows: int, cols: int, device: torch.device | str | None = None) -> None:
        """Allocates the device table [rows, cols] (-1) and lengths [rows] (0)."""
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.bind_rows(rows, cols)
        self._table = torch.full((rows, cols), -1, dtype=torch.int32, device=device)
        self._lens = torch.zeros(rows, dtype=torch.int32, device=device)

    def row_of(self, request_id: str) -> int:
        """The request's device row, -1 before its first sync."""
        out = ctypes.c_int32(0)
        check(lib().cf_bp_row_of(self._h, _b(request_id), ctypes.byref(out)), "row_of")
        return int(out.value)

    def table_deltas(self) -> np.ndarray:
        """Cells changed since the last call, int32 [n, 4] = {row, col, value,
        0} (col = -1: the row length); consumes them."""
        buf = self._delta_buf
        n = ctypes.c_int64(0)
        rc = lib().cf_bp_table_deltas(self._h, buf.ctypes.data, buf.shape[0], ctypes.byref(n))
        if rc != 0 and n.value > buf.shape[0]:  # too short: grow and ask again (nothing was consumed)
            buf = self._delta_buf = np.empty((2 * n.value, 4), dtype=np.int32)
            rc = lib().cf_bp_table_deltas(self._h, buf.ctypes.data, buf.shape[0], ctypes.byref(n))
        check(rc, "table_deltas")
        return buf[: n.value].copy()

    def sync_device(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Applies this step's table changes on the device (one host-to-device
        copy of the deltas and one scatter on the current stream); returns
        (tables int32 [rows, cols], lens int32 [rows])."""
        if self._table is None or self._lens is None:
            raise RuntimeError("bind_device first")
        d = self.table_deltas()
        if len(d):
            k = self._stage_k
            self._stage_k ^= 1
            if self._stage_done[k] is not None:
                self._stage_done[k].synchronize()  # its previous copy (two syncs ago) has long run
            buf = self._stage[k]
            if buf is None or buf.shape[0] < len(d):
                buf = self._stage[k] = torch.empty((max(len(d), 1024), 4), dtype=torch.int32, pin_memory=True)
            host = buf[: len(d)]
            host.numpy()[:] = d
            dev = host.to(self._table.device, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self._table.device))
            self._stage_done[k] = ev
            _ops.block_tables_apply(self._table, self._lens, dev)
        return self._table, self._lens

    def shared_prefix_lens_host(self, rows: int) -> np.ndarray:
        """int32 [rows]: leading tokens each device row shares (same physical
        blocks) with the row before, capped by both lengths."""
        out = np.empty(int(rows), dtype=np.int32)
        check(lib().cf_bp_shared_prefix_lens(self._h, out.ctypes.data, out.size), "shared_prefix_lens")
        return out

    def shared_prefix_lens(self) -> torch.Tensor:
        """The decode kernel's shared-prefix statement for the device rows,
        as an int32 [rows] device tensor."""
        if self._table is None:
            raise RuntimeError("bind_device first")
        return torch.from_numpy(self.shared_prefix_lens_host(self._table.shape[0])).to(self._table.device)


class RequestBatch:
    """A fixed list of request ids, encoded once for the native pool (the
    decode batch of a serving loop, reused step after step)."""

    def __init__(self, request_ids: Iterable[str]) -> None:
        self.ids = list(request_ids)
        self._enc = [_b(r) for r in self.ids]
        self.c_ids = (ctypes.c_char_p * max(len(self.ids), 1))(*self._enc)

    def __len__(self) -> int:
        return len(self.ids)


PyBlockManager = BlockManager

__all__ = ["BlockManager", "PyBlockManager", "RequestBatch"]
