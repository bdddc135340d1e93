"""CPU restatement of the reference's paged-cache I/O semantics (test oracle).

Test infrastructure only: imported by tests/, never by the product.

Restates, in numpy:
  - the write placement of CacheManager.write_paged
    (reference python_runtime/engine/cache_manager.py:139-171) and
    _KVCacheMixin._write_kv_flat (python_runtime/engine/_kv_cache.py:68-104):
    token position p goes to block p // bs, offset p % bs of the FIRST
    request (in the tables' iteration order) whose table covers that block;
    a position no table covers is skipped; the physical id indexes the slab
    like torch indexing (negative ids count from the end); rows are written
    in order, so of two rows bound for one slot the later one stays;
    (a negative position indexes the table from its end, as Python list
    indexing does in the reference loop; the product rejects those);
  - the gather of CacheManager.read_paged (:173-197) and _gather_kv_flat
    (_kv_cache.py:106-132): requests in sorted(request id) order, each
    request's blocks in table order up to max_seq_len, zeros past its table;
  - FP8 slabs (an addition of this build: the reference slabs are
    f32/bf16): codes e4m3fn(x / scale[h]) and values code * scale[h].
"""

from __future__ import annotations

import numpy as np

from oracle import fp8 as ofp8


def write_slots(block_tables: dict[str, list[int]], positions: list[int], block_size: int,
                num_blocks: int) -> list[int]:
    """Slot (phys * bs + offset) of each position; -1 where no table covers it."""
    slots = []
    for pos in positions:
        block_idx, offset = pos // block_size, pos % block_size
        slot = -1
        for blocks in block_tables.values():
            if block_idx < len(blocks):
                phys = int(blocks[block_idx])
                if not -num_blocks <= phys < num_blocks:
                    raise IndexError(f"block id {phys} out of range for {num_blocks} blocks")
                slot = (phys % num_blocks) * block_size + offset
                break
        slots.append(slot)
    return slots


def write_paged(slab: np.ndarray, layer: int, data: np.ndarray, positions: list[int],
                block_tables: dict[str, list[int]], scale: np.ndarray | None = None) -> None:
    """slab [NB, L, bs, H, D] (float values, or uint8 e4m3 codes when `scale`
    is given); data [T, H, D]."""
    nb, _, bs = slab.shape[:3]
    for i, slot in enumerate(write_slots(block_tables, positions, bs, nb)):
        if slot < 0:
            continue
        row = np.asarray(data[i])
        if scale is not None:
            row = ofp8.encode(row.astype(np.float32) / np.asarray(scale, np.float32).reshape(-1, 1))
        slab[slot // bs, layer, slot % bs] = row


def read_paged(slab: np.ndarray, layer: int, max_seq_len: int, block_tables: dict[str, list[int]],
               scale: np.ndarray | None = None) -> np.ndarray:
    """Dense [R, max_seq_len, H, D] rows as float64 (e4m3 codes decoded
    and scaled in float32 when `scale` is given)."""
    if not block_tables:
        raise RuntimeError("Paged slab read requested without active block tables")
    nb, _, bs, h, d = slab.shape
    out = np.zeros((len(block_tables), max_seq_len, h, d), dtype=np.float64)
    for r, (_, blocks) in enumerate(sorted(block_tables.items())):
        for j, phys in enumerate(blocks):
            start = j * bs
            if start >= max_seq_len:
                break
            end = min(start + bs, max_seq_len)
            rows = slab[int(phys) % nb, layer, : end - start]
            if scale is not None:
                # float32 product, as FP8KVCacheQuantizer.dequantize (fp8_kv_cache.py:101-105)
                rows = ofp8.decode(rows).astype(np.float32) * np.asarray(scale, np.float32).reshape(1, -1, 1)
            out[r, start:end] = rows
    return out
