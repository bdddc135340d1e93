"""PagedAttention decode over a paged KV cache, on MI355X.

Drop-in for the reference's `kernels/paged_attention.py::paged_attention`
(reference kernels/paged_attention.py:200-227): same arguments, same
dict-in/dict-out contract, same edge rules as its CPU path (:21-73).  The
work runs in libcf_hip.so's HIP kernels; there is no CPU fallback here.

Added, backward-compatible:
  - keyword-only `k_scale`, `v_scale` (fp32, one per KV head or one in
    total), required when the caches hold float8_e4m3fn codes;
  - keyword-only `partition_tokens` (split-KV partition length);
  - `paged_attention_tensors`, the tensor-native entry the dict API wraps
    (int32 block tables [B, Mb], int32 lengths [B], output [B, Hq, D]);
  - `chunked_prefill_attention`, the attention of a chunked-prefill step
    (reference runtime/src/engine/scheduler.rs:178-226): query chunks
    attending causally to their sequence's cached tokens and to themselves.
"""

from __future__ import annotations

import array
import math

import numpy as np

import torch

from cf_hip import ops as _ops

# Staging for the dict API's tables / lengths / shared-prefix statement:
# per (device, stream), _SLOTS slots of {pinned host buffer, device buffer}.
# A call packs into a slot's host buffer, copies it into the slot's device
# buffer on the stream and records an event; the slot is reused _SLOTS
# calls later, after that event (the host buffer is free once its copy ran;
# the device buffer is read by this stream's earlier kernels only, which
# precede the new copy).  No call allocates in steady state, and calls
# issued back to back wait on the GPU only when the host runs _SLOTS calls
# ahead of it.
_SLOTS = 4
_STAGE: dict[tuple[torch.device, int], list] = {}


def _pack_tables_py(block_tables: dict, seq_lens: dict, block_size: int, nb: int, out: np.ndarray,
                    width: int) -> int:
    """pack_tables in numpy (used when the _tablepack extension is not built)."""
    rids = list(block_tables.keys())
    n_req = len(rids)
    used: list[np.ndarray] = []
    nblk = np.empty(n_req, dtype=np.int64)
    lens = np.empty(n_req, dtype=np.int64)
    for i, rid in enumerate(rids):
        blocks = block_tables[rid]
        seq_len = seq_lens.get(rid, len(blocks) * block_size)
        n_blocks = min(len(blocks), (seq_len + block_size - 1) // block_size)
        if n_blocks <= 0:
            raise RuntimeError(f"request {rid!r}: no KV blocks to attend (seq_len={seq_len})")
        used.append(_as_ids(blocks[:n_blocks]))
        nblk[i] = n_blocks
        lens[i] = min(seq_len, n_blocks * block_size)
    mb = int(nblk.max())
    mat = np.zeros((n_req, mb), dtype=np.int64)
    for i, u in enumerate(used):
        mat[i, : u.shape[0]] = u
    live = np.arange(mb)[None, :] < nblk[:, None]
    bad = live & ((mat < -nb) | (mat >= nb))
    if bad.any():
        i, j = np.argwhere(bad)[0]
        raise IndexError(f"request {rids[i]!r}: block id {int(mat[i, j])} out of range for {nb} cache blocks")
    mat = np.where(mat < 0, mat + nb, mat)
    shared = np.zeros(n_req, dtype=np.int64)
    if n_req > 1:
        same = (mat[1:] == mat[:-1]) & live[1:] & live[:-1]
        lead = np.cumprod(same, axis=1).sum(axis=1)
        shared[1:] = np.maximum(0, np.minimum(np.minimum(lead * block_size, lens[:-1]), lens[1:]))
    out[: n_req * mb] = mat.reshape(-1)
    out[n_req * mb: n_req * (mb + 1)] = lens
    out[n_req * (mb + 1): n_req * (mb + 2)] = shared
    return mb


try:  # the CPython packer next to the ctypes binding (built by csrc/build.py)
    from cf_hip._tablepack import pack as _pack_native
    from cf_hip._tablepack import width as _width_native
except ImportError:  # pragma: no cover - exercised when only the HIP library is built
    _pack_native = None
    _width_native = None


def table_width(block_tables: dict) -> int:
    """The longest block table's length."""
    if _width_native is not None:
        return _width_native(block_tables)
    return max((len(t) for t in block_tables.values()), default=0)


def pack_tables(block_tables: dict, seq_lens: dict, block_size: int, nb: int, out: np.ndarray, width: int) -> int:
    """Request dicts -> int32 out[: n * (mb + 2)] = tables [n, mb] | lengths
    [n] | shared-prefix lengths [n] (the reference's rules,
    kernels/paged_attention.py:36-48; negative ids wrapped); returns mb."""
    if _pack_native is not None:
        return _pack_native(block_tables, seq_lens, int(block_size), int(nb), out, int(width))
    return _pack_tables_py(block_tables, seq_lens, block_size, nb, out, width)


def _as_ids(blocks) -> np.ndarray:
    """Block ids as int64 (Python lists unboxed through array.array, the
    fastest route; anything else through numpy)."""
    if isinstance(blocks, list):
        try:
            return np.frombuffer(array.array("q", blocks), dtype=np.int64)
        except (TypeError, OverflowError):
            pass
    if isinstance(blocks, torch.Tensor):
        blocks = blocks.detach().cpu()
    return np.asarray(blocks, dtype=np.int64)


def _staging(device: torch.device, n: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(pinned host buffer, device buffer) of the next slot, each >= n int32."""
    key = (device, _ops.stream_handle(device))
    st = _STAGE.get(key)
    if st is None:
        st = _STAGE[key] = [[None] * _SLOTS, [None] * _SLOTS, [None] * _SLOTS, 0]
    hosts, devs, events, k = st
    if events[k] is not None:
        events[k].synchronize()
    if hosts[k] is None or hosts[k].numel() < n + 4:
        size = max(n + 4, 1 << 16)  # + 4: the upload moves whole 16-byte words
        hosts[k] = torch.empty(size, dtype=torch.int32, pin_memory=True)
        devs[k] = torch.empty(size, dtype=torch.int32, device=device)
    return hosts[k], devs[k]


def _staged(device: torch.device) -> None:
    st = _STAGE[(device, _ops.stream_handle(device))]
    ev = st[2][st[3]]
    if ev is None:
        ev = st[2][st[3]] = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(device))
    st[3] = (st[3] + 1) % _SLOTS

def _upload(host: torch.Tensor, dbuf: torch.Tensor, n: int, device: torch.device) -> None:
    """host[:n] -> dbuf[:n] on the current stream: with the library's
    compute-queue upload (a kernel reading the pinned buffer, ordered with
    the decode kernels without a copy-engine hand-off), or a torch copy where
    the buffer is not mapped pinned memory."""
    nbytes = ((n + 3) // 4) * 16
    if _ops.stage_from_host(host.data_ptr(), dbuf.data_ptr(), nbytes, device):
        return
    dbuf[:n].copy_(host[:n], non_blocking=True)


DEFAULT_PARTITION_TOKENS = _ops.DEFAULT_PARTITION_TOKENS


def _require_rocm(q: torch.Tensor) -> None:
    if not (isinstance(q, torch.Tensor) and q.is_cuda and torch.version.hip is not None):
        where = q.device if isinstance(q, torch.Tensor) else type(q).__name__
        raise ValueError(
            f"paged_attention runs on ROCm device tensors only (got {where}); "
            "move q, k_cache and v_cache to the GPU"
        )


def paged_attention_tensors(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    block_size: int = 16,
    scale: float | None = None,
    *,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    partition_tokens: int = DEFAULT_PARTITION_TOKENS,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    shared_prefix_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode attention for a batch held in tensors.

    Args:
        q: [B, Hq, D] query, one token per sequence.
        k_cache, v_cache: [num_blocks, block_size, Hkv, D] (any strides).
        block_tables: int32 [B, Mb] physical block ids per sequence.
        seq_lens: int32 [B]; sequence b attends to its first
            min(seq_lens[b], Mb*block_size) tokens (0 gives a zero row).
        block_size: tokens per block (must equal k_cache.shape[1]).
        scale: softmax scale, default 1/sqrt(D).
        k_scale, v_scale: dequant scales for float8_e4m3fn caches.
        shared_prefix_lens: optional int32 [B]; entry b = leading tokens of
            sequence b held in the same physical blocks as sequence b - 1's
            (cf_hip.ops.shared_prefix_lens computes it from host tables).
            Shared blocks are then read once per group of sharers; the
            result is unchanged (up to summation order).  Trusted as given.

    Returns:
        [B, Hq, D] tensor in q's dtype.
    """
    _require_rocm(q)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if block_tables.dtype != torch.int32:
        block_tables = block_tables.to(torch.int32)
    if seq_lens.dtype != torch.int32:
        seq_lens = seq_lens.to(torch.int32)
    return _ops.paged_decode(
        q, k_cache, v_cache, block_tables, seq_lens, float(scale), int(block_size),
        k_scale=k_scale, v_scale=v_scale, partition_tokens=partition_tokens, out=out, workspace=workspace,
        shared_prefix_lens=shared_prefix_lens,
    )


def paged_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: dict[str, list[int]],
    seq_lens: dict[str, int],
    block_size: int = 16,
    scale: float | None = None,
    *,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    partition_tokens: int = DEFAULT_PARTITION_TOKENS,
) -> dict[str, torch.Tensor]:
    """PagedAttention with block table indirection.

    Args:
        q:  Query tensor [batch, num_heads, head_dim] (decode: one token per request).
        k_cache: Paged K cache [num_blocks, block_size, num_kv_heads, head_dim].
        v_cache: Paged V cache [num_blocks, block_size, num_kv_heads, head_dim].
        block_tables: request_id -> list[physical block IDs].
        seq_lens: request_id -> current sequence length.
        block_size: Tokens per KV block (default 16).
        scale: Attention scale (default 1/sqrt(head_dim)).
        k_scale, v_scale: FP8 dequant scales (float8_e4m3fn caches only).

    Returns:
        dict mapping request_id -> output tensor [num_heads, head_dim].

    Request i of the dict (insertion order) uses q[i]; a request missing
    from seq_lens attends to len(blocks) * block_size tokens; a length past
    the table's capacity is cut to it (reference
    kernels/paged_attention.py:36-48).
    """
    _require_rocm(q)
    rids = list(block_tables.keys())
    if len(rids) > q.shape[0]:
        raise IndexError(f"{len(rids)} requests but q holds {q.shape[0]} rows")
    if not rids:
        return {}
    nb = k_cache.shape[0]
    n_req = len(rids)
    width = table_width(block_tables)
    host, dbuf = _staging(q.device, n_req * (width + 2))
    mb = pack_tables(block_tables, seq_lens, block_size, nb, host.numpy(), width)
    used = n_req * (mb + 2)
    dev = dbuf[:used]
    _upload(host, dbuf, used, q.device)
    _staged(q.device)
    dev_tables = dev[: n_req * mb].view(n_req, mb)
    dev_lens = dev[n_req * mb: n_req * (mb + 1)]
    dev_shared = dev[n_req * (mb + 1):]
    out = paged_attention_tensors(
        q[:n_req], k_cache, v_cache, dev_tables, dev_lens, block_size, scale,
        k_scale=k_scale, v_scale=v_scale, partition_tokens=partition_tokens, shared_prefix_lens=dev_shared,
    )
    return dict(zip(rids, out.unbind(0)))


def chunked_prefill_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    q_start: torch.Tensor,
    block_size: int = 16,
    scale: float | None = None,
    *,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Attention of prefill chunks over the paged cache.

    Args:
        q: [Tq, Hq, D] bf16 or float16, the query rows of all chunks.
        k_cache, v_cache: [num_blocks, 16, Hkv, D] in any layout of
            cf_hip.layout.alloc_kv_cache (the reference's token-major one
            included): bfloat16 or float8_e4m3fn under bf16 queries,
            float16 or float8_e4m3fn under float16 queries; the chunk's own
            K/V must already be written.
        block_tables: int32 [N, Mb], one row per chunk's sequence.
        seq_lens: int32 [N], tokens of each sequence including its chunk.
        q_start: int32 [N + 1]; chunk n owns q rows [q_start[n], q_start[n+1]).
        scale: softmax scale, default 1/sqrt(D).

    Row i of a chunk of L rows is the token at position seq_lens[n] - L + i
    and attends to positions [0, seq_lens[n] - L + i] (bottom-right causal;
    with nothing cached this is causal self-attention of the chunk, as the
    reference's flash_attention_fwd(is_causal=True),
    kernels/flash_attention.py:179-202).

    Returns:
        [Tq, Hq, D] in q's dtype.
    """
    _require_rocm(q)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    block_tables, seq_lens, q_start = (t if t.dtype == torch.int32 else t.to(torch.int32)
                                       for t in (block_tables, seq_lens, q_start))
    return _ops.prefill_chunk(
        q, k_cache, v_cache, block_tables, seq_lens, q_start, float(scale), int(block_size),
        k_scale=k_scale, v_scale=v_scale, out=out, workspace=workspace,
    )


__all__ = ["DEFAULT_PARTITION_TOKENS", "chunked_prefill_attention", "paged_attention", "paged_attention_tensors"]
