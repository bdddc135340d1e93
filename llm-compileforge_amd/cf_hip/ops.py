"""Tensor-level wrappers over the cf_hip C ABI.

Every function here takes ROCm device tensors, enqueues HIP kernels on the
current torch stream and returns without synchronizing.  There is no CPU
path: a CPU tensor or a missing libcf_hip.so raises.
"""

from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _abi
from ._abi import check, descriptor, lib, ref, stream_handle

DEFAULT_PARTITION_TOKENS = 512


def _require_device(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if not t.is_cuda or torch.version.hip is None:
        raise ValueError(f"{name} must be a ROCm device tensor (got device {t.device})")


_SAME = contextlib.nullcontext()


def _on(device: torch.device):
    """Makes `device` current for a library call (a no-op when it is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _SAME
    return torch.cuda.device(device)


def _same_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"all tensors must be on {dev}, found one on {t.device}")
    return dev


def decode_workspace_bytes(
    batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_blocks_per_seq: int, block_size: int,
    partition_tokens: int = DEFAULT_PARTITION_TOKENS,
) -> int:
    out = ctypes.c_uint64(0)
    rc = lib().cf_paged_decode_workspace_bytes(
        batch, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size, partition_tokens,
        ctypes.byref(out),
    )
    check(rc, "cf_paged_decode_workspace_bytes")
    return int(out.value)


def new_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A decode workspace of at least `nbytes` bytes (256-byte aligned)."""
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


# One workspace per (device, stream) for callers that pass none: calls on
# one stream run in order, so they may share it.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _cached_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream_handle(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = new_workspace(nbytes, device)
        _WORKSPACES[key] = ws
    return ws


def shared_prefix_lens(block_tables: list[list[int]], seq_lens: list[int], block_size: int) -> list[int]:
    """Tokens each sequence shares with the previous one (host-side).

    Entry b is the number of leading tokens of sequence b stored in the
    same physical blocks, at the same table positions, as those of
    sequence b - 1: the longest common prefix of the two block tables, in
    tokens, cut to both sequences' lengths (entry 0 is 0).  Consecutive
    sequences that a radix-tree prefix cache placed on shared blocks
    (reference runtime/src/cache/radix.rs:50-177, block.rs:273-306) get
    their shared length; this is the `shared_prefix_lens` statement
    `paged_decode` takes.
    """
    out = [0] * len(block_tables)
    for b in range(1, len(block_tables)):
        prev, cur = block_tables[b - 1], block_tables[b]
        n, lim = 0, min(len(prev), len(cur))
        while n < lim and int(prev[n]) == int(cur[n]):
            n += 1
        out[b] = max(0, min(n * block_size, int(seq_lens[b - 1]), int(seq_lens[b])))
    return out


def paged_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float,
    block_size: int,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    partition_tokens: int = DEFAULT_PARTITION_TOKENS,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    shared_prefix_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """Paged decode attention on the GPU; returns out [B, Hq, D] (dtype of q).

    workspace: optional buffer of decode_workspace_bytes() bytes; by default
    a cached one per (device, stream) is used.

    shared_prefix_lens: optional int32 [B] device tensor, entry b = leading
    tokens sequence b shares (same physical blocks) with sequence b - 1
    (see `shared_prefix_lens()`); shared tiles are then read once per
    group of sharing sequences.  The statement is trusted.

    block_tables: int32 [B, Mb]; seq_lens: int32 [B]; caches [NB, bs, Hkv, D]
    with any strides (f32/f16/bf16/e4m3fn); e4m3fn caches need per-KV-head
    fp32 k_scale/v_scale of shape [Hkv] or [1].
    """
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                    ("seq_lens", seq_lens)):
        _require_device(name, t)
    dev = _same_device(q, k_cache, v_cache, block_tables, seq_lens)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    need = decode_workspace_bytes(
        q.shape[0], q.shape[1], k_cache.shape[2], q.shape[2], block_tables.shape[1], block_size, partition_tokens
    )
    ws_ptr = None
    if need > 0:
        if workspace is None:
            workspace = _cached_workspace(need, dev)
        elif workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace of {need} bytes needed, {workspace.numel() * workspace.element_size()} given")
        ws_ptr = workspace.data_ptr()
    ks = descriptor(k_scale) if k_scale is not None else None
    vs = descriptor(v_scale) if v_scale is not None else None
    dsh = None
    if shared_prefix_lens is not None:
        _require_device("shared_prefix_lens", shared_prefix_lens)
        _same_device(q, shared_prefix_lens)
        dsh = descriptor(shared_prefix_lens)
    dq, dk, dv = descriptor(q), descriptor(k_cache), descriptor(v_cache)
    dt, dsl, do = descriptor(block_tables), descriptor(seq_lens), descriptor(out)
    with _on(dev):
        rc = lib().cf_paged_decode_shared(
            ref(dq), ref(dk), ref(dv), ref(dt), ref(dsl), ref(dsh), ref(ks), ref(vs),
            float(scale), int(block_size), int(partition_tokens), ref(do),
            ws_ptr, need, stream_handle(dev),
        )
    check(rc, "cf_paged_decode_shared")
    return out


NOALLOC_SCRATCH_BYTES = 64 << 20  # the library's fixed per-device scratch (cf_paged_decode_shared_noalloc)


def paged_decode_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float,
    block_size: int,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    partition_tokens: int = DEFAULT_PARTITION_TOKENS,
    out: torch.Tensor | None = None,
    shared_prefix_lens: torch.Tensor | None = None,
) -> torch.Tensor:
    """paged_decode for callers that cannot allocate: the library's fixed
    per-device scratch replaces the workspace, so the call itself allocates
    nothing (pass `out` to keep torch from allocating the output).  Calls
    that overlap on one device race on that scratch; a call needing more
    than NOALLOC_SCRATCH_BYTES raises ValueError."""
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                    ("seq_lens", seq_lens)):
        _require_device(name, t)
    dev = _same_device(q, k_cache, v_cache, block_tables, seq_lens)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    ks = descriptor(k_scale) if k_scale is not None else None
    vs = descriptor(v_scale) if v_scale is not None else None
    dsh = None
    if shared_prefix_lens is not None:
        _require_device("shared_prefix_lens", shared_prefix_lens)
        _same_device(q, shared_prefix_lens)
        dsh = descriptor(shared_prefix_lens)
    dq, dk, dv = descriptor(q), descriptor(k_cache), descriptor(v_cache)
    dt, dsl, do = descriptor(block_tables), descriptor(seq_lens), descriptor(out)
    with _on(dev):
        rc = lib().cf_paged_decode_shared_noalloc(
            ref(dq), ref(dk), ref(dv), ref(dt), ref(dsl), ref(dsh), ref(ks), ref(vs),
            float(scale), int(block_size), int(partition_tokens), ref(do), stream_handle(dev),
        )
    check(rc, "cf_paged_decode_shared_noalloc")
    return out


def prefill_workspace_bytes(num_q_tokens: int, num_chunks: int, num_q_heads: int, num_kv_heads: int,
                            head_dim: int, block_size: int = 16) -> int:
    out = ctypes.c_uint64(0)
    rc = lib().cf_prefill_chunk_workspace_bytes(
        num_q_tokens, num_chunks, num_q_heads, num_kv_heads, head_dim, block_size, ctypes.byref(out)
    )
    check(rc, "cf_prefill_chunk_workspace_bytes")
    return int(out.value)


def prefill_chunk(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    q_start: torch.Tensor,
    scale: float,
    block_size: int = 16,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Chunked-prefill attention over the paged cache; returns out [Tq, Hq, D].

    q [Tq, Hq, D] bf16 or fp16 holds the rows of N chunks, chunk n owning
    rows [q_start[n], q_start[n+1]); block_tables int32 [N, Mb]; seq_lens
    int32 [N] counts the sequence's tokens including the chunk (already
    written to the cache).  Row i of a chunk of L rows attends causally to
    cache positions [0, seq_lens[n] - L + i].  Caches: bf16 or e4m3fn under
    bf16 q, fp16 or e4m3fn under fp16 q, block_size 16, in the native or
    paired tile layout or the reference's token-major rows ([NB, 16, Hkv,
    D] contiguous).
    """
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                    ("seq_lens", seq_lens), ("q_start", q_start)):
        _require_device(name, t)
    dev = _same_device(q, k_cache, v_cache, block_tables, seq_lens, q_start)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=dev)
    need = prefill_workspace_bytes(q.shape[0], block_tables.shape[0], q.shape[1], k_cache.shape[2], q.shape[2],
                                   block_size)
    if workspace is None:
        workspace = _cached_workspace(need, dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace of {need} bytes needed, {workspace.numel() * workspace.element_size()} given")
    ks = descriptor(k_scale) if k_scale is not None else None
    vs = descriptor(v_scale) if v_scale is not None else None
    d = [descriptor(t) for t in (q, k_cache, v_cache, block_tables, seq_lens, q_start)]
    do = descriptor(out)
    with _on(dev):
        rc = lib().cf_prefill_chunk_fp8(
            *(ref(x) for x in d), ref(ks), ref(vs), float(scale), int(block_size), ref(do),
            workspace.data_ptr(), need, stream_handle(dev),
        )
    check(rc, "cf_prefill_chunk_fp8")
    return out


class DecodePlan:
    """A paged decode call with its descriptors built once.

    For a serving loop that reruns decode over the same buffers (updated in
    place: q, tables, lengths, cache contents), `run()` costs one C call.
    The plan keeps references to every tensor it describes.
    """

    def __init__(
        self,
        q: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        block_tables: torch.Tensor,
        seq_lens: torch.Tensor,
        scale: float,
        block_size: int,
        k_scale: torch.Tensor | None = None,
        v_scale: torch.Tensor | None = None,
        partition_tokens: int = DEFAULT_PARTITION_TOKENS,
        out: torch.Tensor | None = None,
        shared_prefix_lens: torch.Tensor | None = None,
    ) -> None:
        for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_tables", block_tables),
                        ("seq_lens", seq_lens)):
            _require_device(name, t)
        self.device = _same_device(q, k_cache, v_cache, block_tables, seq_lens)
        if shared_prefix_lens is not None:
            _require_device("shared_prefix_lens", shared_prefix_lens)
            _same_device(q, shared_prefix_lens)
        self.out = out if out is not None else torch.empty(q.shape, dtype=q.dtype, device=self.device)
        self.ws_bytes = decode_workspace_bytes(
            q.shape[0], q.shape[1], k_cache.shape[2], q.shape[2], block_tables.shape[1], block_size,
            partition_tokens,
        )
        self.workspace = new_workspace(self.ws_bytes, self.device)
        self._keep = (q, k_cache, v_cache, block_tables, seq_lens, k_scale, v_scale, shared_prefix_lens)
        self._d = [descriptor(t) for t in (q, k_cache, v_cache, block_tables, seq_lens)]
        self._dsh = descriptor(shared_prefix_lens) if shared_prefix_lens is not None else None
        self._ks = descriptor(k_scale) if k_scale is not None else None
        self._vs = descriptor(v_scale) if v_scale is not None else None
        self._do = descriptor(self.out)
        self._args = (
            *(ref(d) for d in self._d), ref(self._dsh), ref(self._ks), ref(self._vs), float(scale),
            int(block_size), int(partition_tokens), ref(self._do),
            self.workspace.data_ptr() if self.ws_bytes else None, self.ws_bytes,
        )
        self._fn = lib().cf_paged_decode_shared

    def run(self, stream: int | None = None) -> torch.Tensor:
        rc = self._fn(*self._args, stream if stream is not None else stream_handle(self.device))
        check(rc, "cf_paged_decode_shared")
        return self.out


def _as3(x: torch.Tensor) -> torch.Tensor:
    """Presents x to the C ABI as [T, H, D] or [S0, S1, H, D]: the
    second-to-last axis is the head axis (the one scales index)."""
    if x.dim() in (3, 4):
        return x
    if x.dim() == 2:
        return x.unsqueeze(1)
    if x.dim() < 2:
        return x.reshape(1, 1, -1)
    return x.reshape(-1, x.shape[-3], x.shape[-2], x.shape[-1])


def fp8_amax_scale(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-head scales [H] = amax(|x[..., h, :]|)/448 (1.0 for all-zero heads, >= 1e-12)."""
    _require_device("x", x)
    x3 = _as3(x)
    if out is None:
        out = torch.empty(x3.shape[-2], dtype=torch.float32, device=x.device)
    dx, do = descriptor(x3), descriptor(out)
    with torch.cuda.device(x.device):
        rc = lib().cf_fp8_amax_scale(ref(dx), ref(do), stream_handle(x.device))
    check(rc, "cf_fp8_amax_scale")
    return out


def fp8_quantize(x: torch.Tensor, scales: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """e4m3fn(x / scales[h]); scales has one entry per head (axis -2) or one in total."""
    _require_device("x", x)
    _require_device("scales", scales)
    x3 = _as3(x)
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    o3 = _as3(out)
    dx, dsc, do = descriptor(x3), descriptor(scales.reshape(-1)), descriptor(o3)
    with torch.cuda.device(x.device):
        rc = lib().cf_fp8_quantize(ref(dx), ref(dsc), ref(do), stream_handle(x.device))
    check(rc, "cf_fp8_quantize")
    return out


def fp8_quantize_kv(k: torch.Tensor, v: torch.Tensor, k_scales: torch.Tensor, v_scales: torch.Tensor,
                    k_out: torch.Tensor | None = None, v_out: torch.Tensor | None = None
                    ) -> tuple[torch.Tensor, torch.Tensor]:
    """(e4m3fn(k / k_scales[h]), e4m3fn(v / v_scales[h])), the codes of two
    fp8_quantize calls; one launch when k_out / v_out are a cache's native or
    paired K / V views of [S0, 16, H, D] pools."""
    for name, t in (("k", k), ("v", v), ("k_scales", k_scales), ("v_scales", v_scales)):
        _require_device(name, t)
    if k_out is None:
        k_out = torch.empty(k.shape, dtype=torch.float8_e4m3fn, device=k.device)
    if v_out is None:
        v_out = torch.empty(v.shape, dtype=torch.float8_e4m3fn, device=v.device)
    dk, dv = descriptor(_as3(k)), descriptor(_as3(v))
    dks, dvs = descriptor(k_scales.reshape(-1)), descriptor(v_scales.reshape(-1))
    dko, dvo = descriptor(_as3(k_out)), descriptor(_as3(v_out))
    with torch.cuda.device(k.device):
        rc = lib().cf_fp8_quantize_kv(ref(dk), ref(dv), ref(dks), ref(dvs), ref(dko), ref(dvo),
                                      stream_handle(k.device))
    check(rc, "cf_fp8_quantize_kv")
    return k_out, v_out


def fp8_dequantize(q: torch.Tensor, scales: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """f32(q) * scales[h]."""
    _require_device("q", q)
    _require_device("scales", scales)
    q3 = _as3(q)
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    o3 = _as3(out)
    dq, dsc, do = descriptor(q3), descriptor(scales.reshape(-1)), descriptor(o3)
    with torch.cuda.device(q.device):
        rc = lib().cf_fp8_dequantize(ref(dq), ref(dsc), ref(do), stream_handle(q.device))
    check(rc, "cf_fp8_dequantize")
    return out


def kv_write_fp8(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
) -> None:
    """Quantizes new K/V rows [T, Hkv, D] into paged e4m3fn caches at
    slot_mapping[T].  Slots must be distinct (rows repeating a slot race);
    slots outside the cache are skipped."""
    for name, t in (("k_new", k_new), ("v_new", v_new), ("slot_mapping", slot_mapping), ("k_cache", k_cache),
                    ("v_cache", v_cache), ("k_scale", k_scale), ("v_scale", v_scale)):
        _require_device(name, t)
    dev = _same_device(k_new, v_new, slot_mapping, k_cache, v_cache, k_scale, v_scale)
    ds = [descriptor(t) for t in (k_new, v_new, slot_mapping, k_cache, v_cache, k_scale.reshape(-1),
                                   v_scale.reshape(-1))]
    with _on(dev):
        rc = lib().cf_kv_write_fp8(*(ref(d) for d in ds), stream_handle(dev))
    check(rc, "cf_kv_write_fp8")


def paged_write(
    x_new: torch.Tensor, slot_mapping: torch.Tensor, cache: torch.Tensor, scale: torch.Tensor | None = None
) -> None:
    """Writes rows x_new [T, H, D] into a paged cache [NB, bs, H, D] (any
    layout) at slots block * bs + offset; e4m3fn caches quantize with the
    per-head `scale` [H] (or one scale).  Slots outside the cache are
    skipped; slots must be distinct (rows repeating a slot race)."""
    for name, t in (("x_new", x_new), ("slot_mapping", slot_mapping), ("cache", cache)):
        _require_device(name, t)
    dev = _same_device(x_new, slot_mapping, cache)
    ds = [descriptor(t) for t in (x_new, slot_mapping, cache)]
    dsc = None
    if scale is not None:
        _require_device("scale", scale)
        dsc = descriptor(scale.reshape(-1))
    with _on(dev):
        rc = lib().cf_paged_write(ref(ds[0]), ref(ds[1]), ref(ds[2]), ref(dsc), stream_handle(dev))
    check(rc, "cf_paged_write")


def paged_gather(
    cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_len: int,
    out_dtype: torch.dtype | None = None,
    scale: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Dense [R, seq_len, H, D] rows of the tables' first seq_len tokens
    (e4m3fn caches dequantized with `scale`, returned as float32 unless
    out_dtype says otherwise); table entries < 0 give zero rows."""
    _require_device("cache", cache)
    _require_device("block_tables", block_tables)
    dev = _same_device(cache, block_tables)
    if out is None:
        dt = out_dtype or (torch.float32 if cache.dtype == torch.float8_e4m3fn else cache.dtype)
        out = torch.empty(block_tables.shape[0], seq_len, cache.shape[2], cache.shape[3], dtype=dt, device=dev)
    dsc = None
    if scale is not None:
        _require_device("scale", scale)
        dsc = descriptor(scale.reshape(-1))
    dc, dt_, do = descriptor(cache), descriptor(block_tables), descriptor(out)
    with _on(dev):
        rc = lib().cf_paged_gather(ref(dc), ref(dt_), ref(dsc), ref(do), stream_handle(dev))
    check(rc, "cf_paged_gather")
    return out


def stage_from_host(host_ptr: int, dev_ptr: int, nbytes: int, device: torch.device) -> bool:
    """Uploads nbytes (a multiple of 16) from mapped pinned host memory to
    device memory with the library's upload kernel on the current stream;
    False (nothing enqueued) when the host buffer is not mapped pinned
    memory."""
    with _on(device):
        rc = lib().cf_stage_from_host(host_ptr, dev_ptr, nbytes, stream_handle(device))
    if rc == _abi.CF_ERR_INVALID:
        return False
    check(rc, "cf_stage_from_host")
    return True


def block_tables_apply(table: torch.Tensor, lens: torch.Tensor, deltas: torch.Tensor) -> None:
    """Scatters block-table deltas [n, 4] int32 = {row, col, value, 0} into a
    device table [rows, cols] int32 (col = -1: lens[row] = value)."""
    for name, t in (("table", table), ("lens", lens), ("deltas", deltas)):
        _require_device(name, t)
    dev = _same_device(table, lens, deltas)
    dt, dl, dd = descriptor(table), descriptor(lens), descriptor(deltas)
    with _on(dev):
        rc = lib().cf_block_tables_apply(ref(dt), ref(dl), ref(dd), stream_handle(dev))
    check(rc, "cf_block_tables_apply")


def block_span_view(cache: torch.Tensor) -> torch.Tensor:
    """[NB, E] view of a paged tensor whose dim 0 is the block: raises unless
    each block's elements fill one contiguous span."""
    if cache.dim() < 1:
        raise ValueError("cache must have a block dimension")
    nb = cache.shape[0]
    inner = [(n, st) for n, st in zip(cache.shape[1:], cache.stride()[1:]) if n > 1]
    span = 1 + sum((n - 1) * st for n, st in inner)
    elems = 1
    for n, _ in inner:
        elems *= n
    if span != elems or (nb > 1 and cache.stride(0) < elems):
        raise ValueError("cache blocks are not dense contiguous spans")
    return torch.as_strided(cache, (nb, elems), (cache.stride(0) if nb > 1 else elems, 1), cache.storage_offset())


def copy_blocks(cache: torch.Tensor, pairs: torch.Tensor) -> None:
    """Copies whole blocks of a paged tensor (dim 0 = block): block
    pairs[i, 1] <- block pairs[i, 0] (pairs int32 [n, 2] on the device)."""
    _require_device("cache", cache)
    _require_device("pairs", pairs)
    dev = _same_device(cache, pairs)
    flat = block_span_view(cache).view(torch.uint8)  # bytes: any element type
    dc, dp = descriptor(flat), descriptor(pairs)
    with _on(dev):
        rc = lib().cf_copy_blocks(ref(dc), ref(dp), stream_handle(dev))
    check(rc, "cf_copy_blocks")


# ---- side-by-side work on one device ------------------------------------------
# Decode attention is bound by HBM and chunked prefill by the MFMA pipes.  The
# decode kernel keeps one workgroup per CU (166 VGPRs a wave), which leaves
# register room for one prefill workgroup (250 VGPRs a wave) beside it on
# every CU, so the two kernels overlap when they sit on two streams.
_SIDE: dict[int, tuple[torch.cuda.Stream, torch.cuda.Event, torch.cuda.Event]] = {}


def _side_stream(device: torch.device) -> tuple[torch.cuda.Stream, torch.cuda.Event, torch.cuda.Event]:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    entry = _SIDE.get(idx)
    if entry is None:
        # default priority, like every stream of this library
        entry = (torch.cuda.Stream(device=torch.device("cuda", idx)), torch.cuda.Event(), torch.cuda.Event())
        _SIDE[idx] = entry
    return entry


def run_concurrent(main, side, device: torch.device, keep: tuple[torch.Tensor, ...] = ()) -> None:
    """Runs `main()` on the current stream and `side()` on a side stream of
    `device`, so their kernels can execute at the same time.

    Ordering: `side` starts after the work already queued on the current
    stream; work queued on the current stream after this call starts after
    both.  `keep` lists the tensors `side` uses that the caller may free
    afterwards (the caching allocator then waits for the side stream before
    reusing their memory).  Both callables enqueue work only: no host
    synchronization happens here.
    """
    cur = torch.cuda.current_stream(device)
    stream, forked, joined = _side_stream(device)
    forked.record(cur)
    stream.wait_event(forked)
    try:
        main()
        with torch.cuda.stream(stream):
            side()
        for t in keep:
            t.record_stream(stream)
    finally:
        # also when a callable raised: whatever reached the side stream is
        # ordered before the caller's later work
        joined.record(stream)
        cur.wait_event(joined)


class KernelTimer:
    """Sums device time of this library's kernel launches (HIP events)."""

    def __enter__(self) -> "KernelTimer":
        lib().cf_profile_reset()
        lib().cf_profile_enable(1)
        return self

    def __exit__(self, *exc: object) -> None:
        lib().cf_profile_enable(0)

    @staticmethod
    def query(prefix: str) -> tuple[float, int]:
        ms = ctypes.c_double(0.0)
        n = ctypes.c_int64(0)
        check(lib().cf_profile_query(prefix.encode(), ctypes.byref(ms), ctypes.byref(n)), "cf_profile_query")
        return float(ms.value), int(n.value)

    @staticmethod
    def durations(prefix: str) -> list[float]:
        """Per-launch durations (ms, launch order) of kernels named `prefix`*."""
        n = ctypes.c_int64(0)
        check(lib().cf_profile_durations(prefix.encode(), None, 0, ctypes.byref(n)), "cf_profile_durations")
        buf = (ctypes.c_float * max(n.value, 1))()
        check(lib().cf_profile_durations(prefix.encode(), buf, n.value, ctypes.byref(n)), "cf_profile_durations")
        return [float(buf[i]) for i in range(n.value)]

    @staticmethod
    def reserve(events: int) -> None:
        """Creates timing events ahead of a measured pass (two per launch)."""
        check(lib().cf_profile_reserve(int(events)), "cf_profile_reserve")

    @staticmethod
    def reset() -> None:
        lib().cf_profile_reset()


__all__ = [
    "DEFAULT_PARTITION_TOKENS",
    "NOALLOC_SCRATCH_BYTES",
    "DecodePlan",
    "KernelTimer",
    "block_span_view",
    "block_tables_apply",
    "copy_blocks",
    "decode_workspace_bytes",
    "prefill_chunk",
    "prefill_workspace_bytes",
    "new_workspace",
    "run_concurrent",
    "fp8_amax_scale",
    "fp8_dequantize",
    "fp8_quantize",
    "fp8_quantize_kv",
    "kv_write_fp8",
    "paged_decode",
    "paged_decode_noalloc",
    "paged_gather",
    "paged_write",
    "shared_prefix_lens",
    "stage_from_host",
    "_abi",
]
