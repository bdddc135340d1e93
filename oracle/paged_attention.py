"""CPU oracle for paged decode attention.  TEST INFRASTRUCTURE ONLY.

paged_attention_cpu restates the reference's _paged_attention_cpu
(kernels/paged_attention.py:21-73) step by step with torch CPU ops:
  - requests in dict insertion order; request idx uses q[idx] (:36, :54);
  - seq_len = seq_lens.get(rid, len(blocks) * block_size) (:37);
  - n_blocks = min(len(blocks), ceil(seq_len / block_size)) (:38);
  - gather k_cache[bid] / v_cache[bid] in table order, cat, slice
    [:seq_len] (:42-48);
  - GQA: repeat_interleave(Hq // Hkv) over the head axis (:57-60);
  - F.scaled_dot_product_attention, non-causal, scale default 1/sqrt(D)
    (:31-32, :62-70).
For float8_e4m3fn caches the gathered blocks are first dequantized as the
reference's FP8KVCacheQuantizer.dequantize_block does (f32(code) * scale,
compiler/quantize/fp8_kv_cache.py:105) with per-KV-head scales.

paged_attention_fp64 is an independent float64 brute force of the same
semantics with numpy, used to pin the restatement.

Chunked prefill (no reference function attends a chunk to a cached
prefix): a chunk of L rows appended to a sequence that then holds S
tokens puts row i at position S - L + i, attending to [0, S - L + i].
chunk_rows() states the chunk bookkeeping (chunks taken in order, made
disjoint); paged_prefill_fp64 is the float64 brute force;
paged_prefill_by_decode reduces every row to the reference's decode
(paged_attention_cpu with seq_len = position + 1), and with nothing
cached the chunk is causal self-attention (the reference's
_flash_attention_fwd_cpu, kernels/flash_attention.py:28-46).
"""

from __future__ import annotations

import math

import numpy as np
import torch


def _dequant_heads(x: torch.Tensor, scales: torch.Tensor | None) -> torch.Tensor:
    """x [..., Hkv, D] e4m3fn -> float32 with per-head scales."""
    xf = x.float()
    if scales is None:
        return xf
    s = scales.float().reshape(-1)
    if s.numel() == 1:
        return xf * s[0]
    return xf * s.view(*([1] * (x.dim() - 2)), -1, 1)


def paged_attention_cpu(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: dict[str, list[int]],
    seq_lens: dict[str, int],
    block_size: int = 16,
    scale: float | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> dict[str, torch.Tensor]:
    import torch.nn.functional as F  # noqa: N812

    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    fp8 = k_cache.dtype == torch.float8_e4m3fn
    outputs: dict[str, torch.Tensor] = {}
    for idx, (rid, blocks) in enumerate(block_tables.items()):
        seq_len = seq_lens.get(rid, len(blocks) * block_size)
        n_blocks = min(len(blocks), (seq_len + block_size - 1) // block_size)
        k_parts = [k_cache[blocks[j]] for j in range(n_blocks)]
        v_parts = [v_cache[blocks[j]] for j in range(n_blocks)]
        k_seq = torch.cat(k_parts, dim=0)[:seq_len]
        v_seq = torch.cat(v_parts, dim=0)[:seq_len]
        if fp8:
            k_seq = _dequant_heads(k_seq, k_scale)
            v_seq = _dequant_heads(v_seq, v_scale)
        k_seq = k_seq.unsqueeze(0).transpose(1, 2)
        v_seq = v_seq.unsqueeze(0).transpose(1, 2)
        q_i = q[idx].unsqueeze(0).unsqueeze(2)
        if fp8:
            q_i = q_i.float()
        if q_i.shape[1] != k_seq.shape[1]:
            ratio = q_i.shape[1] // k_seq.shape[1]
            k_seq = k_seq.repeat_interleave(ratio, dim=1)
            v_seq = v_seq.repeat_interleave(ratio, dim=1)
        out = F.scaled_dot_product_attention(q_i, k_seq, v_seq, attn_mask=None, dropout_p=0.0,
                                             is_causal=False, scale=scale)
        outputs[rid] = out.squeeze(0).squeeze(1)
    return outputs


def paged_attention_fp64(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    block_tables: list[list[int]],
    seq_lens: list[int],
    block_size: int,
    scale: float,
    k_scale: np.ndarray | None = None,
    v_scale: np.ndarray | None = None,
) -> np.ndarray:
    """float64 reference: q [B, Hq, D]; caches [NB, bs, Hkv, D] as float values
    (already decoded codes when scales are given); returns [B, Hq, D]."""
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    b_, hq, d = q.shape
    hkv = kc.shape[2]
    g = hq // hkv
    ks = np.ones(hkv) if k_scale is None else np.broadcast_to(np.asarray(k_scale, np.float64).reshape(-1), (hkv,))
    vs = np.ones(hkv) if v_scale is None else np.broadcast_to(np.asarray(v_scale, np.float64).reshape(-1), (hkv,))
    out = np.zeros((b_, hq, d))
    for b in range(b_):
        n = min(seq_lens[b], len(block_tables[b]) * block_size)
        if n <= 0:
            continue
        tok = np.arange(n)
        blk = np.asarray(block_tables[b])[tok // block_size]
        off = tok % block_size
        kk = kc[blk, off] * ks[None, :, None]  # [n, Hkv, D]
        vv = vc[blk, off] * vs[None, :, None]
        for h in range(hq):
            s = kk[:, h // g, :] @ q[b, h] * scale
            s = s - s.max()
            p = np.exp(s)
            out[b, h] = (p @ vv[:, h // g, :]) / p.sum()
    return out


def chunk_rows(q_start, seq_lens, tq: int) -> list[tuple[int, int, int]]:
    """(first row, rows L, position of the first row) per chunk: rows
    [max(q_start[n], end of chunk n-1), max(q_start[n+1], that)) clamped to
    [0, tq); the first row sits at seq_lens[n] - L."""
    out = []
    end = 0
    for n in range(len(seq_lens)):
        a = min(max(int(q_start[n]), 0), tq)
        b = min(max(int(q_start[n + 1]), 0), tq)
        row0 = max(a, end)
        row1 = max(b, a, end)
        end = row1
        length = row1 - row0
        out.append((row0, length, int(seq_lens[n]) - length))
    return out


def paged_prefill_fp64(
    q: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    block_tables: list[list[int]],
    seq_lens: list[int],
    q_start: list[int],
    block_size: int,
    scale: float,
    k_scale: np.ndarray | None = None,
    v_scale: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """float64 chunked prefill: q [Tq, Hq, D]; caches [NB, bs, Hkv, D] as
    float values; returns (out [Tq, Hq, D], covered [Tq] bool).  Rows of no
    chunk are NaN; rows at negative positions are zero."""
    q = np.asarray(q, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    tq, hq, d = q.shape
    hkv = kc.shape[2]
    g = hq // hkv
    ks = np.ones(hkv) if k_scale is None else np.broadcast_to(np.asarray(k_scale, np.float64).reshape(-1), (hkv,))
    vs = np.ones(hkv) if v_scale is None else np.broadcast_to(np.asarray(v_scale, np.float64).reshape(-1), (hkv,))
    out = np.full((tq, hq, d), np.nan)
    covered = np.zeros(tq, dtype=bool)
    for n, (row0, length, pos0) in enumerate(chunk_rows(q_start, seq_lens, tq)):
        if length == 0:
            continue
        covered[row0:row0 + length] = True
        out[row0:row0 + length] = 0.0
        cap = len(block_tables[n]) * block_size
        kvlen = max(0, min(pos0 + length, cap))
        if kvlen == 0:
            continue
        tok = np.arange(kvlen)
        blk = np.asarray(block_tables[n])[tok // block_size]
        off = tok % block_size
        kk = kc[blk, off] * ks[None, :, None]
        vv = vc[blk, off] * vs[None, :, None]
        pos = pos0 + np.arange(length)
        mask = tok[None, :] <= pos[:, None]  # [L, kvlen]
        live = mask.any(axis=1)
        for h in range(hq):
            s = q[row0:row0 + length, h, :] @ kk[:, h // g, :].T * scale
            s = np.where(mask, s, -np.inf)
            m = np.where(live, s.max(axis=1), 0.0)
            p = np.where(mask, np.exp(s - m[:, None]), 0.0)
            den = p.sum(axis=1)
            o = (p @ vv[:, h // g, :]) / np.where(live, den, 1.0)[:, None]
            out[row0:row0 + length, h] = np.where(live[:, None], o, 0.0)
    return out, covered


def paged_prefill_by_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: list[list[int]],
    seq_lens: list[int],
    q_start: list[int],
    block_size: int = 16,
    scale: float | None = None,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> dict[int, torch.Tensor]:
    """Chunked prefill as one reference decode per row: row at position p
    is paged_attention_cpu over the sequence's table with seq_len p + 1.
    Returns {row: [Hq, D]} for the rows at non-negative positions."""
    out: dict[int, torch.Tensor] = {}
    for n, (row0, length, pos0) in enumerate(chunk_rows(q_start, seq_lens, q.shape[0])):
        for i in range(length):
            pos = pos0 + i
            if pos < 0:
                continue
            res = paged_attention_cpu(
                q[row0 + i].unsqueeze(0), k_cache, v_cache, {"r": block_tables[n]}, {"r": pos + 1},
                block_size, scale, k_scale, v_scale,
            )
            out[row0 + i] = res["r"]
    return out
