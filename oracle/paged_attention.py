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
