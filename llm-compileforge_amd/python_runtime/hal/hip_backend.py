"""HIP backend of the HAL: the paged-attention path as OpExecutor ops.

Follows the reference's "registered kernel, else fallback" dispatch
(python_runtime/hal/triton_backend.py:58-65): ops this backend implements
run as HIP kernels from libcf_hip.so; any other op goes to the fallback
executor (for example the reference's PyTorchBackend); with no fallback an
unknown op raises ValueError("Unknown op: ...") like the reference's
PyTorchBackend.execute (pytorch_backend/__init__.py:111-113).

Ops:
  paged_attention     inputs [query, key_cache, value_cache, block_table
                      (, seq_lens)] -- the operand list of the reference's
                      planned hal.paged_attention op
                      (sf-dialect/include/Sf/HALOps.td:184-189).  kwargs:
                      seq_lens, block_size, scale, k_scale, v_scale,
                      partition_tokens, shared_prefix_lens.  Returns
                      [B, Hq, D].
  chunked_prefill_attention
                      inputs [query, key_cache, value_cache, block_tables,
                      seq_lens, q_start]; kwargs: block_size, scale,
                      k_scale, v_scale.  Returns [Tq, Hq, D].
  kv_cache_write_fp8  inputs [k_new, v_new, slot_mapping, key_cache,
                      value_cache, k_scale, v_scale]; returns key_cache.
  cache_write         the planned hal.cache_write (HALOps.td:195-199):
                      inputs [key, value, slot_mapping, key_cache,
                      value_cache]; caches of any float dtype and layout,
                      e4m3fn caches quantize with kwargs k_scale / v_scale;
                      slots outside the cache are skipped.  Returns key_cache.
  cache_read          the planned hal.cache_read (HALOps.td:190-194):
                      inputs [key_cache, value_cache, block_table]; kwargs
                      seq_len (default: the whole table), k_scale, v_scale,
                      out_dtype.  Returns [2, R, seq_len, Hkv, D] (keys,
                      values); ids outside the cache read as zeros.
  scaled_dot_product_attention
                      the reference's registered op (pytorch_backend/
                      _ops_attention.py:13-53, registered with 3-4 inputs
                      at :191): inputs [query, key, value(, attn_mask)],
                      kwargs attn_mask, dropout_p, is_causal, scale.  A
                      decode-shaped call -- query [B, H, 1, D] over dense
                      key/value [B, Hkv, S, D] (Hkv = H, or 1 broadcast),
                      one float dtype, no mask, no dropout -- runs on the
                      HIP decode kernels, reading key/value in place as
                      paged blocks; any other call goes to the fallback
                      executor unchanged.
  fp8_amax_scale      inputs [x]; per-head scales [H] (head axis -2).
  fp8_quantize        inputs [x, scales]; e4m3fn codes.
  fp8_dequantize      inputs [codes, scales]; float32 values.
"""

from __future__ import annotations

import math
from collections.abc import Callable
from typing import Any

import torch

from cf_hip import ops as _ops
from python_runtime.hal import registry
from python_runtime.hal.interface import OpExecutor

# op name -> (min inputs, max inputs)
_ARITY: dict[str, tuple[int, int]] = {
    "paged_attention": (4, 5),
    "chunked_prefill_attention": (6, 6),
    "kv_cache_write_fp8": (7, 7),
    "cache_write": (5, 5),
    "cache_read": (3, 3),
    "scaled_dot_product_attention": (3, 4),
    "fp8_amax_scale": (1, 1),
    "fp8_quantize": (2, 2),
    "fp8_dequantize": (2, 2),
}


class HipBackend(OpExecutor):
    """OpExecutor running the paged-attention path on MI355X.

    Args:
        fallback: executor for ops this backend does not implement.
        partition_tokens: default split-KV partition length for decode.
    """

    def __init__(self, fallback: OpExecutor | None = None, partition_tokens: int = _ops.DEFAULT_PARTITION_TOKENS):
        self._fallback = fallback
        self._partition_tokens = partition_tokens
        # dense-SDPA block tables, per (batch, blocks per batch row, blocks, device)
        self._dense_tables: dict[tuple[int, int, int, str], torch.Tensor] = {}
        self._handlers: dict[str, Callable[..., torch.Tensor]] = {
            "paged_attention": self._paged_attention,
            "chunked_prefill_attention": self._chunked_prefill,
            "kv_cache_write_fp8": self._kv_cache_write_fp8,
            "cache_write": self._cache_write,
            "cache_read": self._cache_read,
            "scaled_dot_product_attention": self._sdpa,
            "fp8_amax_scale": lambda inputs, **kw: _ops.fp8_amax_scale(inputs[0]),
            "fp8_quantize": lambda inputs, **kw: _ops.fp8_quantize(inputs[0], inputs[1]),
            "fp8_dequantize": lambda inputs, **kw: _ops.fp8_dequantize(inputs[0], inputs[1]),
        }

    @staticmethod
    def supported_ops() -> list[str]:
        return sorted(_ARITY)

    def execute(self, op_name: str, inputs: list[Any], **kwargs: Any) -> torch.Tensor:
        handler = self._handlers.get(op_name)
        if handler is None:
            if self._fallback is not None:
                return self._fallback.execute(op_name, inputs, **kwargs)
            raise ValueError(f"Unknown op: {op_name}")
        lo, hi = _ARITY[op_name]
        n = len(inputs)
        if n < lo:
            raise ValueError(f"Op '{op_name}' requires at least {lo} inputs, got {n}")
        if n > hi:
            raise ValueError(f"Op '{op_name}' accepts at most {hi} inputs, got {n}")
        return handler(inputs, **kwargs)

    def _paged_attention(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        from kernels.paged_attention import paged_attention_tensors

        q, k_cache, v_cache, table = inputs[:4]
        seq_lens = inputs[4] if len(inputs) > 4 else kw.get("seq_lens")
        block_size = int(kw.get("block_size", k_cache.shape[1]))
        if seq_lens is None:
            # The reference default for a request without a length: the whole table.
            seq_lens = torch.full((table.shape[0],), table.shape[1] * block_size, dtype=torch.int32,
                                  device=table.device)
        elif not isinstance(seq_lens, torch.Tensor):
            seq_lens = torch.tensor(list(seq_lens), dtype=torch.int32, device=table.device)
        return paged_attention_tensors(
            q, k_cache, v_cache, table, seq_lens, block_size, kw.get("scale"),
            k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"),
            partition_tokens=int(kw.get("partition_tokens", self._partition_tokens)),
            shared_prefix_lens=kw.get("shared_prefix_lens"),
        )

    def _sdpa(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        plan = _dense_decode_plan(inputs, kw)
        if plan is None:
            if self._fallback is None:
                raise ValueError("scaled_dot_product_attention: only decode-shaped calls (query length 1, dense "
                                 "key/value, no mask or dropout) run on the HIP backend, and no fallback is set")
            return self._fallback.execute("scaled_dot_product_attention", inputs, **kw)
        q, kv, vv, bs, bpb, nblk, scale = plan
        B, H, _, D = q.shape
        key = (B, bpb, nblk, str(q.device))
        table = self._dense_tables.get(key)
        if table is None:
            table = (torch.arange(B, device=q.device, dtype=torch.int32)[:, None] * bpb
                     + torch.arange(nblk, device=q.device, dtype=torch.int32)[None, :]).contiguous()
            self._dense_tables[key] = table
        lens = torch.full((B,), nblk * bs if not kw.get("is_causal", False) else 1, dtype=torch.int32,
                          device=q.device)
        out = torch.empty(B, H, 1, D, dtype=q.dtype, device=q.device)
        _ops.paged_decode(q[:, :, 0, :], kv, vv, table, lens, scale, bs,
                          partition_tokens=max(self._partition_tokens // bs * bs, bs), out=out[:, :, 0, :])
        return out

    def _chunked_prefill(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        from kernels.paged_attention import chunked_prefill_attention

        q, k_cache, v_cache, tables, seq_lens, q_start = inputs
        return chunked_prefill_attention(
            q, k_cache, v_cache, tables, seq_lens, q_start, int(kw.get("block_size", k_cache.shape[1])),
            kw.get("scale"), k_scale=kw.get("k_scale"), v_scale=kw.get("v_scale"),
        )

    def _kv_cache_write_fp8(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        k_new, v_new, slots, k_cache, v_cache, k_scale, v_scale = inputs
        _ops.kv_write_fp8(k_new, v_new, slots, k_cache, v_cache, k_scale, v_scale)
        return k_cache


    def _cache_write(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        key, value, slots, k_cache, v_cache = inputs
        _ops.paged_write(key, slots, k_cache, kw.get("k_scale"))
        _ops.paged_write(value, slots, v_cache, kw.get("v_scale"))
        return k_cache

    def _cache_read(self, inputs: list[Any], **kw: Any) -> torch.Tensor:
        k_cache, v_cache, table = inputs
        seq_len = int(kw.get("seq_len", table.shape[1] * k_cache.shape[1]))
        dt = kw.get("out_dtype") or (torch.float32 if k_cache.dtype == torch.float8_e4m3fn else k_cache.dtype)
        out = torch.empty(2, table.shape[0], seq_len, k_cache.shape[2], k_cache.shape[3], dtype=dt,
                          device=k_cache.device)
        _ops.paged_gather(k_cache, table, seq_len, scale=kw.get("k_scale"), out=out[0])
        _ops.paged_gather(v_cache, table, seq_len, scale=kw.get("v_scale"), out=out[1])
        return out


def _dense_decode_plan(inputs: list[Any], kw: dict[str, Any]):
    """For a decode-shaped dense SDPA call: (query, key view, value view,
    block_size, blocks per batch row, blocks per sequence, scale), where the
    views present key/value [B, Hkv, S, D] as paged caches [NB, bs, Hkv, D]
    over the same memory (block b * per_row + j holds tokens [j*bs,
    (j+1)*bs) of batch row b).  None when the call is not one this backend
    runs (the fallback executor then takes it as is)."""
    q, k, v = inputs[0], inputs[1], inputs[2]
    mask = kw.get("attn_mask")
    if mask is None and len(inputs) > 3:
        mask = inputs[3]
    if mask is not None or float(kw.get("dropout_p", 0.0) or 0.0) != 0.0:
        return None
    if kw.get("enable_gqa", False):
        return None
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        return None
    if not (q.is_cuda and k.is_cuda and v.is_cuda) or torch.version.hip is None:
        return None
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or q.shape[2] != 1:
        return None
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return None
    B, H, _, D = q.shape
    Bk, Hkv, S, Dk = k.shape
    if tuple(v.shape) != (Bk, Hkv, S, Dk) or Bk != B or Dk != D or S < 1 or D < 1:
        return None
    if Hkv != H and Hkv != 1:  # torch SDPA broadcasts one KV head; other head counts are its error
        return None
    if k.stride() != v.stride() or k.stride(3) != 1 or q.stride(3) != 1:
        return None
    sb, sh, ss, _ = k.stride()
    if ss < 1:
        return None
    bs = 16
    while bs > 1 and (S % bs != 0 or (B > 1 and sb % (bs * ss) != 0)):
        bs //= 2
    nblk = S // bs
    bpb = sb // (bs * ss) if B > 1 else nblk
    nb = (B - 1) * bpb + nblk
    # The last block of the last batch row ends at the tensor's last element
    # (S is a multiple of bs), so both views stay inside key/value.
    kv = torch.as_strided(k, (nb, bs, Hkv, D), (bs * ss, ss, sh, 1), k.storage_offset())
    vv = torch.as_strided(v, (nb, bs, Hkv, D), (bs * ss, ss, sh, 1), v.storage_offset())
    scale = kw.get("scale")
    scale = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    return q, kv, vv, bs, bpb, nblk, scale


def register_hip_backend(name: str = "hip") -> None:
    """Registers HipBackend's factory under `name` (once per process)."""
    if name not in registry.list_backends():
        registry.register(name, lambda **kw: HipBackend(**kw))


__all__ = ["HipBackend", "register_hip_backend"]
