"""Physical layouts of the paged KV cache.

Every cache tensor handed to the kernels has the reference's logical shape
[num_blocks, block_size, num_kv_heads, head_dim] (reference
kernels/paged_attention.py:214-215), so callers index it exactly as the
reference does.  What differs is the storage order behind that view:

  "token_major"  storage [NB, bs, Hkv, D] -- the reference's order.
  "native"       K storage [NB, Hkv, bs, D]: each (block, head) tile is one
                 contiguous bs*D run (2 KiB for e4m3 at D=128, 4 KiB bf16),
                 token rows of D elements inside it;
                 V storage [NB, Hkv, D, bs]: the same tile transposed, so the
                 bs tokens of one channel d are contiguous.
  "paired"       the native K and V tiles of one (block, head) side by side
                 in one allocation, storage [NB, Hkv, {K tile, V tile}]: a
                 (block, head) is one contiguous 2*bs*D run (4 KiB for e4m3
                 at D=128).  k_cache and v_cache are two views of it with the
                 native tile strides.

The native order serves the MFMA decode kernel: a K row is an A-operand row
of the QK^T product, and a run of tokens of one V channel is a B-operand
column of the P.V product, so both load straight from HBM into MFMA
operand registers with no LDS transpose.  A (block, head) tile is a
multiple of the 128-byte cache line and starts on a tile boundary.  The
paired order makes each (block, head) one 4 KiB read instead of two 2 KiB
reads at unrelated addresses, which MI355X's HBM serves faster when the
blocks are scattered: the Llama-3-8B-shaped FP8 decode step takes 110.2 us
paired vs 112.7 us native (same kernel, bit-identical outputs).
"""

from __future__ import annotations

import torch

LAYOUTS = ("paired", "native", "token_major")


def alloc_kv_cache(
    num_blocks: int,
    block_size: int,
    num_kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    device: torch.device | str,
    layout: str = "paired",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Allocates (k_cache, v_cache), each viewed as [NB, bs, Hkv, D]."""
    nb, bs, h, d = num_blocks, block_size, num_kv_heads, head_dim
    if layout == "paired":
        buf = torch.empty(nb, h, 2, bs * d, dtype=dtype, device=device)
        k = buf[:, :, 0].view(nb, h, bs, d).permute(0, 2, 1, 3)
        v = buf[:, :, 1].view(nb, h, d, bs).permute(0, 3, 1, 2)
        return k, v
    if layout == "token_major":
        k = torch.empty(nb, bs, h, d, dtype=dtype, device=device)
        v = torch.empty(nb, bs, h, d, dtype=dtype, device=device)
        return k, v
    if layout == "native":
        k = torch.empty(nb, h, bs, d, dtype=dtype, device=device).permute(0, 2, 1, 3)
        v = torch.empty(nb, h, d, bs, dtype=dtype, device=device).permute(0, 3, 1, 2)
        return k, v
    raise ValueError(f"unknown KV layout {layout!r}; expected one of {LAYOUTS}")


def to_layout(logical: torch.Tensor, layout: str, is_value: bool) -> torch.Tensor:
    """Copies a logical [NB, bs, Hkv, D] tensor into `layout` storage."""
    if logical.dim() != 4:
        raise ValueError("expected a [num_blocks, block_size, num_kv_heads, head_dim] tensor")
    nb, bs, h, d = logical.shape
    if layout == "paired":
        raise ValueError("the paired layout holds K and V together: use to_paired(k, v)")
    if layout == "token_major":
        return logical.contiguous()
    if layout == "native":
        if is_value:
            return logical.permute(0, 2, 3, 1).contiguous().permute(0, 3, 1, 2)
        return logical.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    raise ValueError(f"unknown KV layout {layout!r}; expected one of {LAYOUTS}")


def to_paired(k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Copies logical [NB, bs, Hkv, D] K and V into one paired allocation."""
    if k.dim() != 4 or k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("expected K and V of one [num_blocks, block_size, num_kv_heads, head_dim] shape and dtype")
    nb, bs, h, d = k.shape
    kp, vp = alloc_kv_cache(nb, bs, h, d, k.dtype, k.device, "paired")
    kp.copy_(k)
    vp.copy_(v)
    return kp, vp


def layout_of(cache: torch.Tensor, is_value: bool) -> str:
    """Names the storage order of a [NB, bs, Hkv, D] cache view ("other" if neither)."""
    nb, bs, h, d = cache.shape
    s = cache.stride()
    if s == (bs * h * d, h * d, d, 1):
        return "token_major"
    if not is_value and s == (h * bs * d, d, bs * d, 1):
        return "native"
    if is_value and s == (h * d * bs, 1, d * bs, bs):
        return "native"
    if not is_value and s == (h * 2 * bs * d, d, 2 * bs * d, 1):
        return "paired"
    if is_value and s == (h * 2 * bs * d, 1, 2 * bs * d, bs):
        return "paired"
    return "other"
