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

The native order serves the MFMA decode kernel: a K row is an A-operand row
of the QK^T product, and a run of tokens of one V channel is a B-operand
column of the P.V product, so both load straight from HBM into MFMA
operand registers with no LDS transpose.  A (block, head) tile is a
multiple of the 128-byte cache line and starts on a tile boundary.
"""

from __future__ import annotations

import torch

LAYOUTS = ("native", "token_major")


def alloc_kv_cache(
    num_blocks: int,
    block_size: int,
    num_kv_heads: int,
    head_dim: int,
    dtype: torch.dtype,
    device: torch.device | str,
    layout: str = "native",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Allocates (k_cache, v_cache), each viewed as [NB, bs, Hkv, D]."""
    nb, bs, h, d = num_blocks, block_size, num_kv_heads, head_dim
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
    if layout == "token_major":
        return logical.contiguous()
    if layout == "native":
        if is_value:
            return logical.permute(0, 2, 3, 1).contiguous().permute(0, 3, 1, 2)
        return logical.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    raise ValueError(f"unknown KV layout {layout!r}; expected one of {LAYOUTS}")


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
    return "other"
