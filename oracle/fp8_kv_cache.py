"""The reference's FP8KVCacheQuantizer restated with torch CPU ops.
TEST INFRASTRUCTURE ONLY.

Follows compiler/quantize/fp8_kv_cache.py:19-140 of the reference: the same
amax/448 scale with the 1e-12 clamp and the all-zero rule (:81-86), the
float32 division and torch float8_e4m3fn cast (:89), dequantize as
f32(code) * scale (:105), K and V with independent scales (:107-140).
"""

from __future__ import annotations

import torch


class FP8KVCacheQuantizerRef:
    SUPPORTED_HARDWARE: tuple[str, ...] = ("H100", "H200", "RTX_4090", "RTX_6000_ADA", "MI300")

    def __init__(self, block_size: int = 16) -> None:
        if block_size < 1:
            raise ValueError(f"block_size must be >= 1, got {block_size}")
        self.block_size = block_size
        self.fp8_max = 448.0

    def check_hardware_support(self, device_name: str) -> bool:
        return any(hw in device_name for hw in self.SUPPORTED_HARDWARE)

    def quantize_block(self, kv_block: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        amax = kv_block.float().abs().max()
        if amax == 0:
            scale = torch.tensor(1.0, dtype=torch.float32)
        else:
            scale = torch.clamp(amax / self.fp8_max, min=1e-12)
        return (kv_block.float() / scale).to(torch.float8_e4m3fn), scale

    def dequantize_block(self, quant_block: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        return quant_block.float() * scale

    def quantize_kv(self, k: torch.Tensor, v: torch.Tensor):
        kq, ks = self.quantize_block(k)
        vq, vs = self.quantize_block(v)
        return kq, ks, vq, vs

    def dequantize_kv(self, kq, ks, vq, vs):
        return self.dequantize_block(kq, ks), self.dequantize_block(vq, vs)

    def quantize_per_head(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """quantize_block applied to each head slice x[..., h, :]."""
        codes = torch.empty(x.shape, dtype=torch.float8_e4m3fn)
        scales = torch.empty(x.shape[-2], dtype=torch.float32)
        for h in range(x.shape[-2]):
            c, s = self.quantize_block(x[..., h, :])
            codes[..., h, :] = c
            scales[h] = s
        return codes, scales
