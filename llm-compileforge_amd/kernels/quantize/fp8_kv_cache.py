"""FP8 (OCP E4M3) KV-cache quantization on MI355X.

Drop-in for the reference's `FP8KVCacheQuantizer` (reference
compiler/quantize/fp8_kv_cache.py:19-140): same class, attributes, methods
and results.  Quantized codes and scales are bit-identical to the
reference's torch CPU arithmetic (scale = amax/448 clamped at 1e-12, 1.0 for
an all-zero block; code = float8_e4m3fn(x / scale)); the work runs in
libcf_hip.so's kernels on device tensors.

gfx950 stores the OCP e4m3fn format natively (bias 7, max 448, NaN =
S.1111.111), the format torch.float8_e4m3fn denotes -- not the FNUZ variant
of gfx942.

Additions (the reference has no per-head or paged entry points):
  quantize_per_head  one scale per KV head (axis -2), the per-(layer,
                     KV-head) scaling of a layer's cache;
  write_kv_fp8       quantize new K/V rows straight into paged cache slots.
"""

from __future__ import annotations

import torch

from cf_hip import ops as _ops


class FP8KVCacheQuantizer:
    """Per-block FP8 quantization/dequantization for KV cache tensors.

    Each block passed to quantize_block gets one scale, amax / 448, so
    outliers of one block do not widen another's range.

    Args:
        block_size: Number of tokens per KV block (default 16).
    """

    # The reference's list (fp8_kv_cache.py:32-38) plus the gfx950 parts
    # this build targets.
    SUPPORTED_HARDWARE: tuple[str, ...] = (
        "H100",
        "H200",
        "RTX_4090",
        "RTX_6000_ADA",
        "MI300",
        "MI350",
        "MI355",
    )

    def __init__(self, block_size: int = 16) -> None:
        if block_size < 1:
            raise ValueError(f"block_size must be >= 1, got {block_size}")
        self.block_size = block_size
        self.fp8_max: float = 448.0

    def check_hardware_support(self, device_name: str) -> bool:
        """True if the device name contains one of SUPPORTED_HARDWARE (substring match)."""
        return any(hw in device_name for hw in self.SUPPORTED_HARDWARE)

    def _has_fp8_dtype(self) -> bool:
        """Whether torch exposes float8_e4m3fn."""
        return hasattr(torch, "float8_e4m3fn")

    @staticmethod
    def _check_device(name: str, t: torch.Tensor) -> None:
        if not (isinstance(t, torch.Tensor) and t.is_cuda and torch.version.hip is not None):
            where = t.device if isinstance(t, torch.Tensor) else type(t).__name__
            raise ValueError(f"{name} must be a ROCm device tensor (got {where})")

    def quantize_block(self, kv_block: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Quantizes a KV block with one scale for the whole tensor.

        Returns:
            (quant_block, scale): float8_e4m3fn codes of kv_block's shape and
            a 0-d float32 scale on the same device.
        """
        self._check_device("kv_block", kv_block)
        if not self._has_fp8_dtype():
            raise RuntimeError("torch.float8_e4m3fn is required")
        if kv_block.numel() == 0:
            raise RuntimeError("max(): Expected reduction dim to be specified for input.numel() == 0.")
        rows = kv_block.reshape(-1, 1, kv_block.shape[-1]) if kv_block.dim() > 0 else kv_block.reshape(1, 1, 1)
        scale = _ops.fp8_amax_scale(rows)
        quant = _ops.fp8_quantize(kv_block, scale)
        return quant, scale.reshape(())

    def dequantize_block(self, quant_block: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """float32(quant_block) * scale."""
        self._check_device("quant_block", quant_block)
        if quant_block.dtype != torch.float8_e4m3fn:
            raise ValueError(f"quant_block must be float8_e4m3fn, got {quant_block.dtype}")
        if not isinstance(scale, torch.Tensor):
            scale = torch.tensor(float(scale), dtype=torch.float32, device=quant_block.device)
        return _ops.fp8_dequantize(quant_block, scale.to(device=quant_block.device, dtype=torch.float32))

    def quantize_kv(
        self, k: torch.Tensor, v: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        """Quantizes K and V, each with its own scale."""
        k_quant, k_scale = self.quantize_block(k)
        v_quant, v_scale = self.quantize_block(v)
        return k_quant, k_scale, v_quant, v_scale

    def dequantize_kv(
        self,
        k_quant: torch.Tensor,
        k_scale: torch.Tensor,
        v_quant: torch.Tensor,
        v_scale: torch.Tensor,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Dequantizes K and V to float32."""
        return self.dequantize_block(k_quant, k_scale), self.dequantize_block(v_quant, v_scale)

    # ---- additions ------------------------------------------------------

    def quantize_per_head(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Quantizes x [..., H, D] with one scale per head h (axis -2).

        scales[h] applies quantize_block's rule to x[..., h, :]; returns
        (codes of x's shape, float32 scales [H]).
        """
        self._check_device("x", x)
        if x.dim() < 2:
            raise ValueError("x must have a head axis: [..., num_kv_heads, head_dim]")
        scales = _ops.fp8_amax_scale(x)
        return _ops.fp8_quantize(x, scales), scales

    @staticmethod
    def write_kv_fp8(
        k_new: torch.Tensor,
        v_new: torch.Tensor,
        slot_mapping: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        k_scale: torch.Tensor,
        v_scale: torch.Tensor,
    ) -> None:
        """Quantizes k_new/v_new [T, Hkv, D] into e4m3fn paged caches.

        Token i lands in block slot_mapping[i] // block_size at offset
        slot_mapping[i] % block_size; negative slots are skipped.
        """
        _ops.kv_write_fp8(k_new, v_new, slot_mapping, k_cache, v_cache, k_scale, v_scale)


__all__ = ["FP8KVCacheQuantizer"]
