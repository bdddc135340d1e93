"""Quantization kernels: the FP8 KV-cache quantizer on MI355X."""

from kernels.quantize.fp8_kv_cache import FP8KVCacheQuantizer

__all__ = ["FP8KVCacheQuantizer"]
