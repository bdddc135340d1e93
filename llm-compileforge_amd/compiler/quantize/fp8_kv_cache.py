"""compiler.quantize.fp8_kv_cache: the reference module path of the FP8 KV
quantizer (reference compiler/quantize/fp8_kv_cache.py:19)."""

from kernels.quantize.fp8_kv_cache import FP8KVCacheQuantizer

__all__ = ["FP8KVCacheQuantizer"]
