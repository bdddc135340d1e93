"""compiler.quantize: re-exports the FP8 KV quantizer (reference
compiler/quantize/__init__.py:23)."""

from kernels.quantize.fp8_kv_cache import FP8KVCacheQuantizer

__all__ = ["FP8KVCacheQuantizer"]
