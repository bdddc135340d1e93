"""Engine-side KV cache: CacheManager slabs and the executors' KV mixin, on the GPU."""

from python_runtime.engine._kv_cache import _KVCacheMixin, _normalize_kv_for_cache
from python_runtime.engine.cache_manager import CacheManager, _dict_to_proto_cache_policy

__all__ = ["CacheManager", "_KVCacheMixin", "_dict_to_proto_cache_policy", "_normalize_kv_for_cache"]
