"""Prefix cache over the paged block pool."""

from python_runtime.engine.cache.radix_cache import RadixCache, RadixTreeNode

__all__ = ["RadixCache", "RadixTreeNode"]
