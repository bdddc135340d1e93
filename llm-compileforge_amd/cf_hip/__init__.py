"""cf_hip: MI355X (gfx950) paged decode attention and FP8 KV quantization.

The compute lives in libcf_hip.so (HIP kernels behind the C ABI declared in
include/cf_hip.h); this package holds the ctypes binding (`_abi`), tensor
wrappers (`ops`), physical KV layouts (`layout`) and seeded workloads
(`workloads`).
"""

from . import layout, ops, workloads
from ._abi import lib

__all__ = ["layout", "lib", "ops", "workloads"]
