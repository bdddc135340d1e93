"""Kernel library: the reference's `kernels` import path on MI355X.

`paged_attention` (kernels/paged_attention.py) and the FP8 KV quantizer
(kernels/quantize) run as HIP kernels from libcf_hip.so.  The reference
selects its GPU path with HAS_TRITON (reference kernels/__init__.py:22-27);
this build has no Triton path, so HAS_TRITON is False and HAS_HIP reports
whether the HIP library is present.
"""

from pathlib import Path

HAS_TRITON = False
HAS_HIP = (Path(__file__).resolve().parent.parent / "cf_hip" / "libcf_hip.so").exists()

__all__ = ["HAS_HIP", "HAS_TRITON"]
