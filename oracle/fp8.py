"""ctypes wrapper of the C FP8 oracle (fp8_e4m3.c).  TEST INFRASTRUCTURE ONLY.

Restates compiler/quantize/fp8_kv_cache.py:66-105 of the reference for
numpy float32 inputs: per-tensor or per-head amax scale, IEEE-division
quantize to OCP e4m3fn codes (uint8), exact dequantize.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_fp8.so"
_lib: ctypes.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(_LIB_PATH))
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        h.oracle_e4m3_from_f32.restype = ctypes.c_uint8
        h.oracle_e4m3_from_f32.argtypes = [ctypes.c_float]
        h.oracle_e4m3_to_f32.restype = ctypes.c_float
        h.oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        h.oracle_e4m3_encode.argtypes = [vp, vp, sz]
        h.oracle_e4m3_encode_bits.argtypes = [ctypes.c_uint32, ctypes.c_uint64, vp]
        h.oracle_e4m3_decode.argtypes = [vp, vp, sz]
        h.oracle_fp8_scale_from_amax.restype = ctypes.c_float
        h.oracle_fp8_scale_from_amax.argtypes = [ctypes.c_float]
        h.oracle_fp8_amax.restype = ctypes.c_float
        h.oracle_fp8_amax.argtypes = [vp, sz]
        h.oracle_fp8_quantize.argtypes = [vp, sz, ctypes.c_float, vp]
        h.oracle_fp8_dequantize.argtypes = [vp, sz, ctypes.c_float, vp]
        _lib = h
    return _lib


def _f32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes (uint8), round-to-nearest-even."""
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_e4m3_encode(x.ctypes.data, out.ctypes.data, x.size)
    return out


def encode_bits(start: int, count: int) -> np.ndarray:
    """Codes of the float32 values whose bit patterns are start..start+count-1."""
    out = np.empty(count, dtype=np.uint8)
    lib().oracle_e4m3_encode_bits(start, count, out.ctypes.data)
    return out


def decode(codes: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().oracle_e4m3_decode(c.ctypes.data, out.ctypes.data, c.size)
    return out


def scale_of(x: np.ndarray) -> np.float32:
    """quantize_block's scale: amax/448 (>= 1e-12), 1.0 for an all-zero block."""
    x = _f32(x)
    amax = lib().oracle_fp8_amax(x.ctypes.data, x.size)
    return np.float32(lib().oracle_fp8_scale_from_amax(amax))


def quantize(x: np.ndarray, scale: float) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_fp8_quantize(x.ctypes.data, x.size, ctypes.c_float(scale), out.ctypes.data)
    return out


def dequantize(codes: np.ndarray, scale: float) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().oracle_fp8_dequantize(c.ctypes.data, c.size, ctypes.c_float(scale), out.ctypes.data)
    return out


def quantize_block(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """(codes, scale) for one block, as FP8KVCacheQuantizer.quantize_block."""
    s = scale_of(x)
    return quantize(x, s), s


def quantize_per_head(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """x [..., H, D] -> (codes, scales [H]) with one scale per head (axis -2)."""
    x = _f32(x)
    h = x.shape[-2]
    scales = np.empty(h, dtype=np.float32)
    codes = np.empty(x.shape, dtype=np.uint8)
    for i in range(h):
        xi = np.ascontiguousarray(x[..., i, :])
        scales[i] = scale_of(xi)
        codes[..., i, :] = quantize(xi, scales[i])
    return codes, scales
