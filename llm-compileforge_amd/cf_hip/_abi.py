"""ctypes binding of libcf_hip.so (declarations: include/cf_hip.h).

Descriptors are built the way the reference builds memref descriptors for
its compiled dylibs (reference compiler/dylib_ffi.py:22-56): data pointer,
element offset, sizes and element strides, here taken from a torch tensor.
"""

from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path
from typing import Any

import torch

ABI_VERSION = 1

# include/sfa.h SFADevice
SFA_CPU = 1
SFA_CUDA = 2
SFA_ROCM = 3

# include/cf_hip.h CfDtype
CF_F32 = 0
CF_F16 = 1
CF_BF16 = 2
CF_I64 = 3
CF_I32 = 4
CF_I8 = 5
CF_U8 = 6
CF_F8E4M3FN = 7

CF_OK = 0
CF_ERR_INVALID = -1
CF_ERR_HIP = -2
CF_ERR_WORKSPACE = -3
CF_ERR_UNSUPPORTED = -4
CF_ERR_OUT_OF_BLOCKS = -5
CF_ERR_NOT_FOUND = -6

_DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: CF_F32,
    torch.float16: CF_F16,
    torch.bfloat16: CF_BF16,
    torch.int64: CF_I64,
    torch.int32: CF_I32,
    torch.int8: CF_I8,
    torch.uint8: CF_U8,
    torch.float8_e4m3fn: CF_F8E4M3FN,
}


def _raw(rank: int) -> type[ctypes.Structure]:
    return type(
        f"SFATensorRaw{rank}",
        (ctypes.Structure,),
        {
            "_fields_": [
                ("allocated", ctypes.c_void_p),
                ("aligned", ctypes.c_void_p),
                ("offset", ctypes.c_int64),
                ("sizes", ctypes.c_int64 * rank),
                ("strides", ctypes.c_int64 * rank),
            ]
        },
    )


SFATensorRaw1, SFATensorRaw2, SFATensorRaw3, SFATensorRaw4 = (_raw(r) for r in (1, 2, 3, 4))


class _SFAUnion(ctypes.Union):
    _fields_ = [("r1", SFATensorRaw1), ("r2", SFATensorRaw2), ("r3", SFATensorRaw3), ("r4", SFATensorRaw4)]


class SFATensor(ctypes.Structure):
    _anonymous_ = ("u",)
    _fields_ = [
        ("device", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("elem_size", ctypes.c_int32),
        ("u", _SFAUnion),
    ]


class CfTensor(ctypes.Structure):
    _fields_ = [("t", SFATensor), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)]


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"dtype {dtype} has no cf_hip code") from None


# CfTensor as bytes: SFATensor {device, rank, elem_size (i32), pad, union
# at 16: allocated, aligned (pointers), offset, sizes[r], strides[r] (i64)},
# then dtype, reserved (i32) at 104.  One pack per descriptor (the
# structures below give the same layout; tests/test_abi.py compares them).
_PACK = {r: struct.Struct(f"<iii4xQQq{r}q{r}q{(4 - r) * 16}xii") for r in (1, 2, 3, 4)}


def descriptor(t: torch.Tensor) -> CfTensor:
    """Builds a CfTensor over `t` (no copy; `t` must outlive the call)."""
    rank = t.dim()
    if not 1 <= rank <= 4:
        raise ValueError(f"cf_hip descriptors have rank 1..4, got a rank-{rank} tensor")
    esize = t.element_size()
    off = t.storage_offset()
    # The storage base plus the element offset, like a memref descriptor.
    base = t.data_ptr() - off * esize
    return CfTensor.from_buffer_copy(_PACK[rank].pack(
        SFA_ROCM if t.is_cuda else SFA_CPU, rank, esize, base, base, off, *t.shape, *t.stride(),
        dtype_code(t.dtype), 0))


def _lib_path() -> Path:
    env = os.environ.get("CF_HIP_LIB")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "libcf_hip.so"


_LIB: ctypes.CDLL | None = None

_P = ctypes.POINTER(CfTensor)

# name -> (restype, argtypes); keep in step with include/cf_hip.h
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "cf_abi_version": (ctypes.c_int32, []),
    "cf_last_error": (ctypes.c_int32, [ctypes.c_char_p, ctypes.c_uint64]),
    "cf_paged_decode_workspace_bytes": (
        ctypes.c_int32,
        [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
         ctypes.c_int32, ctypes.POINTER(ctypes.c_uint64)],
    ),
    "cf_paged_decode": (
        ctypes.c_int32,
        [_P, _P, _P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, _P, ctypes.c_void_p,
         ctypes.c_uint64, ctypes.c_void_p],
    ),
    "cf_paged_decode_shared": (
        ctypes.c_int32,
        [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, _P, ctypes.c_void_p,
         ctypes.c_uint64, ctypes.c_void_p],
    ),
    "cf_paged_decode_shared_noalloc": (
        ctypes.c_int32,
        [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, _P, ctypes.c_void_p],
    ),
    "cf_prefill_chunk_workspace_bytes": (
        ctypes.c_int32,
        [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
         ctypes.POINTER(ctypes.c_uint64)],
    ),
    "cf_prefill_chunk_fp8": (
        ctypes.c_int32,
        [_P, _P, _P, _P, _P, _P, _P, _P, ctypes.c_float, ctypes.c_int32, _P, ctypes.c_void_p, ctypes.c_uint64,
         ctypes.c_void_p],
    ),
    "cf_fp8_amax_scale": (ctypes.c_int32, [_P, _P, ctypes.c_void_p]),
    "cf_kv_amax_scale": (ctypes.c_int32, [_P, _P, ctypes.c_void_p]),
    "cf_fp8_quantize": (ctypes.c_int32, [_P, _P, _P, ctypes.c_void_p]),
    "cf_fp8_quantize_kv": (ctypes.c_int32, [_P, _P, _P, _P, _P, _P, ctypes.c_void_p]),
    "cf_fp8_dequantize": (ctypes.c_int32, [_P, _P, _P, ctypes.c_void_p]),
    "cf_kv_write_fp8": (ctypes.c_int32, [_P, _P, _P, _P, _P, _P, _P, ctypes.c_void_p]),
    "cf_paged_write": (ctypes.c_int32, [_P, _P, _P, _P, ctypes.c_void_p]),
    "cf_paged_gather": (ctypes.c_int32, [_P, _P, _P, _P, ctypes.c_void_p]),
    "cf_bp_create": (ctypes.c_int32, [ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ctypes.c_void_p)]),
    "cf_bp_destroy": (ctypes.c_int32, [ctypes.c_void_p]),
    "cf_bp_num_free": (ctypes.c_int32, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_ref_count": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_allocate": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64, ctypes.c_void_p,
                                        ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_free": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p]),
    "cf_bp_free_block": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int64]),
    "cf_bp_increment_ref_count": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int64]),
    "cf_bp_assign_cached_blocks": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p,
                                                    ctypes.c_int64]),
    "cf_bp_ensure_blocks": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64]),
    "cf_bp_share_prefix": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_get_blocks": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_prepare_writes": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                              ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_set_len": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64]),
    "cf_bp_bind_rows": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]),
    "cf_bp_row_of": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)]),
    "cf_bp_table_deltas": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                            ctypes.POINTER(ctypes.c_int64)]),
    "cf_bp_shared_prefix_lens": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "cf_block_tables_apply": (ctypes.c_int32, [_P, _P, _P, ctypes.c_void_p]),
    "cf_copy_blocks": (ctypes.c_int32, [_P, _P, ctypes.c_void_p]),
    "cf_stage_from_host": (ctypes.c_int32, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]),
    "cf_profile_enable": (ctypes.c_int32, [ctypes.c_int32]),
    "cf_profile_reset": (ctypes.c_int32, []),
    "cf_profile_query": (
        ctypes.c_int32,
        [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)],
    ),
    "cf_profile_reserve": (ctypes.c_int32, [ctypes.c_int64]),
    "cf_profile_durations": (
        ctypes.c_int32,
        [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)],
    ),
}


def lib() -> ctypes.CDLL:
    """Loads libcf_hip.so once; raises RuntimeError when it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = _lib_path()
    if not path.exists():
        raise RuntimeError(
            f"libcf_hip.so not found at {path}: build it with "
            "`python llm-compileforge_amd/csrc/build.py` (or __graft_entry__.build())"
        )
    handle = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    version = handle.cf_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libcf_hip.so ABI version {version}, expected {ABI_VERSION}")
    _LIB = handle
    return handle


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().cf_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Maps a C status to the Python exception the reference would raise."""
    if rc == CF_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (CF_ERR_INVALID, CF_ERR_WORKSPACE):
        raise ValueError(msg)
    if rc == CF_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if rc == CF_ERR_NOT_FOUND:
        raise KeyError(msg)
    raise RuntimeError(msg)


def ref(d: CfTensor | None) -> Any:
    return ctypes.byref(d) if d is not None else None


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The current stream of `device` as a hipStream_t value."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream
