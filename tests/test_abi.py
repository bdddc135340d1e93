"""C ABI checks that need no GPU: the library loads, exports every entry
point include/cf_hip.h declares, its descriptor structs have the layout a C
compiler gives include/sfa.h and include/cf_hip.h (the reference's
descriptor layout, include/sfa.h:54-99), and bad arguments come back as
error codes with a message before any HIP call."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from cf_hip import _abi

ROOT = Path(__file__).resolve().parent.parent


def _declared() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(cf_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_loads_and_reports_version():
    lib = _abi.lib()
    assert lib.cf_abi_version() == _abi.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    lib = _abi.lib()
    declared = _declared()
    assert declared, "no declarations found"
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert declared == set(_abi.SIGNATURES), declared ^ set(_abi.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_abi._lib_path())], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\b(cf_[a-z0-9_]+)$", out, flags=re.M))
    assert declared <= exported


def test_descriptor_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stddef.h>
#include <stdio.h>
#include "cf_hip.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(SFATensorRaw1), sizeof(SFATensorRaw2),
         sizeof(SFATensorRaw3), sizeof(SFATensorRaw4), sizeof(SFATensor), offsetof(SFATensor, r4),
         sizeof(CfTensor), offsetof(CfTensor, dtype), offsetof(SFATensorRaw4, strides));
  return 0;
}
''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    c_vals = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    py_vals = [
        ctypes.sizeof(_abi.SFATensorRaw1), ctypes.sizeof(_abi.SFATensorRaw2), ctypes.sizeof(_abi.SFATensorRaw3),
        ctypes.sizeof(_abi.SFATensorRaw4), ctypes.sizeof(_abi.SFATensor), _abi.SFATensor.u.offset,
        ctypes.sizeof(_abi.CfTensor), _abi.CfTensor.dtype.offset, _abi.SFATensorRaw4.strides.offset,
    ]
    assert c_vals == py_vals
    assert c_vals[:4] == [40, 56, 72, 88]  # reference include/sfa.h:19-23


def test_descriptor_of_a_strided_view():
    base = torch.arange(2 * 3 * 4 * 5, dtype=torch.float32).reshape(2, 3, 4, 5)
    view = base.permute(0, 2, 1, 3)[1:]
    d = _abi.descriptor(view)
    assert d.t.rank == 4 and d.t.elem_size == 4 and d.dtype == _abi.CF_F32
    assert d.t.device == _abi.SFA_CPU
    assert list(d.t.r4.sizes) == list(view.shape)
    assert list(d.t.r4.strides) == list(view.stride())
    assert d.t.r4.offset == view.storage_offset()
    assert d.t.r4.aligned + d.t.r4.offset * 4 == view.data_ptr()


@pytest.mark.parametrize("rank", [1, 2, 3, 4])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int32, torch.float8_e4m3fn])
def test_descriptor_fields_every_rank(rank, dtype):
    """The packed descriptor reads back field by field through the ctypes
    structures (the layout of include/cf_hip.h)."""
    full = torch.zeros(7 * 6 * 5 * 4, dtype=torch.float32).to(dtype).reshape(7, 6, 5, 4)
    view = full[(slice(1, None, 2),) * rank].reshape(full[(slice(1, None, 2),) * rank].shape)
    while view.dim() > rank:
        view = view[0]
    d = _abi.descriptor(view)
    raw = getattr(d.t, f"r{rank}")
    assert (d.t.device, d.t.rank, d.t.elem_size) == (_abi.SFA_CPU, rank, view.element_size())
    assert d.dtype == _abi.dtype_code(dtype) and d.reserved == 0
    assert list(raw.sizes) == list(view.shape) and list(raw.strides) == list(view.stride())
    assert raw.offset == view.storage_offset()
    assert raw.allocated == raw.aligned == view.data_ptr() - view.storage_offset() * view.element_size()


def _call_decode(q, k, v, bt, sl, out, ks=None, vs=None, bs=16, pt=512):
    lib = _abi.lib()
    ds = [_abi.descriptor(t) for t in (q, k, v, bt, sl, out)]
    kd = _abi.descriptor(ks) if ks is not None else None
    vd = _abi.descriptor(vs) if vs is not None else None
    return lib.cf_paged_decode(_abi.ref(ds[0]), _abi.ref(ds[1]), _abi.ref(ds[2]), _abi.ref(ds[3]),
                               _abi.ref(ds[4]), _abi.ref(kd), _abi.ref(vd), 0.125, bs, pt, _abi.ref(ds[5]),
                               None, 0, None)


def _decode_args():
    q = torch.zeros(2, 8, 64)
    k = torch.zeros(10, 16, 2, 64)
    v = torch.zeros(10, 16, 2, 64)
    bt = torch.zeros(2, 3, dtype=torch.int32)
    sl = torch.zeros(2, dtype=torch.int32)
    out = torch.zeros(2, 8, 64)
    return q, k, v, bt, sl, out


def test_host_memory_is_rejected_before_launch():
    rc = _call_decode(*_decode_args())
    assert rc == _abi.CF_ERR_INVALID
    assert "device memory" in _abi.last_error()


@pytest.mark.parametrize(
    "mutate, message",
    [
        (lambda a: a.__setitem__(0, torch.zeros(2, 8)), "rank"),
        (lambda a: a.__setitem__(3, torch.zeros(2, 3, dtype=torch.int64)), "block_tables: expected i32"),
        (lambda a: a.__setitem__(2, torch.zeros(10, 16, 2, 64, dtype=torch.float16)), "v_cache dtype"),
        (lambda a: a.__setitem__(5, torch.zeros(2, 8, 32)), "out shape"),
        (lambda a: a.__setitem__(4, torch.zeros(3, dtype=torch.int32)), "seq_lens has 3"),
    ],
)
def test_argument_errors_are_reported(mutate, message):
    args = list(_decode_args())
    mutate(args)
    lib = _abi.lib()
    ds = [_abi.descriptor(t) for t in args]
    for d in ds:
        d.t.device = _abi.SFA_ROCM  # reach the shape checks; nothing is launched
    rc = lib.cf_paged_decode(*(_abi.ref(d) for d in ds[:5]), None, None, 0.125, 16, 512, _abi.ref(ds[5]), None, 0,
                             None)
    assert rc == _abi.CF_ERR_INVALID
    assert message in _abi.last_error()


def test_gqa_ratio_and_partition_checks():
    args = list(_decode_args())
    args[1] = torch.zeros(10, 16, 3, 64)
    args[2] = torch.zeros(10, 16, 3, 64)
    lib = _abi.lib()
    ds = [_abi.descriptor(t) for t in args]
    for d in ds:
        d.t.device = _abi.SFA_ROCM
    rc = lib.cf_paged_decode(*(_abi.ref(d) for d in ds[:5]), None, None, 0.125, 16, 512, _abi.ref(ds[5]), None, 0,
                             None)
    assert rc == _abi.CF_ERR_INVALID and "multiple of num_kv_heads" in _abi.last_error()
    ds = [_abi.descriptor(t) for t in _decode_args()]
    for d in ds:
        d.t.device = _abi.SFA_ROCM
    rc = lib.cf_paged_decode(*(_abi.ref(d) for d in ds[:5]), None, None, 0.125, 16, 24, _abi.ref(ds[5]), None, 0,
                             None)
    assert rc == _abi.CF_ERR_INVALID and "partition_tokens" in _abi.last_error()


def test_fp8_cache_requires_scales_and_workspace_is_checked():
    q, _, _, bt, sl, out = _decode_args()
    k = torch.zeros(10, 16, 2, 64, dtype=torch.float8_e4m3fn)
    lib = _abi.lib()
    ds = [_abi.descriptor(t) for t in (q, k, k, bt, sl, out)]
    for d in ds:
        d.t.device = _abi.SFA_ROCM
    rc = lib.cf_paged_decode(*(_abi.ref(d) for d in ds[:5]), None, None, 0.125, 16, 512, _abi.ref(ds[5]), None, 0,
                             None)
    assert rc == _abi.CF_ERR_INVALID and "k_scale" in _abi.last_error()
    # three blocks of 16 with 16-token partitions -> 3 partitions -> workspace needed
    ds = [_abi.descriptor(t) for t in _decode_args()]
    for d in ds:
        d.t.device = _abi.SFA_ROCM
    rc = lib.cf_paged_decode(*(_abi.ref(d) for d in ds[:5]), None, None, 0.125, 16, 16, _abi.ref(ds[5]), None, 0,
                             None)
    assert rc == _abi.CF_ERR_WORKSPACE and "workspace" in _abi.last_error()


def test_workspace_size_formula():
    n = ctypes.c_uint64()
    lib = _abi.lib()
    def generic_bytes(batch, hq, d, parts):
        if parts <= 1:
            return 0
        rows = batch * hq * parts
        return ((rows * d * 4 + 255) // 256) * 256 + rows * 8

    # block size 8: the generic path only -> partition partials
    assert lib.cf_paged_decode_workspace_bytes(64, 32, 8, 128, 1024, 8, 512, ctypes.byref(n)) == 0
    # 64 x 8 x 16 partitions of 512 tokens already fill the GPU: the caller's length stands
    assert n.value == generic_bytes(64, 32, 128, 1024 * 8 // 512)
    assert lib.cf_paged_decode_workspace_bytes(64, 32, 8, 128, 32, 8, 512, ctypes.byref(n)) == 0
    # 256 tokens: one partition of 512 would give 512 workgroups, so the generic path
    # halves the partition (512 -> 256 -> 128) until 64 x 8 x 2 = 1024 workgroups
    assert n.value == generic_bytes(64, 32, 128, 2)
    assert lib.cf_paged_decode_workspace_bytes(1, 8, 8, 128, 2, 8, 512, ctypes.byref(n)) == 0
    assert n.value == 0  # 16 tokens: one partition at the 32-token floor, no workspace
    # 64 query heads on one KV head: 512-token partitions would need 165 KB of LDS per
    # workgroup, so the generic path halves them to 64 tokens (49 KB): 8192 / 64 partials
    assert lib.cf_paged_decode_workspace_bytes(64, 64, 1, 128, 512, 16, 512, ctypes.byref(n)) == 0
    assert n.value >= generic_bytes(64, 64, 128, 8192 // 64)
    # small batch (the opt-125m shape): 4 x 12 heads, 512 tokens -> partitions of 32 tokens
    assert lib.cf_paged_decode_workspace_bytes(4, 12, 12, 64, 32, 8, 512, ctypes.byref(n)) == 0
    assert n.value == generic_bytes(4, 12, 64, 256 // 32)
    # block size 16: at least the MFMA path's per-wave slots
    assert lib.cf_paged_decode_workspace_bytes(64, 32, 8, 128, 32, 16, 512, ctypes.byref(n)) == 0
    assert n.value > 0 and n.value % 8 == 0
    assert lib.cf_paged_decode_workspace_bytes(64, 32, 8, 128, 32, 16, 24, ctypes.byref(n)) == _abi.CF_ERR_INVALID
    assert lib.cf_paged_decode_workspace_bytes(64, 32, 5, 128, 32, 16, 512, ctypes.byref(n)) == _abi.CF_ERR_INVALID


def test_fp8_entry_points_validate():
    lib = _abi.lib()
    x = _abi.descriptor(torch.zeros(4, 2, 8))
    s = _abi.descriptor(torch.zeros(3))
    x.t.device = s.t.device = _abi.SFA_ROCM
    assert lib.cf_fp8_amax_scale(_abi.ref(x), _abi.ref(s), None) == _abi.CF_ERR_INVALID
    assert "scales has 3 entries" in _abi.last_error()
    o = _abi.descriptor(torch.zeros(4, 2, 8))
    o.t.device = _abi.SFA_ROCM
    s2 = _abi.descriptor(torch.zeros(2))
    s2.t.device = _abi.SFA_ROCM
    assert lib.cf_fp8_quantize(_abi.ref(x), _abi.ref(s2), _abi.ref(o), None) == _abi.CF_ERR_INVALID
    assert "f8e4m3fn" in _abi.last_error()
    # fused K + V: dtype and shape mismatches are refused before any launch
    v = _abi.descriptor(torch.zeros(4, 2, 8, dtype=torch.float16))
    v.t.device = _abi.SFA_ROCM
    assert lib.cf_fp8_quantize_kv(_abi.ref(x), _abi.ref(v), _abi.ref(s2), _abi.ref(s2), _abi.ref(o), _abi.ref(o),
                                  None) == _abi.CF_ERR_INVALID
    assert "differs from k" in _abi.last_error()
    v = _abi.descriptor(torch.zeros(4, 2, 16))
    o8 = _abi.descriptor(torch.zeros(4, 2, 8, dtype=torch.float8_e4m3fn))
    v.t.device = o8.t.device = _abi.SFA_ROCM
    assert lib.cf_fp8_quantize_kv(_abi.ref(x), _abi.ref(v), _abi.ref(s2), _abi.ref(s2), _abi.ref(o8), _abi.ref(o8),
                                  None) == _abi.CF_ERR_INVALID
    assert "v shape differs" in _abi.last_error()
    assert lib.cf_fp8_quantize_kv(_abi.ref(x), _abi.ref(x), _abi.ref(s2), _abi.ref(s2), _abi.ref(o8), _abi.ref(o),
                                  None) == _abi.CF_ERR_INVALID
    assert "f8e4m3fn" in _abi.last_error()


def test_last_error_truncates_safely():
    _call_decode(*_decode_args())
    buf = ctypes.create_string_buffer(8)
    n = _abi.lib().cf_last_error(buf, 8)
    assert n > 8 and len(buf.value) == 7


def test_shared_prefix_statement_is_validated():
    lib = _abi.lib()
    args = list(_decode_args())
    for bad, message in ((torch.zeros(2, dtype=torch.int64), "shared_prefix_lens: expected i32"),
                         (torch.zeros(3, dtype=torch.int32), "shared_prefix_lens has 3 entries")):
        ds = [_abi.descriptor(t) for t in args]
        dsh = _abi.descriptor(bad)
        for d in ds + [dsh]:
            d.t.device = _abi.SFA_ROCM
        rc = lib.cf_paged_decode_shared(*(_abi.ref(d) for d in ds[:5]), _abi.ref(dsh), None, None, 0.125, 16, 512,
                                        _abi.ref(ds[5]), None, 0, None)
        assert rc == _abi.CF_ERR_INVALID and message in _abi.last_error()


def test_prefill_cache_layout_checks():
    """Chunked prefill's layout check, before any HIP call: the reference's
    token-major caches pass it (the call then stops at the missing
    workspace), a view whose token stride would overflow the kernel's 32-bit
    in-block offsets is refused as unsupported, and so is a V tile that is
    neither channel rows of 16 tokens nor token rows."""
    lib = _abi.lib()
    q = torch.zeros(4, 8, 64, dtype=torch.bfloat16)
    cache = torch.zeros(10, 16, 2, 64, dtype=torch.bfloat16)  # [NB, bs, Hkv, D], token-major
    bt = torch.zeros(1, 4, dtype=torch.int32)
    sl = torch.tensor([4], dtype=torch.int32)
    qs = torch.tensor([0, 4], dtype=torch.int32)
    out = torch.zeros(4, 8, 64, dtype=torch.bfloat16)

    def call(k, v):
        ds = [_abi.descriptor(t) for t in (q, k, v, bt, sl, qs, out)]
        for d in ds:
            d.t.device = _abi.SFA_ROCM
        return ds, lambda: lib.cf_prefill_chunk_fp8(*(_abi.ref(d) for d in ds[:6]), None, None, 0.125, 16,
                                                    _abi.ref(ds[6]), None, 0, None)

    ds, run = call(cache, cache)
    assert run() == _abi.CF_ERR_WORKSPACE and "workspace" in _abi.last_error()
    for i in (1, 2):
        ds[i].t.r4.strides[1] = 1 << 28  # 16 rows x 2^28 elements x 2 bytes > 2^32
    assert run() == _abi.CF_ERR_UNSUPPORTED and "token-major" in _abi.last_error()
    # V with channel stride 1 and token stride 1 is no layout the kernel reads
    ds, run = call(cache, cache)
    ds[2].t.r4.strides[1] = 1
    assert run() == _abi.CF_ERR_UNSUPPORTED
