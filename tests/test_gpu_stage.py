"""cf_stage_from_host: the dict API's upload of host-packed tables by a
kernel on the compute queue."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from cf_hip import _abi, ops

pytestmark = pytest.mark.gpu


def test_upload_from_pinned_memory_is_exact(gpu):
    host = torch.empty(70000, dtype=torch.int32, pin_memory=True)
    host.copy_(torch.from_numpy(np.random.default_rng(1).integers(-2**31, 2**31, 70000, dtype=np.int64)
                                .astype(np.int32)))
    dev = torch.full((70000,), -7, dtype=torch.int32, device=gpu)
    for n in (4, 1000, 69996):  # whole 16-byte words
        assert ops.stage_from_host(host.data_ptr(), dev.data_ptr(), 4 * n, gpu)
        torch.cuda.synchronize()
        assert torch.equal(dev[:n].cpu(), host[:n])
        assert bool((dev[69996:] == -7).all())


def test_upload_refuses_what_it_cannot_read(gpu):
    """Pageable host memory is refused before any launch; so are unaligned
    sizes and pointers, and a destination that is not device memory."""
    pageable = np.zeros(1024, dtype=np.int32)
    dev = torch.zeros(1024, dtype=torch.int32, device=gpu)
    pinned = torch.zeros(1024, dtype=torch.int32, pin_memory=True)
    stream = ctypes.c_void_p(_abi.stream_handle(gpu))
    lib = _abi.lib()
    assert lib.cf_stage_from_host(pageable.ctypes.data, dev.data_ptr(), 4096, stream) == _abi.CF_ERR_INVALID
    assert lib.cf_stage_from_host(pinned.data_ptr(), dev.data_ptr(), 4095, stream) == _abi.CF_ERR_INVALID
    assert lib.cf_stage_from_host(pinned.data_ptr() + 4, dev.data_ptr(), 4096, stream) == _abi.CF_ERR_INVALID
    assert lib.cf_stage_from_host(pinned.data_ptr(), pinned.data_ptr(), 4096, stream) == _abi.CF_ERR_INVALID
    assert not ops.stage_from_host(pageable.ctypes.data, dev.data_ptr(), 4096, gpu)
    # the refusals leave no HIP error behind for the next runtime call
    x = torch.randn(64, device=gpu)
    torch.cuda.synchronize()
    assert torch.isfinite(x).all()
