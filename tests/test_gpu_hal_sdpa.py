"""HipBackend's scaled_dot_product_attention (the reference's HAL op,
python_runtime/hal/pytorch_backend/_ops_attention.py:13-53, 3-4 inputs):
decode-shaped calls run on the HIP decode kernels, reading the dense
key/value in place as paged blocks, and match the float64 oracle; other
calls reach the fallback executor unchanged."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import ops
from oracle.paged_attention import paged_attention_fp64
from python_runtime.hal.hip_backend import HipBackend
from python_runtime.hal.interface import OpExecutor
from tests.gpu_util import assert_close

pytestmark = pytest.mark.gpu


class _Recorder(OpExecutor):
    def __init__(self):
        self.calls = []

    def execute(self, op_name, inputs, **kwargs):
        self.calls.append((op_name, len(inputs), sorted(kwargs)))
        return torch.zeros(1)


def _oracle(q, k, v, scale, causal=False):
    """Dense attention through the pinned float64 paged oracle: token s of
    batch row b is block b * S + s of a block_size-1 cache."""
    B, H, _, D = q.shape
    S, Hkv = k.shape[2], k.shape[1]
    kc = k.float().cpu().numpy().transpose(0, 2, 1, 3).reshape(B * S, 1, Hkv, D)
    vc = v.float().cpu().numpy().transpose(0, 2, 1, 3).reshape(B * S, 1, Hkv, D)
    if Hkv == 1 and H > 1:  # torch SDPA broadcasts the single head
        kc = np.repeat(kc, H, axis=2)
        vc = np.repeat(vc, H, axis=2)
    tables = [list(range(b * S, (b + 1) * S)) for b in range(B)]
    lens = [1 if causal else S] * B
    out = paged_attention_fp64(q[:, :, 0].float().cpu().numpy(), kc, vc, tables, lens, 1, scale)
    return out[:, :, None, :]


@pytest.mark.parametrize("dtype,B,H,Hkv,S,D,smax", [
    (torch.bfloat16, 4, 8, 8, 1024, 128, None),   # 16-token blocks
    (torch.bfloat16, 3, 8, 8, 300, 64, None),     # S % 16 != 0: 4-token blocks
    (torch.float16, 2, 16, 1, 777, 64, None),     # one KV head broadcast, odd length: 1-token blocks
    (torch.float32, 5, 4, 4, 96, 80, 160),        # key/value sliced from a longer cache
    (torch.bfloat16, 2, 32, 32, 4096, 128, 8192),
])
def test_sdpa_decode_runs_on_hip(gpu, dtype, B, H, Hkv, S, D, smax):
    print(f"[case] sdpa {dtype} B={B} H={H} Hkv={Hkv} S={S} D={D} smax={smax}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(B * 100 + S)
    q = torch.randn(B, H, 1, D, generator=g, device=gpu).to(dtype)
    full = smax or S
    k = torch.randn(B, Hkv, full, D, generator=g, device=gpu).to(dtype)[:, :, :S]
    v = torch.randn(B, Hkv, full, D, generator=g, device=gpu).to(dtype)[:, :, :S]
    fb = _Recorder()
    be = HipBackend(fallback=fb)
    with ops.KernelTimer() as timer:
        out = be.execute("scaled_dot_product_attention", [q, k, v])
        torch.cuda.synchronize()
        assert timer.query("cf_decode")[1] >= 1
    assert fb.calls == [] and out.shape == (B, H, 1, D) and out.dtype == dtype
    assert_close(out.float().cpu().numpy(), _oracle(q, k, v, 1 / math.sqrt(D)), dtype, f"sdpa {dtype} S={S}")
    # explicit scale, and is_causal with one query token (it sees key 0 only)
    out2 = be.execute("scaled_dot_product_attention", [q, k, v], scale=0.3)
    out3 = be.execute("scaled_dot_product_attention", [q, k, v], is_causal=True)
    torch.cuda.synchronize()
    assert_close(out2.float().cpu().numpy(), _oracle(q, k, v, 0.3), dtype, "sdpa scale 0.3")
    assert_close(out3.float().cpu().numpy(), _oracle(q, k, v, 1 / math.sqrt(D), causal=True), dtype,
                 "sdpa causal")
    assert fb.calls == []


def test_sdpa_other_calls_reach_the_fallback(gpu):
    q = torch.randn(2, 4, 1, 64, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(2, 4, 100, 64, device=gpu, dtype=torch.bfloat16)
    fb = _Recorder()
    be = HipBackend(fallback=fb)
    be.execute("scaled_dot_product_attention", [q, k, k, torch.zeros(2, 1, 1, 100, device=gpu)])
    be.execute("scaled_dot_product_attention", [torch.randn(2, 4, 7, 64, device=gpu, dtype=torch.bfloat16), k, k])
    be.execute("scaled_dot_product_attention", [q, k, k], dropout_p=0.1)
    be.execute("scaled_dot_product_attention", [q, k[:, :2], k[:, :2]])  # 2 KV heads for 4: torch's error case
    be.execute("scaled_dot_product_attention", [q, k.float(), k.float()])  # mixed dtypes
    assert [c[1] for c in fb.calls] == [4, 3, 3, 3, 3]
