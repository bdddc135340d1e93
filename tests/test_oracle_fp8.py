"""Pins the CPU FP8 oracle (oracle/fp8_e4m3.c, oracle/fp8_kv_cache.py).

- exhaustive: the C encoder equals torch's float8_e4m3fn cast (the library
  routine the reference calls at compiler/quantize/fp8_kv_cache.py:89) on
  all 2^32 float32 bit patterns;
- the decode table and hand-derived known answers from the OCP spec
  (tests/golden/fp8_e4m3_vectors.json);
- the scale rule's closed forms (zero block, 1e-12 clamp, amax/448);
- the torch restatement of FP8KVCacheQuantizer agrees with the C oracle
  bit for bit, and passes the reference's own TestFP8KVCache cases
  (tests/test_quantize.py:289-337 of the reference).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8
from oracle.fp8_kv_cache import FP8KVCacheQuantizerRef

GOLDEN = json.loads((Path(__file__).parent / "golden" / "fp8_e4m3_vectors.json").read_text())


def _cos(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().flatten(), b.float().flatten()
    return torch.nn.functional.cosine_similarity(a.unsqueeze(0), b.unsqueeze(0)).item()


def test_exhaustive_encoder_matches_torch_cast():
    chunk = 1 << 26
    bad = 0
    for start in range(0, 1 << 32, chunk):
        mine = fp8.encode_bits(start, chunk)
        bits = torch.arange(start, start + chunk, dtype=torch.int64).to(torch.int32)
        torch_codes = bits.view(torch.float32).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        bad += int(np.count_nonzero(mine != torch_codes))
    assert bad == 0


def test_decode_table_matches_definition_and_torch():
    codes = np.arange(256, dtype=np.uint8)
    mine = fp8.decode(codes)
    torch_vals = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    for row in GOLDEN["decode"]:
        c = row["code"]
        if row["nan"]:
            assert np.isnan(mine[c]) and np.isnan(torch_vals[c])
        else:
            want = np.array([row["f32_bits"]], dtype=np.uint32).view(np.float32)[0]
            assert mine[c].view(np.uint32) == want.view(np.uint32), c
            assert torch_vals[c].view(np.uint32) == want.view(np.uint32), c


def test_known_answers():
    bits = np.array([e["f32_bits"] for e in GOLDEN["encode"]], dtype=np.uint32)
    want = np.array([e["code"] for e in GOLDEN["encode"]], dtype=np.uint8)
    got = fp8.encode(bits.view(np.float32))
    bad = [(e["why"], hex(g)) for e, g, w in zip(GOLDEN["encode"], got, want) if g != w]
    assert not bad


def test_known_answers_catch_a_round_half_up_encoder():
    """A plausible mistake (ties away from zero) must fail the known answers."""
    def half_up(x: np.ndarray) -> np.ndarray:
        vals = fp8.decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
        out = []
        for v in x.astype(np.float64):
            a = abs(v)
            if np.isnan(v) or a >= 480:
                out.append(0x7F | (0x80 if np.signbit(v) else 0))
                continue
            d = np.abs(vals - a)
            best = np.flatnonzero(d == d.min())
            out.append(int(best.max()) | (0x80 if np.signbit(v) else 0))
        return np.array(out, dtype=np.uint8)

    bits = np.array([e["f32_bits"] for e in GOLDEN["encode"]], dtype=np.uint32)
    want = np.array([e["code"] for e in GOLDEN["encode"]], dtype=np.uint8)
    assert np.any(half_up(bits.view(np.float32)) != want)


@pytest.mark.parametrize(
    "amax, want",
    [
        (0.0, 1.0),
        (448.0, 1.0),
        (896.0, 2.0),
        (1e-10, 1e-12),  # 1e-10/448 < 1e-12 -> clamped
        (4.48e-10, np.float32(np.float32(4.48e-10) / np.float32(448.0))),
    ],
)
def test_scale_rule_closed_forms(amax, want):
    x = np.zeros(64, dtype=np.float32)
    x[5] = -amax
    s = fp8.scale_of(x)
    assert s == np.float32(want)


def test_scale_matches_torch_restatement_bitwise():
    q = FP8KVCacheQuantizerRef()
    g = torch.Generator().manual_seed(3)
    for i in range(200):
        x = torch.randn(16, 8, 128, generator=g) * float(10.0 ** torch.randint(-12, 6, (1,), generator=g))
        if i % 7 == 0:
            x[torch.rand(x.shape, generator=g) < 0.01] *= 8
        codes_t, scale_t = q.quantize_block(x)
        codes_o, scale_o = fp8.quantize_block(x.numpy())
        assert np.float32(scale_t.item()).view(np.uint32) == scale_o.view(np.uint32)
        assert np.array_equal(codes_t.view(torch.uint8).numpy(), codes_o)


def test_per_head_restatements_agree():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(40, 8, 128, generator=g) * torch.logspace(-8, 3, 8).view(1, 8, 1)).to(torch.bfloat16)
    x[:, 3] = 0
    ct, st = FP8KVCacheQuantizerRef().quantize_per_head(x)
    co, so = fp8.quantize_per_head(x.float().numpy())
    assert np.array_equal(st.numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(ct.view(torch.uint8).numpy(), co)
    assert st[3].item() == 1.0


def test_dequantize_is_exact_product():
    codes = np.arange(256, dtype=np.uint8)
    s = np.float32(0.0123)
    got = fp8.dequantize(codes, s)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float() * torch.tensor(s)
    assert np.array_equal(np.isnan(got), np.isnan(want.numpy()))
    m = ~np.isnan(got)
    assert np.array_equal(got[m].view(np.uint32), want.numpy()[m].view(np.uint32))


# The reference's TestFP8KVCache cases, run on the restatement.
def test_reference_roundtrip_case():
    torch.manual_seed(42)
    k = torch.randn(16, 8, 128)
    v = torch.randn(16, 8, 128)
    q = FP8KVCacheQuantizerRef(block_size=16)
    kq, ks, vq, vs = q.quantize_kv(k, v)
    kf, vf = q.dequantize_kv(kq, ks, vq, vs)
    assert _cos(k, kf) >= 0.99 and _cos(v, vf) >= 0.99


def test_reference_zero_block_case():
    q = FP8KVCacheQuantizerRef(block_size=16)
    kq, ks = q.quantize_block(torch.zeros(16, 4, 64))
    assert torch.allclose(q.dequantize_block(kq, ks), torch.zeros(16, 4, 64), atol=1e-6)
    assert ks.item() == 1.0


def test_reference_small_scale_case():
    k = torch.randn(4, 2, 32) * 0.02
    q = FP8KVCacheQuantizerRef(block_size=4)
    kq, ks = q.quantize_block(k)
    assert _cos(k, q.dequantize_block(kq, ks)) >= 0.95


def test_reference_hardware_and_block_size_cases():
    q = FP8KVCacheQuantizerRef()
    assert q.check_hardware_support("NVIDIA H100")
    assert q.check_hardware_support("AMD MI300")
    assert not q.check_hardware_support("NVIDIA A100")
    assert not q.check_hardware_support("CPU")
    with pytest.raises(ValueError, match="block_size"):
        FP8KVCacheQuantizerRef(block_size=0)
