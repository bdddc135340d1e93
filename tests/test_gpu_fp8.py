"""GPU FP8 quantization: codes and scales bit-identical to the CPU oracle.

Covers the device e4m3fn encoder on all 2^32 float32 bit patterns, per-head
and per-block scales (outliers, all-zero heads, the 1e-12 clamp, bf16/fp16/
fp32 inputs), exact dequantization, the paged KV write (int32/int64 slots,
skipped slots, both layouts) and the reference's TestFP8KVCache cases
(tests/test_quantize.py:289-337 of the reference) on the device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cf_hip import layout as L
from cf_hip import ops
from kernels.quantize import FP8KVCacheQuantizer
from oracle import fp8 as ofp8
from tests.gpu_util import codes

pytestmark = pytest.mark.gpu


def test_device_encoder_exhaustive(gpu):
    one = torch.ones(1, dtype=torch.float32, device=gpu)  # x / 1.0 == x exactly
    chunk = 1 << 28
    bad = 0
    for start in range(0, 1 << 32, chunk):
        bits = torch.arange(start, start + chunk, dtype=torch.int64, device=gpu).to(torch.int32)
        got = ops.fp8_quantize(bits.view(torch.float32).view(1, 1, -1), one).view(torch.uint8).view(-1).cpu().numpy()
        want = ofp8.encode_bits(start, chunk)
        bad += int(np.count_nonzero(got != want))
        del bits
    print(f"[fp8] exhaustive mismatches: {bad}", flush=True)
    assert bad == 0


def test_quantize_with_a_scale_exhaustive(gpu):
    """All 2^32 float32 patterns divided by a scale that is not a power of
    two (x * (1/s) and x / s then differ in the last bit for many inputs):
    the device codes equal the oracle's IEEE division then RNE encode."""
    s = 0.0671234
    sc = torch.full((1,), s, dtype=torch.float32, device=gpu)
    chunk = 1 << 28
    bad = 0
    for start in range(0, 1 << 32, chunk):
        bits = torch.arange(start, start + chunk, dtype=torch.int64, device=gpu).to(torch.int32)
        got = ops.fp8_quantize(bits.view(torch.float32).view(1, 1, -1), sc).view(torch.uint8).view(-1).cpu().numpy()
        x = np.arange(start, start + chunk, dtype=np.uint32).view(np.float32)
        bad += int(np.count_nonzero(got != ofp8.quantize(x, s)))
        del bits, x
    print(f"[fp8] exhaustive mismatches with scale {s}: {bad}", flush=True)
    assert bad == 0


@pytest.mark.parametrize("seed", range(4))
def test_quantize_near_midpoints_many_scales(gpu, seed):
    """Inputs within 24 ulp of x = M * s for every midpoint M between adjacent
    e4m3 codes (subnormal codes, normal codes, and 464 between 448 and the
    NaN code), both signs, at 64 random scales: the inputs where x * (1/s)
    and x / s may encode differently, which the encoder resolves without a
    division in the normal range."""
    rng = np.random.default_rng(100 + seed)
    vals = ofp8.decode(np.arange(0x00, 0x7F, dtype=np.uint8)).astype(np.float64)  # 0 .. 448
    mids = np.concatenate([(vals[:-1] + vals[1:]) / 2, [464.0]])
    ks = np.arange(-24, 25, dtype=np.int64)
    for s in (rng.uniform(0.5, 2.0, 64) * 2.0 ** rng.integers(-40, 40, 64)).astype(np.float32):
        x0 = (mids * np.float64(s)).astype(np.float32)
        bits = x0.view(np.uint32).astype(np.int64)[:, None] + ks[None, :]
        x = bits.astype(np.uint32).view(np.float32).reshape(-1)
        x = np.concatenate([x, -x])
        got = ops.fp8_quantize(torch.from_numpy(x).to(gpu).view(1, 1, -1),
                               torch.full((1,), float(s), dtype=torch.float32, device=gpu))
        got = got.view(torch.uint8).view(-1).cpu().numpy()
        want = ofp8.quantize(x, s)
        assert np.array_equal(got, want), (float(s), int(np.count_nonzero(got != want)))


@pytest.mark.parametrize("s", [3.0, 1.0 / 3.0, 1.234e-5, 7.77e3, 1e-12, 1e-39, 3e38])
def test_quantize_scales_on_random_patterns(gpu, s):
    """2^26 random float32 patterns (every exponent, NaN and inf included)
    per scale, including scales whose reciprocal is not normal."""
    g = torch.Generator(device=gpu).manual_seed(int(s * 1000) % 997)
    bits = torch.randint(-(2**31), 2**31, (1 << 26,), generator=g, device=gpu, dtype=torch.int64).to(torch.int32)
    x = bits.view(torch.float32)
    sc = torch.full((1,), s, dtype=torch.float32, device=gpu)
    got = ops.fp8_quantize(x.view(1, 1, -1), sc).view(torch.uint8).view(-1).cpu().numpy()
    want = ofp8.quantize(x.cpu().numpy(), np.float32(s))
    assert np.array_equal(got, want), int(np.count_nonzero(got != want))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_per_head_quantize_bit_exact(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(1)
    x = torch.randn(3000, 8, 128, generator=g, device=gpu)
    x = torch.where(torch.rand(x.shape, generator=g, device=gpu) < 0.01, x * 8, x)
    x = x * torch.logspace(-14, 4, 8, device=gpu).view(1, 8, 1)
    x[:, 5] = 0.0
    x[7, 6, 3] = -0.0
    x = x.to(dtype)
    scales = ops.fp8_amax_scale(x)
    q = ops.fp8_quantize(x, scales)
    torch.cuda.synchronize()
    want_codes, want_scales = ofp8.quantize_per_head(x.float().cpu().numpy())
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), want_scales.view(np.uint32))
    assert np.array_equal(codes(q), want_codes)
    assert scales[5].item() == 1.0


@pytest.mark.parametrize("layout", ["paired", "native", "token_major"])
@pytest.mark.parametrize("nb,bs,h,d,dtype", [(37, 16, 8, 128, torch.bfloat16), (5, 16, 4, 64, torch.float16),
                                             (9, 8, 2, 32, torch.float32), (3, 16, 1, 128, torch.bfloat16)])
def test_quantize_into_cache_layouts_bit_exact(gpu, layout, nb, bs, h, d, dtype):
    """A pool quantized straight into each cache layout's K and V views
    (token-major, tile-ordered and transposed writes) holds the oracle's
    codes at every logical position."""
    g = torch.Generator(device=gpu).manual_seed(nb * 1000 + d)
    for is_v in (False, True):
        x = (torch.randn(nb, bs, h, d, generator=g, device=gpu) * torch.logspace(-3, 2, h, device=gpu).view(1, 1, h, 1))
        x = x.to(dtype)
        scales = ops.fp8_amax_scale(x)
        kc, vc = L.alloc_kv_cache(nb, bs, h, d, torch.float8_e4m3fn, gpu, layout)
        dst = vc if is_v else kc
        dst.view(torch.uint8).fill_(0xAA)
        ops.fp8_quantize(x, scales, out=dst)
        torch.cuda.synchronize()
        want, _ = ofp8.quantize_per_head(x.float().cpu().numpy().reshape(-1, h, d))
        assert np.array_equal(codes(dst.contiguous()).reshape(-1, h, d), want), (layout, is_v)


@pytest.mark.parametrize("layout", ["paired", "native", "token_major"])
@pytest.mark.parametrize("nb,h,d,dtype", [(41, 8, 128, torch.bfloat16), (7, 4, 64, torch.float16),
                                          (5, 2, 80, torch.float32), (3, 1, 128, torch.bfloat16),
                                          (2, 16, 32, torch.bfloat16)])
def test_quantize_kv_into_cache_layouts_bit_exact(gpu, layout, nb, h, d, dtype):
    """fp8_quantize_kv (one launch on native / paired tiles, two otherwise)
    writes, for K and V with their own per-head scales, the oracle's codes at
    every logical position -- the same codes as fp8_quantize on each."""
    g = torch.Generator(device=gpu).manual_seed(nb * 7 + d)
    mag = torch.logspace(-4, 3, h, device=gpu).view(1, 1, h, 1)
    k = (torch.randn(nb, 16, h, d, generator=g, device=gpu) * mag).to(dtype)
    v = (torch.randn(nb, 16, h, d, generator=g, device=gpu) * mag.flip(2)).to(dtype)
    v[:, :, 0] = 0.0  # an all-zero head: scale 1.0
    ks, vs = ops.fp8_amax_scale(k), ops.fp8_amax_scale(v)
    kc, vc = L.alloc_kv_cache(nb, 16, h, d, torch.float8_e4m3fn, gpu, layout)
    kc.view(torch.uint8).fill_(0x55)
    vc.view(torch.uint8).fill_(0x55)
    ops.fp8_quantize_kv(k, v, ks, vs, kc, vc)
    torch.cuda.synchronize()
    for x, sc, out in ((k, ks, kc), (v, vs, vc)):
        want, want_s = ofp8.quantize_per_head(x.float().cpu().numpy().reshape(-1, h, d))
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
        assert np.array_equal(codes(out).reshape(-1, h, d), want), layout
        assert torch.equal(out.contiguous().view(torch.uint8), ops.fp8_quantize(x, sc).view(torch.uint8))


def test_quantize_kv_strided_inputs_and_extreme_scales(gpu):
    """Inputs that are views with gaps between rows, and scales at the edges
    of the fp32 range (reciprocals that are not normal take the division),
    give the per-tensor codes; a block size other than 16 takes two launches."""
    g = torch.Generator(device=gpu).manual_seed(3)
    big = torch.randn(6, 16, 4, 160, generator=g, device=gpu).to(torch.bfloat16)
    k, v = big[..., :128], big[..., 32:]          # rows 320 bytes apart, V at a 64-byte offset
    kc, vc = L.alloc_kv_cache(6, 16, 4, 128, torch.float8_e4m3fn, gpu, "paired")
    for ks in (torch.tensor([1e-12, 3e38, 1.0, 2.0 ** -126], device=gpu),
               torch.tensor([0.75, 1e-30, 448.0, 5e-39], device=gpu)):
        vs = ks.flip(0).contiguous()
        ops.fp8_quantize_kv(k, v, ks, vs, kc, vc)
        torch.cuda.synchronize()
        assert torch.equal(kc.contiguous().view(torch.uint8), ops.fp8_quantize(k, ks).view(torch.uint8))
        assert torch.equal(vc.contiguous().view(torch.uint8), ops.fp8_quantize(v, vs).view(torch.uint8))
        # the oracle with the scales given
        want = np.stack([ofp8.quantize(k[:, :, i].float().cpu().numpy(), np.float32(ks[i].item()))
                         for i in range(4)], axis=2).reshape(-1, 4, 128)
        assert np.array_equal(codes(kc).reshape(-1, 4, 128), want)
    # the one-launch shape with the same extreme scales
    k2, v2 = k.contiguous(), v.contiguous()
    ks = torch.tensor([1e-12, 3e38, 1.0, 2.0 ** -126], device=gpu)
    ops.fp8_quantize_kv(k2, v2, ks, ks, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(kc.contiguous().view(torch.uint8), ops.fp8_quantize(k2, ks).view(torch.uint8))
    assert torch.equal(vc.contiguous().view(torch.uint8), ops.fp8_quantize(v2, ks).view(torch.uint8))
    k8, v8 = k2.reshape(12, 8, 4, 128), v2.reshape(12, 8, 4, 128)
    kc8, vc8 = L.alloc_kv_cache(12, 8, 4, 128, torch.float8_e4m3fn, gpu, "paired")
    ops.fp8_quantize_kv(k8, v8, ks, ks, kc8, vc8)
    torch.cuda.synchronize()
    assert torch.equal(kc8.contiguous().view(torch.uint8), ops.fp8_quantize(k8, ks).view(torch.uint8))
    assert torch.equal(vc8.contiguous().view(torch.uint8), ops.fp8_quantize(v8, ks).view(torch.uint8))


def test_quantize_block_and_dequantize_bit_exact(gpu):
    quant = FP8KVCacheQuantizer(block_size=16)
    g = torch.Generator(device=gpu).manual_seed(2)
    for i in range(20):
        x = torch.randn(16, 8, 128, generator=g, device=gpu) * 10.0 ** (i - 12)
        q, s = quant.quantize_block(x)
        wc, ws = ofp8.quantize_block(x.cpu().numpy())
        assert s.dim() == 0 and s.dtype == torch.float32
        assert np.float32(s.item()).view(np.uint32) == ws.view(np.uint32)
        assert np.array_equal(codes(q), wc)
        deq = quant.dequantize_block(q, s)
        assert np.array_equal(deq.cpu().numpy().view(np.uint32), ofp8.dequantize(wc, ws).view(np.uint32))


def test_reference_fp8_cases_on_device(gpu):
    quant = FP8KVCacheQuantizer(block_size=16)
    torch.manual_seed(42)
    k = torch.randn(16, 8, 128).to(gpu)
    v = torch.randn(16, 8, 128).to(gpu)
    kq, ks, vq, vs = quant.quantize_kv(k, v)
    kf, vf = quant.dequantize_kv(kq, ks, vq, vs)
    cos = torch.nn.functional.cosine_similarity
    assert cos(k.flatten()[None], kf.flatten()[None]).item() >= 0.99
    assert cos(v.flatten()[None], vf.flatten()[None]).item() >= 0.99
    z = torch.zeros(16, 4, 64, device=gpu)
    zq, zs = quant.quantize_block(z)
    assert torch.allclose(quant.dequantize_block(zq, zs), z, atol=1e-6) and zs.item() == 1.0
    small = torch.randn(4, 2, 32, device=gpu) * 0.02
    sq, ss = FP8KVCacheQuantizer(block_size=4).quantize_block(small)
    assert cos(small.flatten()[None], quant.dequantize_block(sq, ss).flatten()[None]).item() >= 0.95
    assert quant.check_hardware_support("AMD MI300") and quant.check_hardware_support("AMD Instinct MI355X")
    assert not quant.check_hardware_support("NVIDIA A100") and not quant.check_hardware_support("CPU")


@pytest.mark.parametrize("layout", ["paired", "native", "token_major"])
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_kv_write_bit_exact(gpu, layout, slot_dtype):
    nb, bs, h, d, t = 40, 16, 8, 128, 300
    g = torch.Generator(device=gpu).manual_seed(3)
    kc, vc = L.alloc_kv_cache(nb, bs, h, d, torch.float8_e4m3fn, gpu, layout)
    kc.view(torch.uint8).fill_(0xAA)
    vc.view(torch.uint8).fill_(0xAA)
    k_new = torch.randn(t, h, d, generator=g, device=gpu).to(torch.bfloat16)
    v_new = torch.randn(t, h, d, generator=g, device=gpu).to(torch.bfloat16)
    ks = ops.fp8_amax_scale(k_new)
    vs = ops.fp8_amax_scale(v_new)
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(4))[:t]
    slots[::37] = -1
    FP8KVCacheQuantizer.write_kv_fp8(k_new, v_new, slots.to(gpu, slot_dtype), kc, vc, ks, vs)
    torch.cuda.synchronize()
    kcodes, vcodes = codes(kc), codes(vc)
    wk = ofp8.quantize_per_head(k_new.float().cpu().numpy())[0]
    wv = ofp8.quantize_per_head(v_new.float().cpu().numpy())[0]
    written = np.zeros((nb, bs), dtype=bool)
    for i, s in enumerate(slots.tolist()):
        if s < 0:
            continue
        written[s // bs, s % bs] = True
        assert np.array_equal(kcodes[s // bs, s % bs], wk[i])
        assert np.array_equal(vcodes[s // bs, s % bs], wv[i])
    assert np.all(kcodes[~written] == 0xAA) and np.all(vcodes[~written] == 0xAA)


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("h,d", [(8, 128), (3, 64)])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_kv_write_runs_bit_exact(gpu, slot_dtype, h, d, x_dtype):
    """Slot patterns of a mixed step on the native layout: chunks starting
    mid-block (runs crossing the kernel's 16-row groups), whole blocks,
    partial last blocks, single decode tokens (a whole 16-row group of
    them), invalid slots inside a run and past the cache's end, and
    consecutive slots crossing a block boundary."""
    nb, bs = 64, 16
    gen = torch.Generator().manual_seed(5)
    slots: list[int] = []
    slots += list(range(5 * bs + 7, 5 * bs + 7 + 45))  # chunk from mid-block 5 into blocks 6, 7, 8
    slots += list(range(20 * bs, 20 * bs + 32))  # two whole blocks
    slots += [33 * bs + 3, 40 * bs + 15, 41 * bs]  # decode tokens; 40:15 -> 41:0 crosses a block
    slots += list(range(50 * bs + 2, 50 * bs + 13))  # partial run
    slots += [-1, 52 * bs + 1, 52 * bs + 2, -1, 52 * bs + 4]  # holes
    slots += list(range(60 * bs, 60 * bs + 16))  # one more whole block, unaligned to the row groups
    lone = [9, 11, 13, 15, 17, 19, 22, 24, 26, 28, 30, 34, 36, 38, 42, 44, 46, 48, 54, 56]
    slots += [b * bs + i for i, b in enumerate(lone)]  # decode tokens only, 20 blocks no other row uses
    slots += [nb * bs - 3, nb * bs - 2, nb * bs - 1, nb * bs, nb * bs + 1, nb * bs + 40]  # the cache's end
    inside = [x for x in slots if 0 <= x < nb * bs]
    assert len(set(inside)) == len(inside)  # distinct slots: rows repeating a slot race
    t = len(slots)
    kc, vc = L.alloc_kv_cache(nb, bs, h, d, torch.float8_e4m3fn, gpu, "native")
    kc.view(torch.uint8).fill_(0xAA)
    vc.view(torch.uint8).fill_(0xAA)
    k_new = torch.randn(t, h, d, generator=gen).to(x_dtype).to(gpu)
    v_new = torch.randn(t, h, d, generator=gen).to(x_dtype).to(gpu)
    ks = ops.fp8_amax_scale(k_new)
    vs = ops.fp8_amax_scale(v_new)
    FP8KVCacheQuantizer.write_kv_fp8(k_new, v_new, torch.tensor(slots, dtype=slot_dtype, device=gpu), kc, vc, ks, vs)
    torch.cuda.synchronize()
    kcodes, vcodes = codes(kc), codes(vc)
    wk = ofp8.quantize_per_head(k_new.float().cpu().numpy())[0]
    wv = ofp8.quantize_per_head(v_new.float().cpu().numpy())[0]
    written = np.zeros((nb, bs), dtype=bool)
    for i, s in enumerate(slots):
        if s < 0 or s >= nb * bs:
            continue
        written[s // bs, s % bs] = True
        assert np.array_equal(kcodes[s // bs, s % bs], wk[i]), (i, s)
        assert np.array_equal(vcodes[s // bs, s % bs], wv[i]), (i, s)
    assert np.all(kcodes[~written] == 0xAA) and np.all(vcodes[~written] == 0xAA)
