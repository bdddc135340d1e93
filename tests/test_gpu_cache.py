"""GPU parity of the paged-cache I/O path: cf_paged_write / cf_paged_gather
kernels, the CacheManager and _KVCacheMixin drop-ins, and attention read
straight from CacheManager slabs.

Writes and reads are bit-exact against the CPU oracle (oracle/
cache_manager.py, oracle/fp8.py) and torch's CPU dtype casts (the
reference's slab assignment casts with torch).  Attention is compared with
the float64 oracle at the decode tolerance (max-abs 2e-2 against the
exact value rounded to bf16, cosine >= 0.9999; tests/gpu_util.py).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cf_hip import ops
from gpu_util import assert_close, codes
from oracle import cache_manager as ocm
from oracle import fp8 as ofp8
from oracle.paged_attention import paged_attention_fp64
from python_runtime.engine import CacheManager, _KVCacheMixin

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn
BS = 16


def _bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a tensor (any strides) in logical order."""
    t = t.detach().contiguous().cpu()
    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.view(width).numpy()


def _cache(nb, h, d, dtype, layout, dev, gen):
    """[NB, bs, H, D] cache of random content in a given storage order."""
    if layout == "contig":
        base = torch.randn(nb, BS, h, d, generator=gen)
        perm = (0, 1, 2, 3)
    elif layout == "k_native":
        base = torch.randn(nb, h, BS, d, generator=gen)
        perm = (0, 2, 1, 3)
    else:  # v_native
        base = torch.randn(nb, h, d, BS, generator=gen)
        perm = (0, 3, 1, 2)
    return base.to(dtype).to(dev).permute(*perm)


def _cast_rows(x32: torch.Tensor, dtype: torch.dtype, scale: np.ndarray | None) -> torch.Tensor:
    """Rows [T, H, D] as the slab stores them: torch CPU cast, or e4m3fn
    codes of x / scale[h] (the fp8 oracle)."""
    if dtype == E4M3:
        c = ofp8.encode(x32.numpy() / scale.reshape(1, -1, 1).astype(np.float32))
        return torch.from_numpy(c).view(E4M3)
    return x32.to(dtype)


@pytest.mark.parametrize("cache_dt", [torch.float32, torch.bfloat16, torch.float16, E4M3])
@pytest.mark.parametrize("x_dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["contig", "k_native", "v_native"])
@pytest.mark.parametrize("d", [128, 40])
def test_paged_write_kernel(gpu, cache_dt, x_dt, layout, d):
    print(f"[case] paged_write cache={cache_dt} x={x_dt} layout={layout} D={d}", flush=True)
    gen = torch.Generator().manual_seed(7)
    nb, h, t = 12, 4, 70
    cache = _cache(nb, h, d, cache_dt, layout, gpu, gen)
    before = cache.detach().cpu().clone()
    x = torch.randn(t, h, d, generator=gen).to(x_dt)
    slots = torch.randperm(nb * BS, generator=gen)[:t].to(torch.int64)
    slots[::9] = -1
    slots[5] = nb * BS  # out of range: skipped
    scale = (torch.rand(h, generator=gen) * 0.5 + 0.05).float()
    xd = x.to(gpu)
    if layout == "v_native":  # strided rows: [T, H, D] view of [H, T, D] storage
        xd = x.permute(1, 0, 2).contiguous().to(gpu).permute(1, 0, 2)
    sd = slots.to(torch.int32 if d == 40 else torch.int64).to(gpu)
    ops.paged_write(xd, sd, cache, scale.to(gpu) if cache_dt == E4M3 else None)
    torch.cuda.synchronize()
    want = before.clone()
    rows = _cast_rows(x.float(), cache_dt, scale.numpy())
    for i, s in enumerate(slots.tolist()):
        if 0 <= s < nb * BS:
            want[s // BS, s % BS] = rows[i]
    np.testing.assert_array_equal(_bits(cache), _bits(want))


@pytest.mark.parametrize("cache_dt,out_dt", [
    (torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32),
    (torch.float32, torch.bfloat16), (E4M3, torch.float32), (E4M3, torch.bfloat16),
])
@pytest.mark.parametrize("layout", ["contig", "k_native", "v_native"])
@pytest.mark.parametrize("d", [64, 24])
def test_paged_gather_kernel(gpu, cache_dt, out_dt, layout, d):
    print(f"[case] paged_gather cache={cache_dt} out={out_dt} layout={layout} D={d}", flush=True)
    gen = torch.Generator().manual_seed(11)
    nb, h, r, mb, s_len = 10, 2, 5, 3, 60  # s_len > mb * bs: padding past every table
    cache = _cache(nb, h, d, cache_dt, layout, gpu, gen)
    tables = torch.randint(0, nb, (r, mb), generator=gen, dtype=torch.int32)
    tables[1, 2] = -1
    tables[3, 0] = nb + 4  # outside the cache: zero rows
    scale = (torch.rand(h, generator=gen) + 0.25).float()
    got = ops.paged_gather(cache, tables.to(gpu), s_len, out_dtype=out_dt,
                           scale=scale.to(gpu) if cache_dt == E4M3 else None)
    torch.cuda.synchronize()
    cpu = cache.detach().cpu()
    if cache_dt == E4M3:
        vals = torch.from_numpy(ofp8.decode(codes(cpu)).astype(np.float32) * scale.numpy().reshape(1, 1, -1, 1))
    else:
        vals = cpu.float()
    want = torch.zeros(r, s_len, h, d)
    for ri in range(r):
        for s in range(s_len):
            jb = s // BS
            if jb < mb and 0 <= int(tables[ri, jb]) < nb:
                want[ri, s] = vals[int(tables[ri, jb]), s % BS]
    np.testing.assert_array_equal(_bits(got), _bits(want.to(out_dt)))


def _policy(dtype, layers=3, heads=8, dim=64):
    slab = {"storage": "paged", "dims": {"layers": layers, "heads": heads, "dim": dim}, "dtype": dtype}
    return {
        "slabs": [dict(slab, slab_id="k"), dict(slab, slab_id="v")],
        "intercepts": [
            {"slab_id": "k", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[1]"},
            {"slab_id": "v", "op_name": "scaled_dot_product_attention", "direction": "read_write",
             "source": "operand[2]"},
        ],
        "block_size": BS,
        "max_requests": 8,
    }


def _oracle_slab(mgr, name):
    s = mgr._slabs[name].detach().contiguous().cpu()
    return s.view(torch.uint8).numpy().copy() if s.dtype == E4M3 else s.double().numpy()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16", "float64", "float8_e4m3fn"])
def test_cache_manager_write_read_vs_oracle(gpu, dtype):
    """Several layers, overlapping tables in unsorted dict order, uncovered
    and repeated positions, host and device positions: slab bytes and reads
    equal the oracle's."""
    print(f"[case] CacheManager {dtype}", flush=True)
    gen = torch.Generator().manual_seed(3)
    mgr = CacheManager(_policy(dtype), num_blocks=24, device=gpu)
    fp8 = dtype == "float8_e4m3fn"
    tdt = torch.bfloat16 if fp8 else mgr._slabs["k"].dtype
    scales = {}
    if fp8:
        for name in ("k", "v"):
            sc = (torch.rand(3, 8, generator=gen) * 0.2 + 0.05).float()
            mgr.set_kv_scales(name, sc)
            scales[name] = sc.numpy()
    ref = {name: _oracle_slab(mgr, name) for name in ("k", "v")}
    bt = {"zeta": [4, 9, 2], "alpha": [4, 9, 17, 11, 5], "mid": [20, 21]}
    mgr.begin_step(bt)
    for layer in range(3):
        for name in ("k", "v"):
            pos = [0, 3, 17, 33, 47, 48, 50, 79, 80, 100, 17]  # 80+: uncovered; 17 twice
            data = torch.randn(len(pos), 8, 64, generator=gen).to(tdt)
            mgr.write_paged(name, layer, data, torch.tensor(pos))
            sc = scales[name][layer] if fp8 else None
            ocm.write_paged(ref[name], layer, data.double().numpy(), pos, bt, scale=sc)
            dpos = [1, 2, 34, 64]
            data2 = torch.randn(len(dpos), 8, 64, generator=gen).to(tdt)
            mgr.write_paged(name, layer, data2.to(gpu), torch.tensor(dpos, device=gpu))
            ocm.write_paged(ref[name], layer, data2.double().numpy(), dpos, bt, scale=sc)
    torch.cuda.synchronize()
    for name in ("k", "v"):
        np.testing.assert_array_equal(_oracle_slab(mgr, name), ref[name])
        for layer in range(3):
            for max_len in (1, 35, 90):
                got = mgr.read_paged(name, layer, max_len)
                sc = scales[name][layer] if fp8 else None
                want = ocm.read_paged(ref[name], layer, max_len, bt, scale=sc)
                assert got.dtype == (torch.float32 if fp8 else mgr._slabs[name].dtype)
                np.testing.assert_array_equal(got.double().cpu().numpy(), want)


def test_cache_manager_reference_cases(gpu):
    """The reference's own CacheManager tests (test_cache_manager.py:106-172), on the GPU."""
    mgr = CacheManager(_policy("float32", layers=4), num_blocks=16, device=gpu)
    mgr.begin_step({"r0": [0, 1]})
    k, v = torch.randn(6, 8, 64), torch.randn(6, 8, 64)
    mgr.write_paged("k", 0, k, torch.arange(6))
    mgr.write_paged("v", 0, v, torch.arange(6))
    assert mgr.read_paged("k", 0, 6).shape == (1, 6, 8, 64)
    assert torch.equal(mgr.read_paged("k", 0, 6)[0].cpu(), k)
    assert torch.equal(mgr.read_paged("v", 0, 6)[0].cpu(), v)
    mgr.begin_step({"r0": [0]})
    mgr.write_paged("k", 0, torch.ones(1, 8, 64), torch.tensor([0]))
    mgr.write_paged("k", 1, torch.ones(1, 8, 64) * 2, torch.tensor([0]))
    assert torch.equal(mgr.read_paged("k", 0, 1).cpu(), torch.ones(1, 1, 8, 64))
    assert torch.equal(mgr.read_paged("k", 1, 1).cpu(), torch.ones(1, 1, 8, 64) * 2)
    mgr.begin_step({"r0": [0, 1]})
    kd = torch.randn(32, 8, 64)
    mgr.write_paged("k", 0, kd, torch.arange(32))
    assert torch.equal(mgr.read_paged("k", 0, 32)[0].cpu(), kd)
    mgr.begin_step({"r0": [0, 1], "r1": [2]})
    k0, k1 = torch.randn(16, 8, 64), torch.randn(1, 8, 64)
    mgr.write_paged("k", 0, k0, torch.arange(0, 16))
    mgr.write_paged("k", 0, k1, torch.tensor([16]))
    res = mgr.read_paged("k", 0, 17).cpu()
    assert res.shape[0] == 2 and torch.equal(res[0, :16], k0)
    assert not torch.allclose(res[0, 0], res[1, 0])
    # SDPA operand formats: [1, H, S, D] and [S, H*D]
    mgr.begin_step({"r0": [3]})
    x = torch.randn(1, 8, 5, 64)
    mgr.write_paged("k", 2, x, torch.arange(5))
    assert torch.equal(mgr.read_paged("k", 2, 5)[0].cpu(), x[0].permute(1, 0, 2))
    mgr.write_paged("v", 2, x[0].permute(1, 0, 2).reshape(5, 512), torch.arange(5))
    assert torch.equal(mgr.read_paged("v", 2, 5)[0].cpu(), x[0].permute(1, 0, 2))


class _Exec(_KVCacheMixin):
    def __init__(self):
        self._kv_cache = None
        self._block_tables = {}
        self._block_size = 16
        self._num_kv_heads = 0
        self._head_dim = 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, E4M3])
def test_kv_mixin(gpu, dtype):
    """The reference's mixin tests (test_mlir_executor.py:79-110) plus an
    FP8 cache, against the oracle."""
    print(f"[case] mixin {dtype}", flush=True)
    ex = _Exec()
    kv = ex.prepare_kv_blocks(num_layers=4, num_kv_heads=2, head_dim=4, block_size=4, num_blocks=8, dtype=dtype,
                              device=gpu)
    ex.set_kv_cache(kv, block_tables={"r0": [0, 1]}, num_kv_heads=2, head_dim=4, block_size=4)
    gen = torch.Generator().manual_seed(5)
    k_data, v_data = torch.randn(4, 2, 4, generator=gen), torch.randn(4, 2, 4, generator=gen)
    if dtype == E4M3:
        ex.set_kv_scales(torch.tensor([[0.01, 0.02]]).expand(4, 2, 2) * torch.arange(1, 5).view(4, 1, 1))
    ex.write_kv_to_cache(k_data, v_data, torch.tensor([0, 1, 2, 3]), {"r0": [0, 1]}, layer_idx=0)
    kg, vg = ex.gather_kv_from_cache({"r0": [0, 1]}, max_seq_len=4, layer_idx=0)
    assert kg.shape == (1, 4, 2, 4)
    if dtype == E4M3:
        for src, got, kvi in ((k_data, kg, 0), (v_data, vg, 1)):
            sc = ex._kv_scales[0, kvi].cpu().numpy()
            slab = np.zeros((8, 1, 4, 2, 4), np.uint8)
            ocm.write_paged(slab, 0, src.numpy(), [0, 1, 2, 3], {"r0": [0, 1]}, scale=sc)
            want = ocm.read_paged(slab, 0, 4, {"r0": [0, 1]}, scale=sc)
            np.testing.assert_array_equal(got.double().cpu().numpy(), want)
    else:
        assert torch.equal(kg.cpu(), k_data.to(dtype).unsqueeze(0))
        assert torch.equal(vg.cpu(), v_data.to(dtype).unsqueeze(0))
    ex.set_kv_cache(kv, block_tables={"r0": [0]}, num_kv_heads=2, head_dim=4, block_size=4)
    ones = torch.ones(4, 2, 4)
    ex.write_kv_to_cache(ones, ones * 0, torch.tensor([0, 1, 2, 3]), {"r0": [0]}, layer_idx=0)
    ex.write_kv_to_cache(ones * 2, ones * 0, torch.tensor([0, 1, 2, 3]), {"r0": [0]}, layer_idx=1)
    kg0, _ = ex.gather_kv_from_cache({"r0": [0]}, max_seq_len=4, layer_idx=0)
    kg1, _ = ex.gather_kv_from_cache({"r0": [0]}, max_seq_len=4, layer_idx=1)
    if dtype != E4M3:
        assert torch.equal(kg0.cpu().float(), torch.ones(1, 4, 2, 4))
        assert torch.equal(kg1.cpu().float(), torch.ones(1, 4, 2, 4) * 2)


@pytest.mark.parametrize("dtype", ["bfloat16", "float8_e4m3fn"])
def test_cache_manager_attend(gpu, dtype):
    """Decode attention straight from CacheManager slabs (native layouts,
    shared-prefix tables, per-layer FP8 scales) vs the float64 oracle over
    the slab contents."""
    print(f"[case] attend {dtype}", flush=True)
    gen = torch.Generator().manual_seed(9)
    L, hq, hkv, d = 2, 32, 8, 128
    mgr = CacheManager(_policy(dtype, layers=L, heads=hkv, dim=d), num_blocks=96, device=gpu)
    prefix = [0, 1, 2, 3]
    bt = {"r3": prefix + [10, 11, 12], "r1": prefix + [20, 21], "r2": [30, 31, 32, 33, 34, 35, 36, 37],
          "r0": prefix[:2] + [40]}
    fp8 = dtype == "float8_e4m3fn"
    rows = {}
    for layer in range(L):
        for name in ("k", "v"):
            rows[layer, name] = (torch.randn(16 * 8, hkv, d, generator=gen) * (1 + layer)).to(torch.bfloat16)
            if fp8:
                mgr.calibrate_kv_scales(name, layer, rows[layer, name].to(gpu))
    for key in bt:  # one request per step, as a prefill writes it; shared blocks get the same rows
        mgr.begin_step({key: bt[key]})
        ln = len(bt[key]) * 16
        for layer in range(L):
            for name in ("k", "v"):
                mgr.write_paged(name, layer, rows[layer, name][:ln], torch.arange(ln))
    mgr.begin_step(bt)
    ids = sorted(bt)
    lens = [len(bt[k]) * 16 - 5 for k in ids]
    q = torch.randn(len(ids), hq, d, generator=gen).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    for layer in range(L):
        got = mgr.attend(q.to(gpu), layer, seq_lens=lens)
        torch.cuda.synchronize()
        kc = mgr.layer_view("k", layer).detach().cpu()
        vc = mgr.layer_view("v", layer).detach().cpu()
        tables = [list(bt[k]) for k in ids]
        if fp8:
            kf = ofp8.decode(codes(kc))
            vf = ofp8.decode(codes(vc))
            ks, vs = mgr.kv_scales("k")[layer].cpu().numpy(), mgr.kv_scales("v")[layer].cpu().numpy()
        else:
            kf, vf, ks, vs = kc.float().numpy(), vc.float().numpy(), None, None
        want = paged_attention_fp64(q.float().numpy(), kf, vf, tables, lens, 16, scale, ks, vs)
        assert_close(got.float().cpu().numpy(), want, torch.bfloat16, f"attend {dtype} layer {layer}")
        full = mgr.attend(q.to(gpu), layer)  # every table full
        want_full = paged_attention_fp64(q.float().numpy(), kf, vf, tables, [len(t) * 16 for t in tables], 16,
                                         scale, ks, vs)
        assert_close(full.float().cpu().numpy(), want_full, torch.bfloat16, f"attend {dtype} full {layer}")


def test_cache_manager_from_fp8_policy_blob(gpu):
    """An FP8 policy blob with stored scales drives the writes: slab codes and
    reads equal the oracle's with those scales."""
    from compiler.cache_policy import CachePolicy, serialize_cache_policy

    policy = CachePolicy.for_llama(2, 4, 32, kv_dtype="float8_e4m3fn")
    gen = torch.Generator().manual_seed(21)
    sc = {n: (torch.rand(2, 4, generator=gen) * 0.1 + 0.01) for n in ("k", "v")}
    for n in ("k", "v"):
        policy.set_kv_scales(n, sc[n])
    mgr = CacheManager(serialize_cache_policy(policy), num_blocks=6, device=gpu)
    bt = {"b": [5, 0], "a": [3]}
    mgr.begin_step(bt)
    ref = {n: np.zeros((6, 2, 16, 4, 32), np.uint8) for n in ("k", "v")}
    for layer in range(2):
        for n in ("k", "v"):
            x = torch.randn(32, 4, 32, generator=gen).to(torch.bfloat16)
            mgr.write_paged(n, layer, x, torch.arange(32))
            s32 = mgr.kv_scales(n)[layer].cpu().numpy()
            ocm.write_paged(ref[n], layer, x.double().numpy(), list(range(32)), bt, scale=s32)
    torch.cuda.synchronize()
    for n in ("k", "v"):
        np.testing.assert_array_equal(_oracle_slab(mgr, n), ref[n])
        for layer in range(2):
            s32 = mgr.kv_scales(n)[layer].cpu().numpy()
            np.testing.assert_array_equal(s32, sc[n][layer].numpy().astype(np.float32))
            got = mgr.read_paged(n, layer, 40).double().cpu().numpy()
            np.testing.assert_array_equal(got, ocm.read_paged(ref[n], layer, 40, bt, scale=s32))


def test_hal_cache_ops(gpu):
    """HipBackend cache_write / cache_read equal the row I/O entry points."""
    from python_runtime.hal.hip_backend import HipBackend
    from cf_hip.layout import alloc_kv_cache

    gen = torch.Generator().manual_seed(13)
    be = HipBackend()
    kc, vc = alloc_kv_cache(6, 16, 2, 64, E4M3, gpu, "native")
    kc2, vc2 = alloc_kv_cache(6, 16, 2, 64, E4M3, gpu, "native")
    for c in (kc, vc, kc2, vc2):  # unwritten slots must agree too
        c.view(torch.uint8).zero_()
    ks = (torch.rand(2, generator=gen) + 0.1).to(gpu)
    vs = (torch.rand(2, generator=gen) + 0.1).to(gpu)
    k = torch.randn(20, 2, 64, generator=gen).to(torch.bfloat16).to(gpu)
    v = torch.randn(20, 2, 64, generator=gen).to(torch.bfloat16).to(gpu)
    slots = torch.randperm(96, generator=gen)[:20].to(gpu)
    assert be.execute("cache_write", [k, v, slots, kc, vc], k_scale=ks, v_scale=vs) is kc
    ops.paged_write(k, slots, kc2, ks)
    ops.paged_write(v, slots, vc2, vs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(codes(kc), codes(kc2))
    np.testing.assert_array_equal(codes(vc), codes(vc2))
    table = torch.tensor([[3, 1], [5, -1]], dtype=torch.int32, device=gpu)
    out = be.execute("cache_read", [kc, vc, table], k_scale=ks, v_scale=vs, seq_len=20)
    assert out.shape == (2, 2, 20, 2, 64) and out.dtype == torch.float32
    assert torch.equal(out[0], ops.paged_gather(kc, table, 20, scale=ks))
    assert torch.equal(out[1], ops.paged_gather(vc, table, 20, scale=vs))
