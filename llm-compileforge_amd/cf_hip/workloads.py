"""Seeded synthetic decode workloads with the shapes of the benchmark configs.

Each generator returns a DecodeCase holding the logical inputs: queries,
KV sources (fp32 or bf16, before any FP8 quantization), block tables and
sequence lengths.  `materialize` turns a case into device caches in a
chosen physical layout, quantizing with this library's FP8 kernels.

Configs (names used by bench.py and the tests):
  c1_opt125m    B=4,   Hq=Hkv=12, D=64,  fp32 caches, ctx U{128..512},
                pool of 256 blocks, tables = consecutive runs of one seeded
                permutation of the pool (disjoint across sequences).
  c2_tinyllama  B=32,  Hq=32/Hkv=4, D=64, bf16 caches, ctx U{256..2048},
                disjoint random blocks from an 8192-block pool.
  c3_llama3_8b  B=64,  Hq=32/Hkv=8, D=128, e4m3 caches with per-KV-head
                scales, KV sources bf16 N(0,1) with 1% of elements x8,
                ctx U{1024..8192}; sequences 0..B/2-1 share a 1024-token
                (64-block) prefix mapped to the same physical blocks.
  c4_llama3_70b B=128, Hq=64/Hkv=8, D=128, e4m3, ctx = round(lognormal(
                ln 4096, sigma=1)) clipped to [512, 32768].
All use block_size 16 and softmax scale 1/sqrt(D).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import layout as _layout


@dataclass
class DecodeCase:
    name: str
    q: torch.Tensor  # [B, Hq, D]
    k: torch.Tensor  # logical [NB, bs, Hkv, D], source dtype
    v: torch.Tensor
    block_tables: list[list[int]]
    seq_lens: list[int]
    block_size: int
    scale: float
    kv_dtype: torch.dtype  # dtype of the cache the kernel reads
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    @property
    def num_kv_heads(self) -> int:
        return self.k.shape[2]

    @property
    def head_dim(self) -> int:
        return self.q.shape[2]

    def tables_tensor(self, device: torch.device | str) -> torch.Tensor:
        mb = max(1, max(len(t) for t in self.block_tables))
        out = torch.zeros(len(self.block_tables), mb, dtype=torch.int32)
        for i, t in enumerate(self.block_tables):
            if t:
                out[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        return out.to(device)

    def seq_lens_tensor(self, device: torch.device | str) -> torch.Tensor:
        return torch.tensor(self.seq_lens, dtype=torch.int32).to(device)


def _ctx_uniform(gen: torch.Generator, b: int, lo: int, hi: int) -> list[int]:
    return torch.randint(lo, hi + 1, (b,), generator=gen).tolist()


def _randn(shape: tuple[int, ...], dtype: torch.dtype, device: torch.device, seed: int) -> torch.Tensor:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)


def _with_outliers(x: torch.Tensor, seed: int, frac: float = 0.01, mult: float = 8.0) -> torch.Tensor:
    g = torch.Generator(device=x.device)
    g.manual_seed(seed)
    mask = torch.rand(x.shape, generator=g, device=x.device) < frac
    return torch.where(mask, x * mult, x)


def _tables_from_perm(perm: list[int], lens: list[int], bs: int, shared: list[int] | None = None,
                      n_shared_seqs: int = 0) -> list[list[int]]:
    tables = []
    pos = 0
    for i, n in enumerate(lens):
        nblk = (n + bs - 1) // bs
        t: list[int] = []
        if shared and i < n_shared_seqs:
            t = list(shared[:nblk])
        need = nblk - len(t)
        t += perm[pos : pos + need]
        pos += need
        tables.append(t)
    if pos > len(perm):
        raise ValueError("block pool too small for the sampled lengths")
    return tables


def make_case(config: str, device: torch.device | str = "cpu", seed: int = 0, batch: int | None = None) -> DecodeCase:
    """Builds config `config` (see module docstring), optionally with fewer sequences."""
    device = torch.device(device)
    gen = torch.Generator().manual_seed(seed)
    bs = 16
    if config == "c1_opt125m":
        b, hq, hkv, d, nb = batch or 4, 12, 12, 64, 256
        lens = _ctx_uniform(gen, b, 128, 512)
        perm = torch.randperm(nb, generator=gen).tolist()
        tables = _tables_from_perm(perm, lens, bs)
        src_dtype, kv_dtype = torch.float32, torch.float32
        q_dtype = torch.float32
        outliers = False
        meta: dict = {}
    elif config == "c2_tinyllama":
        b, hq, hkv, d, nb = batch or 32, 32, 4, 64, 8192
        lens = _ctx_uniform(gen, b, 256, 2048)
        perm = torch.randperm(nb, generator=gen).tolist()
        tables = _tables_from_perm(perm, lens, bs)
        src_dtype = kv_dtype = q_dtype = torch.bfloat16
        outliers = False
        meta = {}
    elif config == "c3_llama3_8b":
        b, hq, hkv, d = batch or 64, 32, 8, 128
        lens = _ctx_uniform(gen, b, 1024, 8192)
        prefix_blocks = 1024 // bs
        n_shared = b // 2
        need = prefix_blocks + sum((n + bs - 1) // bs for n in lens) - n_shared * prefix_blocks
        nb = max(need, 64 * 512 * b // 64)
        perm = torch.randperm(nb, generator=gen).tolist()
        shared, rest = perm[:prefix_blocks], perm[prefix_blocks:]
        tables = _tables_from_perm(rest, lens, bs, shared, n_shared)
        src_dtype, kv_dtype, q_dtype = torch.bfloat16, torch.float8_e4m3fn, torch.bfloat16
        outliers = True
        meta = {"shared_prefix_blocks": prefix_blocks, "shared_seqs": n_shared}
    elif config == "c4_llama3_70b":
        b, hq, hkv, d = batch or 128, 64, 8, 128
        ln = torch.empty(b).log_normal_(mean=math.log(4096.0), std=1.0, generator=gen)
        lens = [int(min(max(round(x), 512), 32768)) for x in ln.tolist()]
        nb = sum((n + bs - 1) // bs for n in lens) + 64
        perm = torch.randperm(nb, generator=gen).tolist()
        tables = _tables_from_perm(perm, lens, bs)
        src_dtype, kv_dtype, q_dtype = torch.bfloat16, torch.float8_e4m3fn, torch.bfloat16
        outliers = True
        meta = {"lognormal_sigma": 1.0}
    else:
        raise ValueError(f"unknown config {config!r}")

    q = _randn((b, hq, d), q_dtype, device, seed + 1)
    k = _randn((nb, bs, hkv, d), src_dtype, device, seed + 2)
    v = _randn((nb, bs, hkv, d), src_dtype, device, seed + 3)
    if outliers:
        k = _with_outliers(k, seed + 4).to(src_dtype)
        v = _with_outliers(v, seed + 5).to(src_dtype)
    return DecodeCase(config, q, k, v, tables, lens, bs, 1.0 / math.sqrt(d), kv_dtype, meta)


def materialize(case: DecodeCase, layout: str = "native"):
    """Device caches for `case`: (k_cache, v_cache, k_scale, v_scale).

    e4m3 configs quantize the sources with per-KV-head scales (amax over the
    whole pool of that head / 448) using this library's kernels; scales are
    None for unquantized caches.
    """
    from . import ops

    dev = case.k.device
    nb, bs, hkv, d = case.k.shape
    if case.kv_dtype == torch.float8_e4m3fn:
        k_scale = ops.fp8_amax_scale(case.k)
        v_scale = ops.fp8_amax_scale(case.v)
        kc, vc = _layout.alloc_kv_cache(nb, bs, hkv, d, torch.float8_e4m3fn, dev, layout)
        ops.fp8_quantize(case.k, k_scale, out=kc)
        ops.fp8_quantize(case.v, v_scale, out=vc)
        return kc, vc, k_scale, v_scale
    kc, vc = _layout.alloc_kv_cache(nb, bs, hkv, d, case.kv_dtype, dev, layout)
    kc.copy_(case.k)
    vc.copy_(case.v)
    return kc, vc, None, None


def kv_bytes_per_token(case: DecodeCase) -> int:
    esize = torch.tensor([], dtype=case.kv_dtype).element_size()
    return 2 * case.num_kv_heads * case.head_dim * esize


def algorithmic_bytes(case: DecodeCase) -> dict[str, int]:
    """Bytes one decode call must move at minimum.

    unique: every physical (block, token) row read by any sequence counted
    once, plus q, out, block tables, lengths and scales.  logical: the same
    with shared prefix rows counted once per sequence that reads them.
    """
    bs = case.block_size
    per_tok = kv_bytes_per_token(case)
    rows: dict[int, int] = {}
    logical_tokens = 0
    for t, n in zip(case.block_tables, case.seq_lens):
        n = min(n, len(t) * bs)
        logical_tokens += n
        for j in range((n + bs - 1) // bs):
            used = min(bs, n - j * bs)
            rows[t[j]] = max(rows.get(t[j], 0), used)
    unique_tokens = sum(rows.values())
    qo = 2 * case.q.numel() * case.q.element_size()
    tables = sum(len(t) for t in case.block_tables) * 4 + 4 * case.batch
    scales = 2 * 4 * case.num_kv_heads if case.kv_dtype == torch.float8_e4m3fn else 0
    extra = qo + tables + scales
    return {
        "unique": unique_tokens * per_tok + extra,
        "logical": logical_tokens * per_tok + extra,
        "unique_kv": unique_tokens * per_tok,
        "tokens": logical_tokens,
    }
