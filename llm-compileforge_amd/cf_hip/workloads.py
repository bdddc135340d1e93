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

  c5_mixed      one mixed chunked-prefill + decode step at the c3 shape
                (Hq=32/Hkv=8, D=128, e4m3): 8 chunks of 512 new tokens with
                a cached prefix of U{0..4096} tokens, plus 248 decodes with
                ctx U{512..8192}.  The 8*512 + 248 new K/V rows (bf16
                N(0,1)) are written into the cache in the step, quantized
                with per-KV-head scales calibrated over the pool and the new
                rows (amax/448); then decode and prefill attention read the
                FP8 cache.  Built by make_mixed_case.
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
    if device.type == "meta":  # shapes only (tables, lengths and slots are still sampled)
        return torch.empty(shape, dtype=dtype, device=device)
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


def materialize(case: DecodeCase, layout: str = "paired"):
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
        ops.fp8_quantize_kv(case.k, case.v, k_scale, v_scale, kc, vc)
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


@dataclass
class MixedCase:
    """One chunked-prefill + decode step (see c5_mixed)."""

    name: str
    k_pool: torch.Tensor  # logical [NB, bs, Hkv, D] cache contents before the step (source dtype)
    v_pool: torch.Tensor
    k_new: torch.Tensor  # [T_new, Hkv, D]: chunk rows in q order, then one row per decode
    v_new: torch.Tensor
    slots: list[int]  # cache slot (block * bs + offset) of each new row
    q_prefill: torch.Tensor  # [Tq, Hq, D]
    q_decode: torch.Tensor  # [Bd, Hq, D]
    prefill_tables: list[list[int]]
    prefill_lens: list[int]  # cached + chunk tokens
    q_start: list[int]  # [N + 1]
    decode_tables: list[list[int]]
    decode_lens: list[int]
    block_size: int
    scale: float
    kv_dtype: torch.dtype
    meta: dict = field(default_factory=dict)

    @property
    def num_kv_heads(self) -> int:
        return self.k_pool.shape[2]


def make_mixed_case(
    config: str = "c5_mixed",
    device: torch.device | str = "cpu",
    seed: int = 0,
    *,
    chunks: list[int] | None = None,
    cached: list[int] | None = None,
    decode_lens: list[int] | None = None,
    num_q_heads: int = 32,
    num_kv_heads: int = 8,
    head_dim: int = 128,
    kv_dtype: torch.dtype = torch.float8_e4m3fn,
) -> MixedCase:
    """Builds c5_mixed, or the same step with other chunk lengths, cached
    prefixes, decode lengths or head shape (explicit lists override the
    sampled ones)."""
    if config != "c5_mixed":
        raise ValueError(f"unknown mixed config {config!r}")
    device = torch.device(device)
    gen = torch.Generator().manual_seed(seed)
    bs = 16
    if chunks is None:
        chunks = [512] * 8
    if cached is None:
        cached = _ctx_uniform(gen, len(chunks), 0, 4096)
    if decode_lens is None:
        decode_lens = _ctx_uniform(gen, 248, 512, 8192)
    if len(cached) != len(chunks):
        raise ValueError("chunks and cached must have the same length")
    prefill_lens = [c + n for c, n in zip(cached, chunks)]
    lens = prefill_lens + list(decode_lens)
    nb = sum((n + bs - 1) // bs for n in lens) + 16
    perm = torch.randperm(nb, generator=gen).tolist()
    tables = _tables_from_perm(perm, lens, bs)
    ptables, dtables = tables[: len(chunks)], tables[len(chunks):]
    slots: list[int] = []
    for t, c, n in zip(ptables, cached, chunks):
        slots += [t[p // bs] * bs + p % bs for p in range(c, c + n)]
    for t, n in zip(dtables, decode_lens):
        slots.append(t[(n - 1) // bs] * bs + (n - 1) % bs)
    q_start = [0]
    for n in chunks:
        q_start.append(q_start[-1] + n)
    hq, hkv, d = num_q_heads, num_kv_heads, head_dim
    src = torch.bfloat16
    k_pool = _randn((nb, bs, hkv, d), src, device, seed + 2)
    v_pool = _randn((nb, bs, hkv, d), src, device, seed + 3)
    k_new = _randn((len(slots), hkv, d), src, device, seed + 4)
    v_new = _randn((len(slots), hkv, d), src, device, seed + 5)
    q_prefill = _randn((q_start[-1], hq, d), torch.bfloat16, device, seed + 6)
    q_decode = _randn((len(decode_lens), hq, d), torch.bfloat16, device, seed + 7)
    return MixedCase(config, k_pool, v_pool, k_new, v_new, slots, q_prefill, q_decode, ptables, prefill_lens,
                     q_start, dtables, list(decode_lens), bs, 1.0 / math.sqrt(d), kv_dtype,
                     {"cached": list(cached), "chunks": list(chunks)})


def _int_tensor(rows: list[list[int]], device) -> torch.Tensor:
    mb = max([1] + [len(t) for t in rows])
    out = torch.zeros(len(rows), mb, dtype=torch.int32)
    for i, t in enumerate(rows):
        if t:
            out[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
    return out.to(device)


def materialize_mixed(case: MixedCase, layout: str = "paired") -> dict[str, torch.Tensor | None]:
    """Device tensors of the step: the cache before the step (e4m3 with
    scales calibrated over pool and new rows, or bf16) and every input of
    the write, decode and prefill calls."""
    from . import ops

    dev = case.k_pool.device
    nb, bs, hkv, d = case.k_pool.shape
    t: dict[str, torch.Tensor | None] = {}
    if case.kv_dtype == torch.float8_e4m3fn:
        ks = torch.maximum(ops.fp8_amax_scale(case.k_pool), ops.fp8_amax_scale(case.k_new))
        vs = torch.maximum(ops.fp8_amax_scale(case.v_pool), ops.fp8_amax_scale(case.v_new))
        kc, vc = _layout.alloc_kv_cache(nb, bs, hkv, d, torch.float8_e4m3fn, dev, layout)
        ops.fp8_quantize_kv(case.k_pool, case.v_pool, ks, vs, kc, vc)
        t.update(k_scale=ks, v_scale=vs)
    else:
        kc, vc = _layout.alloc_kv_cache(nb, bs, hkv, d, case.kv_dtype, dev, layout)
        kc.copy_(case.k_pool)
        vc.copy_(case.v_pool)
        t.update(k_scale=None, v_scale=None)
    t.update(
        k_cache=kc, v_cache=vc,
        k_new=case.k_new, v_new=case.v_new,
        slots=torch.tensor(case.slots, dtype=torch.int64).to(dev),
        q_prefill=case.q_prefill, q_decode=case.q_decode,
        prefill_tables=_int_tensor(case.prefill_tables, dev),
        prefill_lens=torch.tensor(case.prefill_lens, dtype=torch.int32).to(dev),
        q_start=torch.tensor(case.q_start, dtype=torch.int32).to(dev),
        decode_tables=_int_tensor(case.decode_tables, dev),
        decode_lens=torch.tensor(case.decode_lens, dtype=torch.int32).to(dev),
    )
    return t


def mixed_algorithmic(case: MixedCase) -> dict[str, float]:
    """Minimum bytes and flops of the step's parts.

    write: new rows read (source dtype) + codes written; decode: KV bytes of
    every decode's context + q/o; prefill: KV bytes of each chunk's
    sequence (read once) + q/o, and the QK^T + PV flops of the causal rows
    (4 * D flops per (row, query head, attended token))."""
    esize = torch.tensor([], dtype=case.kv_dtype).element_size()
    hkv, d = case.num_kv_heads, case.k_pool.shape[3]
    hq = case.q_prefill.shape[1]
    per_tok = 2 * hkv * d * esize
    t_new = len(case.slots)
    write = 2 * t_new * hkv * d * (case.k_new.element_size() + esize)
    qo_d = 2 * case.q_decode.numel() * 2
    decode = sum(case.decode_lens) * per_tok + qo_d
    qo_p = 2 * case.q_prefill.numel() * 2
    prefill = sum(case.prefill_lens) * per_tok + qo_p
    attended = 0
    for (c, n) in zip(case.meta["cached"], case.meta["chunks"]):
        attended += n * c + n * (n + 1) // 2
    flops = 4.0 * d * hq * attended
    return {"write_bytes": write, "decode_bytes": decode, "prefill_bytes": prefill, "prefill_flops": flops,
            "decode_tokens": len(case.decode_lens), "prefill_tokens": t_new - len(case.decode_lens)}
