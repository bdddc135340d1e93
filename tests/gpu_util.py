"""Helpers shared by the GPU parity tests (comparison metrics, oracle glue)."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle.paged_attention import paged_attention_fp64


def metrics(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    err = float(np.abs(g - r).max()) if g.size else 0.0
    den = math.sqrt(float((g @ g) * (r @ r)))
    cos = float(g @ r / den) if den > 0 else 1.0
    return err, cos


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of the bfloat16 grid at |x| (8 significant bits)."""
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0**-126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def assert_close(got, ref, dtype: torch.dtype, what: str = "") -> None:
    """Parity against the float64 oracle.

    fp32 outputs: max-abs <= 1e-5.  bf16 outputs (bf16 or e4m3 caches):
    cosine >= 0.9999 and every element within max(2e-2, one bf16 ulp of the
    exact value) -- an output stored in bfloat16 is off by up to half an ulp
    from the exact value whatever computed it (0.03 at |o| = 14), so the
    2e-2 bound applies where the bf16 grid is finer than it.
    """
    err, cos = metrics(got, ref)
    print(f"[parity] {what} max_abs={err:.3e} cosine={cos:.7f}", flush=True)
    if dtype == torch.float32:
        assert err <= 1e-5, (what, err)
    else:
        g = np.asarray(got, dtype=np.float64)
        r = np.asarray(ref, dtype=np.float64)
        bound = np.maximum(2e-2, bf16_ulp(r))
        excess = float((np.abs(g - r) - bound).max()) if g.size else 0.0
        assert cos >= 0.9999 and excess <= 0.0, (what, err, cos, excess)


def codes(t: torch.Tensor) -> np.ndarray:
    """e4m3fn tensor (any strides) -> uint8 codes in logical order."""
    return t.contiguous().view(torch.uint8).cpu().numpy()


def oracle_decode(case, kc: torch.Tensor, vc: torch.Tensor, ks, vs, tables=None, lens=None) -> np.ndarray:
    """fp64 oracle on exactly the cache contents the kernel read (only the
    blocks the tables reference are copied back)."""
    tables = [list(t) for t in (tables if tables is not None else case.block_tables)]
    lens = list(lens if lens is not None else case.seq_lens)
    used = sorted({b for t in tables for b in t})
    remap = {b: i for i, b in enumerate(used)}
    tables = [[remap[b] for b in t] for t in tables]
    idx = torch.tensor(used, dtype=torch.long, device=kc.device)
    kc, vc = kc[idx], vc[idx]
    if kc.dtype == torch.float8_e4m3fn:
        k = ofp8.decode(codes(kc))
        v = ofp8.decode(codes(vc))
        ksn, vsn = ks.cpu().numpy(), vs.cpu().numpy()
    else:
        k = kc.float().cpu().numpy()
        v = vc.float().cpu().numpy()
        ksn = vsn = None
    return paged_attention_fp64(case.q.float().cpu().numpy(), k, v, tables, lens, case.block_size, case.scale,
                                ksn, vsn)
