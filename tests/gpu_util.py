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


def round_to(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """float64 values rounded to `dtype` (round to nearest even), as float64."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float64))
    return t.to(dtype).to(torch.float64).numpy()


def assert_close(got, ref, dtype: torch.dtype, what: str = "") -> None:
    """Parity against the float64 oracle.

    fp32 outputs: max-abs <= 1e-5 against the exact value.  bf16 / fp16
    outputs (16-bit, or e4m3 caches): the oracle is rounded to the output
    dtype first -- the value a correctly rounded kernel would store -- and
    every element must be within 2e-2 of it, with cosine >= 0.9999.  The
    worst element is printed.
    """
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    if dtype != torch.float32:
        r = round_to(r, dtype)
    err, cos = metrics(g, r)
    worst = ""
    if g.size:
        i = int(np.abs(g - r).argmax())
        idx = np.unravel_index(i, g.shape)
        worst = f" worst at {tuple(int(x) for x in idx)}: got {g.flat[i]:.6g} want {r.flat[i]:.6g}"
    print(f"[parity] {what} max_abs={err:.3e} cosine={cos:.7f}{worst}", flush=True)
    if dtype == torch.float32:
        assert err <= 1e-5, (what, err)
    else:
        assert err <= 2e-2 and cos >= 0.9999, (what, err, cos, worst)


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
