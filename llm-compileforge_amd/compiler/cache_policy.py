"""Cache policy: the declarative KV-cache contract between compiler and runtime.

Drop-in for the reference's compiler/cache_policy.py: the same classes,
factories, dict form (metadata.json) and proto form (the SfaCachePolicy
blob, include/sfa_abi.proto:256-286), so policies written by either side
load on the other.  Additions, all optional and backward compatible:

- `kv_dtype` on `for_llama` / `for_config` / `for_mixed_linear` picks the
  K/V slab dtype; "float8_e4m3fn" gives FP8 slabs (default "float32", the
  reference's).
- `_SlabSpec.scales`: per-(layer, KV head) dequantization scales of an FP8
  slab, [num_layers][num_heads]; written to the dict as "scales" and to the
  proto as SfaSlabSpec field 209 only when set; `CachePolicy.set_kv_scales`
  stores calibrated scales.
- `parse_cache_policy`, the inverse of `serialize_cache_policy`.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any

KV_DTYPES = ("float32", "float16", "bfloat16", "float8_e4m3fn")
_SDPA = "scaled_dot_product_attention"


@dataclass
class _SlabSpec:
    """One cache region (reference cache_policy.py:17-52).

    slab_id: logical name ("k", "v", "state", ...); storage: "paged" |
    "flat" | "circular" | "fixed"; dims: allocation hints such as
    {"layers", "heads", "dim"}; layout: dim-order string ("BNLD", "RLD");
    dtype: element type name; scales: FP8 slabs only, [layers][heads]
    dequantization scales (None = all 1.0).
    """

    slab_id: str
    storage: str
    dims: dict[str, int]
    layout: str
    dtype: str = "float32"
    scales: list[list[float]] | None = None

    def to_dict(self) -> dict[str, Any]:
        out: dict[str, Any] = {
            "slab_id": self.slab_id,
            "storage": self.storage,
            "dims": self.dims,
            "layout": self.layout,
            "dtype": self.dtype,
        }
        if self.scales is not None:
            out["scales"] = [list(row) for row in self.scales]
        return out

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> _SlabSpec:
        scales = d.get("scales")
        return cls(
            slab_id=d["slab_id"],
            storage=d["storage"],
            dims={k: int(v) for k, v in d["dims"].items()},
            layout=d["layout"],
            dtype=d.get("dtype", "float32"),
            scales=None if scales is None else [[float(x) for x in row] for row in scales],
        )


@dataclass
class _InterceptSpec:
    """When and how the executor intercepts an op for cache I/O (reference
    cache_policy.py:55-104): `source` is "operand[N]" or "output", `layer`
    "sequential" or a static index; func_index / output_index pin an
    intercept to one producer output after binding."""

    slab_id: str
    op_name: str
    direction: str
    source: str
    layer: str = "sequential"
    func_index: int | None = None
    output_index: int | None = None

    def to_dict(self) -> dict[str, Any]:
        out: dict[str, Any] = {
            "slab_id": self.slab_id,
            "op_name": self.op_name,
            "direction": self.direction,
            "source": self.source,
            "layer": self.layer,
        }
        for key in ("func_index", "output_index"):
            if getattr(self, key) is not None:
                out[key] = getattr(self, key)
        return out

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> _InterceptSpec:
        return cls(
            slab_id=d["slab_id"],
            op_name=d["op_name"],
            direction=d["direction"],
            source=d["source"],
            layer=d.get("layer", "sequential"),
            func_index=d.get("func_index"),
            output_index=d.get("output_index"),
        )


def _config_value(config: Any, name: str, default: Any = None) -> Any:
    """A config field from a mapping or an attribute object."""
    if isinstance(config, dict):
        return config.get(name, default)
    return getattr(config, name, default)


def _check_kv_dtype(kv_dtype: str) -> str:
    if kv_dtype not in KV_DTYPES:
        raise ValueError(f"kv_dtype must be one of {KV_DTYPES}, got {kv_dtype!r}")
    return kv_dtype


def _kv_slabs(num_layers: int, num_kv_heads: int, head_dim: int, kv_dtype: str) -> list[_SlabSpec]:
    dims = {"layers": num_layers, "heads": num_kv_heads, "dim": head_dim}
    return [_SlabSpec(name, "paged", dict(dims), "BNLD", _check_kv_dtype(kv_dtype)) for name in ("k", "v")]


def _kv_intercepts() -> list[_InterceptSpec]:
    return [_InterceptSpec("k", _SDPA, "read_write", "operand[1]"),
            _InterceptSpec("v", _SDPA, "read_write", "operand[2]")]


@dataclass
class CachePolicy:
    """Declarative model cache strategy (reference cache_policy.py:107-410):
    slabs to pre-allocate, per-op cache I/O, paged block size and the pool
    capacity of fixed slabs."""

    slabs: list[_SlabSpec] = field(default_factory=list)
    intercepts: list[_InterceptSpec] = field(default_factory=list)
    block_size: int = 16
    max_requests: int = 256

    @property
    def is_empty(self) -> bool:
        return len(self.slabs) == 0

    @classmethod
    def none(cls) -> CachePolicy:
        """No cache: the executor recomputes every step."""
        return cls()

    @classmethod
    def for_config(cls, config: Any, block_size: int = 16, kv_dtype: str = "float32") -> CachePolicy:
        """SDPA K/V policy from a model config (mapping or attribute object;
        a nested `text_config` is used when present).

        head_dim falls back to hidden_size / num_attention_heads and
        num_key_value_heads to num_attention_heads.  Raises ValueError for
        missing or inconsistent attention fields; configs whose
        `layer_types` mix linear and full attention get `for_mixed_linear`.
        """
        nested = _config_value(config, "text_config")
        cfg = config if nested is None else nested
        n_layers = _config_value(cfg, "num_hidden_layers")
        n_heads = _config_value(cfg, "num_attention_heads")
        n_kv = _config_value(cfg, "num_key_value_heads") or n_heads
        missing = [k for k, v in (("num_hidden_layers", n_layers), ("num_attention_heads", n_heads),
                                  ("num_key_value_heads", n_kv)) if v is None]
        if missing:
            raise ValueError(f"Config is missing attention fields required for CachePolicy: {missing}")
        head_dim = _config_value(cfg, "head_dim")
        if head_dim is None:
            hidden = _config_value(cfg, "hidden_size")
            if hidden is None:
                raise ValueError("Config is missing both head_dim and hidden_size")
            if int(hidden) % int(n_heads):
                raise ValueError(f"hidden_size={hidden} is not divisible by num_attention_heads={n_heads}")
            head_dim = int(hidden) // int(n_heads)
        kinds = _config_value(cfg, "layer_types")
        if kinds is not None:
            kinds = [str(t) for t in ([kinds] if isinstance(kinds, str) else kinds)]
            n_full = sum(t == "full_attention" for t in kinds)
            if n_full != len(kinds):

                def get(name: str, default: int = 0) -> int:
                    return int(_config_value(cfg, name, default) or default)

                return cls.for_mixed_linear(
                    num_layers=int(n_layers), num_full_layers=n_full, num_linear_layers=len(kinds) - n_full,
                    num_kv_heads=int(n_kv), head_dim=int(head_dim),
                    linear_num_key_heads=get("linear_num_key_heads"),
                    linear_num_value_heads=get("linear_num_value_heads"),
                    linear_key_head_dim=get("linear_key_head_dim"),
                    linear_value_head_dim=get("linear_value_head_dim"),
                    linear_conv_kernel_dim=get("linear_conv_kernel_dim", 4),
                    block_size=block_size, kv_dtype=kv_dtype,
                )
            if len(kinds) != int(n_layers):
                raise ValueError(f"layer_types length {len(kinds)} != num_hidden_layers {n_layers}")
        return cls.for_llama(int(n_layers), int(n_kv), int(head_dim), block_size=block_size, kv_dtype=kv_dtype)

    @classmethod
    def for_mixed_linear(
        cls,
        num_layers: int,
        num_full_layers: int,
        num_linear_layers: int,
        num_kv_heads: int,
        head_dim: int,
        linear_num_key_heads: int,
        linear_num_value_heads: int,
        linear_key_head_dim: int,
        linear_value_head_dim: int,
        linear_conv_kernel_dim: int = 4,
        block_size: int = 16,
        kv_dtype: str = "float32",
    ) -> CachePolicy:
        """Full-attention layers get paged K/V slabs; the linear-attention
        layers two fixed state slabs: the delta-rule state [heads, key_dim,
        value_dim] and the short-convolution state [channels, kernel] with
        channels = 2 * key_heads * key_dim + value_heads * value_dim."""
        channels = 2 * linear_num_key_heads * linear_key_head_dim + linear_num_value_heads * linear_value_head_dim
        slabs = _kv_slabs(num_full_layers, num_kv_heads, head_dim, kv_dtype) + [
            _SlabSpec("recurrent_state", "fixed",
                      {"layers": num_linear_layers, "heads": linear_num_value_heads,
                       "key_dim": linear_key_head_dim, "value_dim": linear_value_head_dim}, "BHKV"),
            _SlabSpec("conv_state", "fixed",
                      {"layers": num_linear_layers, "channels": channels, "kernel": linear_conv_kernel_dim}, "BCK"),
        ]
        intercepts = _kv_intercepts() + [
            _InterceptSpec(name, "linear_attn", "read_write", name) for name in ("recurrent_state", "conv_state")
        ]
        return cls(slabs=slabs, intercepts=intercepts, block_size=block_size)

    @classmethod
    def from_dict(cls, d: dict[str, Any] | None) -> CachePolicy:
        if d is None:
            return cls.none()
        return cls(
            slabs=[_SlabSpec.from_dict(s) for s in d.get("slabs", [])],
            intercepts=[_InterceptSpec.from_dict(i) for i in d.get("intercepts", [])],
            block_size=int(d.get("block_size", 16)),
            max_requests=int(d.get("max_requests", 256)),
        )

    def to_dict(self) -> dict[str, Any]:
        return {
            "slabs": [s.to_dict() for s in self.slabs],
            "intercepts": [i.to_dict() for i in self.intercepts],
            "block_size": self.block_size,
            "max_requests": self.max_requests,
        }

    @classmethod
    def for_llama(
        cls, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int = 16, kv_dtype: str = "float32"
    ) -> CachePolicy:
        """Paged "k"/"v" slabs [layers, heads, dim] read and written at SDPA
        operands 1 and 2."""
        return cls(slabs=_kv_slabs(num_layers, num_kv_heads, head_dim, kv_dtype), intercepts=_kv_intercepts(),
                   block_size=block_size)

    @classmethod
    def for_rwkv(cls, num_layers: int, state_dim: int, max_requests: int = 256) -> CachePolicy:
        """One fixed "state" slab [requests, layers, state_dim] at state_evolve's output."""
        return cls(
            slabs=[_SlabSpec("state", "fixed", {"layers": num_layers, "dim": state_dim}, "RLD")],
            intercepts=[_InterceptSpec("state", "state_evolve", "read_write", "output")],
            max_requests=max_requests,
        )

    def set_kv_scales(self, slab_id: str, scales: Any) -> None:
        """Stores an FP8 slab's dequantization scales, [layers][heads] (any
        nested sequence or tensor of that shape); finite and positive."""
        spec = next((s for s in self.slabs if s.slab_id == slab_id), None)
        if spec is None:
            raise KeyError(f"no slab {slab_id!r}")
        if spec.dtype != "float8_e4m3fn":
            raise ValueError(f"slab {slab_id!r} has dtype {spec.dtype}; scales belong to float8_e4m3fn slabs")
        rows = [[float(x) for x in row] for row in (scales.tolist() if hasattr(scales, "tolist") else scales)]
        want = (int(spec.dims.get("layers", 0)), int(spec.dims.get("heads", 0)))
        if len(rows) != want[0] or any(len(r) != want[1] for r in rows):
            raise ValueError(f"scales must be [{want[0]}][{want[1]}]")
        if not all(math.isfinite(x) and x > 0 for r in rows for x in r):
            raise ValueError("scales must be finite and positive")
        spec.scales = rows


def bind_cache_policy(policy: CachePolicy, bindings: list[tuple[int, int, str]]) -> CachePolicy:
    """Replaces each SDPA intercept template by one entry per binding
    (func_index, output_index, slab_id), the keys the runtime matches
    (reference cache_policy.py:413-464).  Other intercepts are kept; a
    binding whose slab has no template gets read_write / operand[1] /
    sequential.  No bindings: the policy is returned as is.  The input
    policy is not modified."""
    if not bindings:
        return policy
    templates = {i.slab_id: i for i in policy.intercepts if i.op_name == _SDPA}
    out = [i for i in policy.intercepts if i.op_name != _SDPA]
    for fi, oi, slab_id in bindings:
        t = templates.get(slab_id)
        out.append(_InterceptSpec(
            slab_id=slab_id, op_name=_SDPA,
            direction=t.direction if t else "read_write",
            source=t.source if t else "operand[1]",
            layer=t.layer if t else "sequential",
            func_index=fi, output_index=oi,
        ))
    return CachePolicy(slabs=list(policy.slabs), intercepts=out, block_size=policy.block_size,
                       max_requests=policy.max_requests)


def to_proto(policy: CachePolicy) -> Any:
    """The SfaCachePolicy message of a policy (field mapping of the
    reference's serialize_cache_policy, cache_policy.py:467-501)."""
    from compiler.sfa_cache_proto import SfaCachePolicy

    msg = SfaCachePolicy()
    for s in policy.slabs:
        sp = msg.slabs.add()
        sp.name, sp.slab_type, sp.layout, sp.dtype = s.slab_id, s.storage, s.layout, s.dtype
        sp.num_blocks = int(s.dims.get("blocks", 0))
        sp.block_size = policy.block_size
        sp.num_layers = int(s.dims.get("layers", 0))
        sp.num_heads = int(s.dims.get("heads", 0))
        sp.head_dim = int(s.dims.get("dim", 0))
        if s.scales is not None:
            sp.scales.extend(x for row in s.scales for x in row)
    for i in policy.intercepts:
        ip = msg.intercepts.add()
        ip.slab_id, ip.op_name_pattern, ip.intercept_type = i.slab_id, i.op_name, i.direction
        ip.source, ip.layer = i.source, i.layer
        ip.param_indices.extend(int(x) for x in (i.func_index, i.output_index) if x is not None)
    msg.block_size = policy.block_size
    msg.max_requests = policy.max_requests
    return msg


def serialize_cache_policy(policy: CachePolicy) -> bytes:
    """The SfaCachePolicy protobuf blob of a policy (what a compiled
    artifact embeds as its `sfa_cache_policy` symbol)."""
    return bytes(to_proto(policy).SerializeToString())


def parse_cache_policy(blob: bytes) -> CachePolicy:
    """Inverse of serialize_cache_policy.  The proto flattens dims to
    layers/heads/dim (+ blocks), so other dims keys of fixed slabs do not
    survive the trip; param_indices [f, o] come back as func_index /
    output_index."""
    from compiler.sfa_cache_proto import SfaCachePolicy

    msg = SfaCachePolicy()
    msg.ParseFromString(blob)
    slabs = []
    for sp in msg.slabs:
        dims = {"layers": sp.num_layers, "heads": sp.num_heads, "dim": sp.head_dim}
        if sp.num_blocks:
            dims["blocks"] = sp.num_blocks
        scales = None
        if len(sp.scales):
            if len(sp.scales) != sp.num_layers * sp.num_heads:
                raise ValueError(f"slab {sp.name!r}: {len(sp.scales)} scales for "
                                 f"{sp.num_layers} x {sp.num_heads} (layer, head) pairs")
            flat = list(sp.scales)
            scales = [flat[r * sp.num_heads:(r + 1) * sp.num_heads] for r in range(sp.num_layers)]
        slabs.append(_SlabSpec(sp.name, sp.slab_type, dims, sp.layout, sp.dtype or "float32", scales))
    intercepts = []
    for ip in msg.intercepts:
        idx = list(ip.param_indices)
        intercepts.append(_InterceptSpec(
            ip.slab_id, ip.op_name_pattern, ip.intercept_type, ip.source, ip.layer or "sequential",
            func_index=idx[0] if len(idx) > 0 else None, output_index=idx[1] if len(idx) > 1 else None,
        ))
    return CachePolicy(slabs=slabs, intercepts=intercepts, block_size=msg.block_size or 16,
                       max_requests=msg.max_requests or 256)


__all__ = [
    "KV_DTYPES",
    "CachePolicy",
    "_InterceptSpec",
    "_SlabSpec",
    "bind_cache_policy",
    "parse_cache_policy",
    "serialize_cache_policy",
    "to_proto",
]
