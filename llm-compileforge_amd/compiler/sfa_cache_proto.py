"""Protobuf messages of the cache-policy contract, built without protoc.

The reference declares SfaSlabSpec, SfaInterceptSpec and SfaCachePolicy in
include/sfa_abi.proto:256-286 (package `sfa`) and imports the
protoc-generated `gen.proto.python.sfa_abi_pb2`, which is not part of its
sources.  This module declares the same three messages, field for field and
number for number, through a descriptor built in code, in a private
descriptor pool (so a generated sfa_abi_pb2 loaded in the same process does
not clash).  The wire format is therefore the reference's: a blob from
either side parses on the other.

One field is added: SfaSlabSpec.scales = 209 (repeated float, packed), the
dequantization scale of each (layer, KV head) of an FP8 slab, row-major
[num_layers, num_heads]; empty means 1.0.  Readers that do not know it skip
it, as proto3 requires.
"""

from __future__ import annotations

from google.protobuf import descriptor_pb2, descriptor_pool, message_factory

_F = descriptor_pb2.FieldDescriptorProto

# (name, number, type, repeated)
_SLAB_FIELDS = [
    ("name", 200, _F.TYPE_STRING, False),
    ("slab_type", 201, _F.TYPE_STRING, False),
    ("layout", 202, _F.TYPE_STRING, False),
    ("dtype", 203, _F.TYPE_STRING, False),
    ("num_blocks", 204, _F.TYPE_UINT32, False),
    ("block_size", 205, _F.TYPE_UINT32, False),
    ("num_layers", 206, _F.TYPE_UINT32, False),
    ("num_heads", 207, _F.TYPE_UINT32, False),
    ("head_dim", 208, _F.TYPE_UINT32, False),
    ("scales", 209, _F.TYPE_FLOAT, True),
]
_INTERCEPT_FIELDS = [
    ("slab_id", 210, _F.TYPE_STRING, False),
    ("op_name_pattern", 211, _F.TYPE_STRING, False),
    ("intercept_type", 212, _F.TYPE_STRING, False),
    ("source", 213, _F.TYPE_STRING, False),
    ("layer", 214, _F.TYPE_STRING, False),
    ("param_indices", 215, _F.TYPE_UINT32, True),
]


def _build_pool() -> descriptor_pool.DescriptorPool:
    fdp = descriptor_pb2.FileDescriptorProto(name="cf_sfa_cache_policy.proto", package="sfa", syntax="proto3")

    def message(name: str, fields: list[tuple[str, int, int, bool]]) -> descriptor_pb2.DescriptorProto:
        m = fdp.message_type.add(name=name)
        for fname, num, ftype, rep in fields:
            m.field.add(name=fname, number=num, type=ftype,
                        label=_F.LABEL_REPEATED if rep else _F.LABEL_OPTIONAL)
        return m

    message("SfaSlabSpec", _SLAB_FIELDS)
    message("SfaInterceptSpec", _INTERCEPT_FIELDS)
    pol = fdp.message_type.add(name="SfaCachePolicy")
    pol.field.add(name="slabs", number=220, type=_F.TYPE_MESSAGE, type_name=".sfa.SfaSlabSpec",
                  label=_F.LABEL_REPEATED)
    pol.field.add(name="intercepts", number=221, type=_F.TYPE_MESSAGE, type_name=".sfa.SfaInterceptSpec",
                  label=_F.LABEL_REPEATED)
    pol.field.add(name="block_size", number=222, type=_F.TYPE_UINT32, label=_F.LABEL_OPTIONAL)
    pol.field.add(name="max_requests", number=223, type=_F.TYPE_UINT32, label=_F.LABEL_OPTIONAL)
    pool = descriptor_pool.DescriptorPool()
    pool.Add(fdp)
    return pool


_POOL = _build_pool()
SfaSlabSpec = message_factory.GetMessageClass(_POOL.FindMessageTypeByName("sfa.SfaSlabSpec"))
SfaInterceptSpec = message_factory.GetMessageClass(_POOL.FindMessageTypeByName("sfa.SfaInterceptSpec"))
SfaCachePolicy = message_factory.GetMessageClass(_POOL.FindMessageTypeByName("sfa.SfaCachePolicy"))

__all__ = ["SfaCachePolicy", "SfaInterceptSpec", "SfaSlabSpec"]
