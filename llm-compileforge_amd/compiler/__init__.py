"""Import-path shim: the reference exposes the FP8 KV quantizer under
compiler.quantize (reference compiler/quantize/__init__.py:15-25)."""
