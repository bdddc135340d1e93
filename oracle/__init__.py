"""CPU oracle for the paged-decode + FP8-KV path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import or run anything here, and only as the checker (or the timed CPU
baseline), never as the product path.

Contents and what pins each part:
  fp8_e4m3.c / fp8.py   OCP e4m3fn encoder/decoder, amax->scale rule and
                        quantize, restating compiler/quantize/fp8_kv_cache.py
                        :66-105 of the reference.  Pinned by an exhaustive
                        comparison over all 2^32 fp32 inputs with torch's
                        float8_e4m3fn cast (the library routine the reference
                        calls), the 256-code decode table, known answers from
                        the OCP spec (tests/golden/) and closed-form scale
                        cases (zero block, clamp at 1e-12).
  fp8_kv_cache.py       The reference FP8KVCacheQuantizer restated with torch
                        CPU ops; pinned against fp8.py bit for bit and by the
                        reference's own TestFP8KVCache cases.
  paged_attention.py    _paged_attention_cpu restated (reference
                        kernels/paged_attention.py:21-73) with torch CPU
                        SDPA, plus an independent float64 brute force; the
                        two are checked against each other and against
                        invariants (block permutation, shared prefix, GQA as
                        repeated MHA, truncation rules).

The reference itself is never imported or run: every function above is
pinned by a library routine, mathematics or golden vectors.
"""
