"""The no-allocation decode entry point (cf_paged_decode_shared_noalloc)
against the workspace entry point it shares its kernels with
(cf_paged_decode_shared), through the C ABI.  Runs last: it is collected
after every other test file."""

from __future__ import annotations

import ctypes

import pytest
import torch

from cf_hip import _abi, ops, workloads
from cf_hip import layout as L

pytestmark = pytest.mark.gpu


def _noalloc(case, kc, vc, ks, vs, tables, lens, shared, out):
    """One call of the C entry point through ctypes, no Python wrapper."""
    ds = [_abi.descriptor(t) for t in (case.q, kc, vc, tables, lens)]
    dsh = _abi.descriptor(shared) if shared is not None else None
    dks = _abi.descriptor(ks) if ks is not None else None
    dvs = _abi.descriptor(vs) if vs is not None else None
    do = _abi.descriptor(out)
    rc = _abi.lib().cf_paged_decode_shared_noalloc(
        *(ctypes.byref(d) for d in ds), _abi.ref(dsh), _abi.ref(dks), _abi.ref(dvs), ctypes.c_float(case.scale),
        16, 512, ctypes.byref(do), ctypes.c_void_p(_abi.stream_handle(case.q.device)))
    return rc


def _with_workspace(case, kc, vc, ks, vs, tables, lens, shared):
    need = ops.decode_workspace_bytes(case.batch, case.q.shape[1], case.num_kv_heads, case.head_dim,
                                      tables.shape[1], 16)
    ws = ops.new_workspace(need, case.q.device)
    return ops.paged_decode(case.q, kc, vc, tables, lens, case.scale, 16, ks, vs, workspace=ws,
                            shared_prefix_lens=shared)


def test_noalloc_matches_workspace_entry_point(gpu):
    """Two calls in a row -- the full c3 batch with the shared-prefix
    statement, then a smaller c2 batch (another shape, other kernels'
    template) -- each bitwise equal to cf_paged_decode_shared on the same
    inputs; then a repeat of the first call, over the scratch the smaller
    call left behind."""
    calls = []
    big = workloads.make_case("c3_llama3_8b", device=gpu, seed=3)
    bkc, bvc, bks, bvs = workloads.materialize(big, "paired")
    sh = torch.tensor(ops.shared_prefix_lens(big.block_tables, big.seq_lens, 16), dtype=torch.int32, device=gpu)
    calls.append((big, bkc, bvc, bks, bvs, big.tables_tensor(gpu), big.seq_lens_tensor(gpu), sh))
    small = workloads.make_case("c2_tinyllama", device=gpu, seed=4, batch=5)
    skc, svc, sks, svs = workloads.materialize(small, "native")
    calls.append((small, skc, svc, sks, svs, small.tables_tensor(gpu), small.seq_lens_tensor(gpu), None))
    calls.append(calls[0])
    for i, args in enumerate(calls):
        case = args[0]
        print(f"[case] no-alloc call {i}: {case.name} batch {case.batch}", flush=True)
        out = torch.full(case.q.shape, float("nan"), dtype=case.q.dtype, device=gpu)
        rc = _noalloc(*args, out)
        assert rc == 0, _abi.last_error()
        want = _with_workspace(*args)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"call {i}: no-alloc output differs from the workspace entry point"


def test_noalloc_allocates_nothing_and_replays_in_a_graph(gpu):
    """The entry point under HIP graph capture (torch.cuda.graph): captured
    once, replayed four times with eager work between the replays (other
    no-alloc and workspace calls over the same scratch and a refill of the
    output), each replay bitwise equal to the workspace entry point; torch's
    allocator sees no allocation across an eager call or a replay."""
    case = workloads.make_case("c3_llama3_8b", device=gpu, seed=5, batch=16)
    kc, vc, ks, vs = workloads.materialize(case, "paired")
    sh = torch.tensor(ops.shared_prefix_lens(case.block_tables, case.seq_lens, 16), dtype=torch.int32, device=gpu)
    args = (case, kc, vc, ks, vs, case.tables_tensor(gpu), case.seq_lens_tensor(gpu), sh)
    want = _with_workspace(*args)
    other = workloads.make_case("c2_tinyllama", device=gpu, seed=6, batch=7)
    okc, ovc, oks, ovs = workloads.materialize(other, "native")
    oargs = (other, okc, ovc, oks, ovs, other.tables_tensor(gpu), other.seq_lens_tensor(gpu), None)
    oout = torch.empty(other.q.shape, dtype=other.q.dtype, device=gpu)
    out = torch.full(case.q.shape, float("nan"), dtype=case.q.dtype, device=gpu)
    torch.cuda.synchronize()
    print("[case] no-alloc eager call, allocator counters", flush=True)
    before = torch.cuda.memory_allocated(gpu)
    assert _noalloc(*args, out) == 0, _abi.last_error()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(gpu) == before
    assert torch.equal(out, want)
    print("[case] no-alloc captured in a graph", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _noalloc(*args, out)
    assert rc == 0, _abi.last_error()
    torch.cuda.synchronize()
    for r in range(4):
        print(f"[case] graph replay {r}", flush=True)
        out.fill_(float("nan"))
        assert _noalloc(*oargs, oout) == 0, _abi.last_error()  # leaves other contents in the scratch
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated(gpu)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(gpu) == before
        assert torch.equal(out, want), f"replay {r} differs from the workspace entry point"
        _with_workspace(*oargs)
        torch.cuda.synchronize()


def test_noalloc_rejects_calls_beyond_its_scratch(gpu):
    """A batch whose workspace exceeds the fixed scratch is refused before any
    launch, with CF_ERR_WORKSPACE and the need in the message."""
    b, hq, hkv, d = 4096, 64, 8, 128
    need = ops.decode_workspace_bytes(b, hq, hkv, d, 4, 16)
    assert need > ops.NOALLOC_SCRATCH_BYTES
    q = torch.zeros(b, hq, d, dtype=torch.bfloat16, device=gpu)
    kc, vc = L.alloc_kv_cache(8, 16, hkv, d, torch.bfloat16, gpu, "native")  # the MFMA path's layout
    kc.zero_()
    vc.zero_()
    tables = torch.zeros(b, 4, dtype=torch.int32, device=gpu)
    lens = torch.full((b,), 64, dtype=torch.int32, device=gpu)
    out = torch.empty_like(q)
    case = workloads.DecodeCase("over", q, kc, kc, [], [], 16, 0.1, torch.bfloat16)
    rc = _noalloc(case, kc, vc, None, None, tables, lens, None, out)
    assert rc == _abi.CF_ERR_WORKSPACE
    assert "fixed scratch" in _abi.last_error()
    with pytest.raises(ValueError):
        ops.paged_decode_noalloc(q, kc, vc, tables, lens, 0.1, 16, out=out)
