"""The paired scan instance (one work-group per 32 value columns of a
(sequence, head)) against the 16-column instance, through the C ABI's
deltanet_chunk_prefill_cols: bitwise the same o and final state, since each
half runs the 16-column arithmetic operation for operation.  The library picks
the paired instance by itself once the 16-column groups outnumber the CUs, so
the oracle-parity tests of packed batches (test_gpu_prefill.py: the
8-sequence batch, the edge lengths, the per-sequence equality) and of the fp16
batch (test_gpu_fused.py: B=2 HV=32) run it too; here both instances are
forced on the same inputs, including shapes where the library would not pick
the paired one, and the paired instance's bounded waits are checked to give up
cleanly.
"""
import ctypes as ct

import pytest
import torch

import gdn_cases as gc
from gdn_hip import capi

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return capi.lib()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _run(lib, dev, d, cu, cols, spin=0):
    """One call of deltanet_chunk_prefill_cols; returns (o, sf, status)."""
    q, k, v, g, beta, s0 = d
    B, T, HK, D = q.shape
    HV = v.shape[2]
    N = len(cu) - 1 if cu is not None else B
    if cu is not None:
        wsb = lib.deltanet_prefill_varlen_live_workspace_size(T, N, HV, D, D, 64)
    else:
        wsb = lib.deltanet_prefill_live_workspace_size(B, T, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    sf = torch.empty(N, HV, D, D, dtype=torch.float32, device=dev)
    cud = cu.to(dev) if cu is not None else None
    print(f"[pair] cols={cols} N={N} T={T} HV={HV} spin={spin}", flush=True)
    err = lib.deltanet_chunk_prefill_cols(
        capi.ptr(q), capi.ptr(k), capi.ptr(v), capi.ptr(g), capi.ptr(beta), o.data_ptr(),
        s0.data_ptr(), sf.data_ptr(), cud.data_ptr() if cud is not None else None, N, T, HV, HK,
        ws.data_ptr(), wsb, _stream(), cols, ct.c_uint(spin))
    assert err == capi.HIP_SUCCESS, err
    st = lib.deltanet_prefill_status(ws.data_ptr(), wsb, _stream())
    torch.cuda.synchronize()
    return o, sf, st


def _same(lib, dev, d, cu, tag):
    o16, s16, st16 = _run(lib, dev, d, cu, 16)
    o32, s32, st32 = _run(lib, dev, d, cu, 32)
    assert st16 == capi.HIP_SUCCESS and st32 == capi.HIP_SUCCESS, (st16, st32)
    assert torch.equal(o16, o32), f"{tag}: o differs, max {(o16.float() - o32.float()).abs().max()}"
    assert torch.equal(s16, s32), f"{tag}: state differs, max {(s16 - s32).abs().max()}"


def test_pair_equals_16col_varlen_8_sequences(lib, dev):
    """The 8-sequence packed batch (seed-7 lengths, 19,861 tokens, HV=32)."""
    q, k, v, g, beta, s0, cu = gc.varlen_inputs()
    _same(lib, dev, [t.to(dev) for t in (q, k, v, g, beta, s0)], cu, "varlen 8 seqs")


def test_pair_equals_16col_planner_shape(lib, dev):
    """B=1 T=1141 HV=32, where the library runs the 16-column instance."""
    d = [t.to(dev) for t in gc.prefill_inputs()]
    _same(lib, dev, d, None, "T1141 HV32")


def test_pair_equals_16col_edges(lib, dev):
    """Empty, single-token and chunk-boundary lengths, one and two ring
    rounds (1..3 chunks) and a sequence ending exactly on a stage reuse."""
    lens = torch.tensor([0, 1, 63, 64, 65, 0, 130, 5, 128, 192, 193])
    q, k, v, g, beta, s0, cu = gc.varlen_inputs(lens)
    _same(lib, dev, [t.to(dev) for t in (q, k, v, g, beta, s0)], cu, "varlen edges")


@pytest.mark.parametrize("B,T,HK,HV", [(3, 300, 2, 4), (3, 300, 16, 16), (3, 200, 4, 12),
                                       (40, 100, 1, 1)])
def test_pair_equals_16col_batch_head_maps(lib, dev, B, T, HK, HV):
    """Fixed-length batches: GQA 2, 1 and 3, a head count that is not a
    multiple of 8 (HV=12: partial XCD rows of the group-id map), and 40
    one-head sequences (the library picks the paired instance there)."""
    d = [t.to(dev) for t in gc.make_gdn_inputs(61 + HV + B, B=B, T=T, HK=HK, HV=HV, g_shift=2.0)]
    _same(lib, dev, d, None, f"B{B} T{T} HK{HK} HV{HV}")


def test_pair_spin_limit_reports_timeout(lib, dev):
    """The paired instance's waits limited to one poll (spin_limit 0 would
    mean the library's own limit here) give up at once: every kernel returns
    normally and the status word reports hipErrorLaunchTimeOut; a normal
    call on fresh buffers succeeds."""
    q, k, v, g, beta, s0, cu = gc.varlen_inputs(torch.tensor([300, 200, 64]))
    d = [t.to(dev) for t in (q, k, v, g, beta, s0)]
    _, _, st = _run(lib, dev, d, cu, 32, spin=1)
    assert st == capi.HIP_ERROR_LAUNCH_TIMEOUT, st
    _, _, st = _run(lib, dev, d, cu, 32)
    assert st == capi.HIP_SUCCESS, st


def test_cols_rejects(lib, dev):
    d = [t.to(dev) for t in gc.make_gdn_inputs(5, B=1, T=64, HK=2, HV=4)]
    q, k, v, g, beta, s0 = d
    wsb = lib.deltanet_prefill_live_workspace_size(1, 64, 4, 128, 128, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    sf = torch.empty_like(s0)
    for cols in (8, 24, 64, -16):
        assert lib.deltanet_chunk_prefill_cols(
            capi.ptr(q), capi.ptr(k), capi.ptr(v), capi.ptr(g), capi.ptr(beta), o.data_ptr(),
            s0.data_ptr(), sf.data_ptr(), None, 1, 64, 4, 2, ws.data_ptr(), wsb, _stream(), cols,
            ct.c_uint(0)) == capi.HIP_ERROR_INVALID_VALUE


def test_pair_noalloc_matches_workspace_entry(lib, dev):
    """The allocation-free entry at a shape where the library picks the
    paired scan (B=2 T=300 HV=32: 320 chunk-heads, inside its array) gives
    bitwise the workspace entry's o and final state, and reports success."""
    q, k, v, g, beta, s0 = [t.to(dev) for t in gc.make_gdn_inputs(71, B=2, T=300, HK=16, HV=32,
                                                                   g_shift=2.0)]
    B, T, HK, D = q.shape
    HV = v.shape[2]
    wsb = lib.deltanet_prefill_live_workspace_size(B, T, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    o1, o2 = torch.empty_like(v), torch.empty_like(v)
    s1, s2 = torch.empty_like(s0), torch.empty_like(s0)
    args = [capi.ptr(t) for t in (q, k, v, g, beta)]
    print(f"[pair] noalloc B={B} T={T} HV={HV}", flush=True)
    assert lib.deltanet_chunk_prefill(*args, o1.data_ptr(), s0.data_ptr(), s1.data_ptr(), B, T,
                                      HV, HK, D, D, 64, ws.data_ptr(), wsb, _stream(),
                                      0) == capi.HIP_SUCCESS
    assert lib.deltanet_chunk_prefill_noalloc(*args, o2.data_ptr(), s0.data_ptr(), s2.data_ptr(),
                                              B, T, HV, HK, D, D, 64,
                                              _stream()) == capi.HIP_SUCCESS
    assert lib.deltanet_prefill_noalloc_status(_stream()) == capi.HIP_SUCCESS
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
