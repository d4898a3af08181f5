"""The C ABI called directly (ctypes, raw device pointers, torch's raw HIP
stream), as a caller of the reference's C entry points would
(kernels/chunk_delta_cuda.h:39-55): deltanet_chunk_prefill and
deltanet_chunk_prefill_varlen against the fp64 oracle, and the status word
of the bounded waits (deltanet_prefill_status).
"""
import ctypes as ct

import pytest
import torch

import gdn_cases as gc
from gdn_hip import capi
from oracle import gdn_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return capi.lib()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_capi_prefill_matches_oracle(lib, dev):
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(31, B=2, T=200, HK=2, HV=4)
    print(f"[capi] deltanet_chunk_prefill B=2 T=200 HK=2 HV=4", flush=True)
    d = [t.to(dev) for t in (q, k, v, g, beta, s0)]
    o = torch.empty_like(d[2])
    sf = torch.empty_like(d[5])
    B, T, HK, D = q.shape
    HV = v.shape[2]
    wsb = lib.deltanet_prefill_live_workspace_size(B, T, HV, D, D, 64)
    assert 0 < wsb < lib.deltanet_prefill_workspace_size(B, T, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    err = lib.deltanet_chunk_prefill(*[capi.ptr(t) for t in d[:5]], o.data_ptr(),
                                     d[5].data_ptr(), sf.data_ptr(), B, T, HV, HK, D, D, 64,
                                     ws.data_ptr(), wsb, _stream(), 0)
    assert err == capi.HIP_SUCCESS
    assert lib.deltanet_prefill_status(ws.data_ptr(), wsb, _stream()) == capi.HIP_SUCCESS
    o_ref, s_ref = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    gc.assert_abs(gc.parity(o, o_ref), what="capi o")
    gc.assert_abs(gc.parity(sf, s_ref), what="capi state")
    # the live size is the minimum: one byte less is rejected on the host
    assert lib.deltanet_chunk_prefill(*[capi.ptr(t) for t in d[:5]], o.data_ptr(),
                                      d[5].data_ptr(), sf.data_ptr(), B, T, HV, HK, D, D, 64,
                                      ws.data_ptr(), wsb - 1, _stream(), 0) == capi.HIP_ERROR_INVALID_VALUE


def test_capi_varlen_matches_oracle(lib, dev):
    lengths = [70, 1, 0, 129, 64]
    q, k, v, g, beta, s0, cu = gc.varlen_inputs(lengths)
    print(f"[capi] deltanet_chunk_prefill_varlen lengths={lengths}", flush=True)
    d = [t.to(dev) for t in (q, k, v, g, beta, s0)]
    cud = cu.to(dev)
    o = torch.zeros_like(d[2])
    sf = torch.empty_like(d[5])
    total, N, HV, HK, D = int(cu[-1]), len(lengths), v.shape[2], q.shape[2], 128
    wsb = lib.deltanet_prefill_varlen_live_workspace_size(total, N, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    err = lib.deltanet_chunk_prefill_varlen(*[capi.ptr(t) for t in d[:5]], o.data_ptr(),
                                            d[5].data_ptr(), sf.data_ptr(), cud.data_ptr(), N,
                                            total, HV, HK, D, D, 64, ws.data_ptr(), wsb,
                                            _stream(), 0)
    assert err == capi.HIP_SUCCESS
    assert lib.deltanet_prefill_status(ws.data_ptr(), wsb, _stream()) == capi.HIP_SUCCESS
    o_ref, s_ref = orc.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, s0, dtype=torch.float64)
    gc.assert_abs(gc.parity(o, o_ref), what="capi varlen o")
    gc.assert_abs(gc.parity(sf, s_ref), what="capi varlen state")


def test_capi_spin_limit_reports_timeout(lib, dev):
    """Waits limited to zero polls give up at once: every kernel still
    returns normally and the status word turns into hipErrorLaunchTimeOut;
    the next normal call on the same workspace reports success again."""
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(32, B=1, T=300, HK=2, HV=4)
    d = [t.to(dev) for t in (q, k, v, g, beta, s0)]
    o = torch.empty_like(d[2])
    sf = torch.empty_like(d[5])
    B, T, HK, D = q.shape
    HV = v.shape[2]
    wsb = lib.deltanet_prefill_live_workspace_size(B, T, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    args = [capi.ptr(t) for t in d[:5]] + [o.data_ptr(), d[5].data_ptr(), sf.data_ptr(),
                                           B, T, HV, HK, ws.data_ptr(), wsb, _stream()]
    print("[capi] deltanet_chunk_prefill_spin spin_limit=0", flush=True)
    assert lib.deltanet_chunk_prefill_spin(*args, ct.c_uint(0)) == capi.HIP_SUCCESS
    assert lib.deltanet_prefill_status(ws.data_ptr(), wsb, _stream()) == capi.HIP_ERROR_LAUNCH_TIMEOUT
    print("[capi] deltanet_chunk_prefill after the timed-out call", flush=True)
    assert lib.deltanet_chunk_prefill(*args[:8], B, T, HV, HK, D, D, 64, ws.data_ptr(), wsb,
                                      _stream(), 0) == capi.HIP_SUCCESS
    assert lib.deltanet_prefill_status(ws.data_ptr(), wsb, _stream()) == capi.HIP_SUCCESS


def test_torch_op_spin_limit_and_checked_mode(ops, dev):
    q, k, v, g, beta, s0 = [t.to(dev) for t in gc.make_gdn_inputs(33, B=1, T=300, HK=2, HV=4)]
    print("[capi] torch _chunk_prefill_spin_limit spin=0", flush=True)
    o, sf, st = ops._chunk_prefill_spin_limit(q, k, v, g, beta, s0, 0)
    assert int(st.item()) == 1
    o2, sf2, st2 = ops._chunk_prefill_spin_limit(q, k, v, g, beta, s0, 1 << 20)
    assert int(st2.item()) == 0
    o3, sf3 = ops.chunk_prefill(q, k, v, g, beta, s0, checked=True)
    assert torch.equal(o2, o3) and torch.equal(sf2, sf3)
