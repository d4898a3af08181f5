"""deltanet_chunk_prefill_noalloc (the allocation-free prefill, whose
workspace is a static device array) against deltanet_chunk_prefill with a
caller workspace, through the C ABI: identical o and final state on two calls
in a row, the second on a smaller input, a clear status word after each
(deltanet_prefill_noalloc_status), and a host-side reject of a size the array
cannot hold."""
import pytest
import torch

import gdn_cases as gc
from gdn_hip import capi

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _run_pair(lib, dev, seed, B, T, HK, HV):
    q, k, v, g, beta, s0 = [t.to(dev) for t in gc.make_gdn_inputs(seed, B=B, T=T, HK=HK, HV=HV)]
    D = 128
    print(f"[noalloc] B={B} T={T} HK={HK} HV={HV} seed={seed}", flush=True)
    o_ref = torch.empty_like(v)
    s_ref = torch.empty_like(s0)
    wsb = lib.deltanet_prefill_live_workspace_size(B, T, HV, D, D, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    args = [capi.ptr(t) for t in (q, k, v, g, beta)]
    assert lib.deltanet_chunk_prefill(*args, o_ref.data_ptr(), s0.data_ptr(), s_ref.data_ptr(),
                                      B, T, HV, HK, D, D, 64, ws.data_ptr(), wsb, _stream(),
                                      0) == capi.HIP_SUCCESS
    o = torch.full_like(v, float("nan"))
    sf = torch.full_like(s0, float("nan"))
    assert lib.deltanet_chunk_prefill_noalloc(*args, o.data_ptr(), s0.data_ptr(), sf.data_ptr(),
                                              B, T, HV, HK, D, D, 64, _stream()) == capi.HIP_SUCCESS
    # no bounded wait of the call gave up (the status word in the array's header)
    assert lib.deltanet_prefill_noalloc_status(_stream()) == capi.HIP_SUCCESS
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref), "o differs from the workspace entry"
    assert torch.equal(sf, s_ref), "final state differs from the workspace entry"


def test_noalloc_matches_workspace_entry(dev):
    lib = capi.lib()
    _run_pair(lib, dev, 41, B=1, T=1141, HK=16, HV=32)   # the planner shape
    _run_pair(lib, dev, 42, B=2, T=100, HK=2, HV=4)      # then a smaller input


def test_noalloc_rejects_oversize(dev):
    lib = capi.lib()
    # 23 chunks x 32 heads = 736 chunk-heads > 712
    B, T, HK, HV, D = 1, 23 * 64, 16, 32, 128
    dummy = torch.empty(16, device=dev)
    p = dummy.data_ptr()
    print(f"[noalloc] reject T={T} HV={HV}", flush=True)
    assert lib.deltanet_chunk_prefill_noalloc(p, p, p, p, p, p, p, p, B, T, HV, HK, D, D, 64,
                                              _stream()) == capi.HIP_ERROR_INVALID_VALUE
