"""The two-level chunk-group scan prototype (deltanet_chunk_prefill_twolevel)
against the oracle and against the plain prefill, through the C ABI: the
T=1141 HV=32 layer at 3 and 4 segments, the 8-sequence packed batch at 4
segments, and edge lengths (one-chunk sequences keep one segment, an empty
sequence passes its state through).  Bars: max |err| <= 2e-2 and the
reference harness's fixture bar against the fp64 oracle; the plain call's
outputs within 2e-3 (o) and 5e-4 (state).  The prototype is less exact than
the plain scan: a segment's transition Phi is scanned from the identity,
whose fp16-rounded state operand carries absolute errors ~5e-4 that the
combine then multiplies into the entry states."""
import ctypes as ct

import pytest
import torch

import gdn_cases as gc
from gdn_hip import capi
from oracle import gdn_oracle as orc

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def run_twolevel(lib, dev, q, k, v, g, beta, s0, cu, segments, events=None):
    """o, final state from the two-level entry; cu is None (fixed length,
    q of shape [B, T, ...]) or a host int32 tensor [N + 1] over packed rows."""
    if cu is None:
        N, T = q.shape[0], q.shape[1]
        cu_p = None
    else:
        N, T = len(cu) - 1, int(cu[-1])
        cu_h = (ct.c_int32 * len(cu))(*[int(x) for x in cu])
        cu_p = ct.cast(cu_h, ct.c_void_p)
    HV, HK = v.shape[2], q.shape[2]
    d = [t.to(dev) for t in (q, k, v, g, beta)]
    s0d = s0.to(dev) if s0 is not None else None
    o = torch.empty_like(d[2])
    sf = torch.empty(N, HV, 128, 128, device=dev)
    wsb = lib.deltanet_prefill_twolevel_workspace_size(cu_p, N, T, HV, segments)
    assert wsb > 0
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    ev, nev = (None, 0) if events is None else (events, 6)
    err = lib.deltanet_chunk_prefill_twolevel(*[capi.ptr(t) for t in d], o.data_ptr(),
                                              capi.ptr(s0d), sf.data_ptr(), cu_p, N, T, HV, HK,
                                              segments, ws.data_ptr(), wsb, _stream(), ev, nev)
    assert err == 0, err
    torch.cuda.synchronize()
    return o, sf


def _check(o, sf, o_ref, s_ref, o_plain, s_plain, tag):
    mo, ms = gc.parity(o, o_ref), gc.parity(sf, s_ref)
    dp_o = (o.float() - o_plain.float()).abs().max().item()
    dp_s = (sf - s_plain).abs().max().item()
    print(f"[twolevel] {tag}\n    o: {gc.fmt(mo)}\n    S: {gc.fmt(ms)}\n"
          f"    vs plain: max|do| {dp_o:.2e} max|dS| {dp_s:.2e}", flush=True)
    gc.assert_abs(mo, what=f"{tag} o")
    gc.assert_abs(ms, what=f"{tag} state")
    gc.assert_fixture_bar(o, o_ref, sf, s_ref, what=tag)
    assert dp_o <= 2e-3 and dp_s <= 5e-4


@pytest.mark.parametrize("segments", [3, 4])
def test_twolevel_T1141_HV32(ops, dev, segments):
    lib = capi.lib()
    q, k, v, g, beta, s0 = gc.prefill_inputs()
    o, sf = run_twolevel(lib, dev, q, k, v, g, beta, s0, None, segments)
    o_ref, s_ref = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    o_p, s_p = ops.chunk_prefill(*[t.to(dev) for t in (q, k, v, g, beta, s0)])
    _check(o, sf, o_ref, s_ref, o_p, s_p, f"T1141 HV32, {segments} segments")


def test_twolevel_varlen_8_sequences(ops, dev):
    lib = capi.lib()
    q, k, v, g, beta, s0, cu = gc.varlen_inputs()
    o, sf = run_twolevel(lib, dev, q, k, v, g, beta, s0, cu, 4)
    o_ref, s_ref = orc.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, s0, dtype=torch.float64)
    o_p, s_p = ops.chunk_prefill(*[t.to(dev) for t in (q, k, v, g, beta, s0)],
                                 cu_seqlens=cu.to(dev))
    _check(o, sf, o_ref, s_ref, o_p, s_p, "varlen 8 sequences, 4 segments")


def test_twolevel_edges(ops, dev):
    """Empty, single-token and one-chunk sequences (one segment each) beside
    longer ones; the empty sequence's state passes through."""
    lib = capi.lib()
    lens = torch.tensor([0, 1, 64, 65, 200, 130])
    q, k, v, g, beta, s0, cu = gc.varlen_inputs(lens)
    o, sf = run_twolevel(lib, dev, q, k, v, g, beta, s0, cu, 3)
    o_ref, s_ref = orc.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, s0, dtype=torch.float64)
    o_p, s_p = ops.chunk_prefill(*[t.to(dev) for t in (q, k, v, g, beta, s0)],
                                 cu_seqlens=cu.to(dev))
    _check(o, sf, o_ref, s_ref, o_p, s_p, "varlen edges, 3 segments")
    assert torch.equal(sf[0].cpu(), s0[0].float())
