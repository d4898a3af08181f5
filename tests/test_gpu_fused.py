"""GPU parity of the fused prefill (deltanet_chunk_prefill_fused through the
torch op chunk_prefill_fused): raw q/k/v and gate inputs in, o and the
in-place final state out, against the CPU oracle of the reference
TensorRT adapter's step (gdnChunkPrefillSm87.cu:189-316), computed in fp64
on the same inputs.  Bars as for the prefill: max |err| <= 2e-2 on o and on
the final state, and the reference harness's row-cos / max-rel bar.  The
fused path is also compared with the unfused one fed the adapter's
preprocessing done by torch on the GPU.
"""
import pytest
import torch

import gdn_cases as gc
from oracle import gdn_oracle as orc

pytestmark = pytest.mark.gpu


def _fused(ops, dev, q, k, v, a, b, A_log, dt_bias, s0, tag, ref_bar=True):
    print(f"[fused] {tag} q={tuple(q.shape)} v={tuple(v.shape)} {q.dtype}", flush=True)
    st = s0.to(dev).contiguous()
    o = ops.chunk_prefill_fused(*[t.to(dev) for t in (q, k, v, a, b, A_log, dt_bias)], st)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.fused_prefill(q, k, v, a, b, A_log, dt_bias, s0, dtype=torch.float64)
    assert o.dtype == q.dtype and o.shape == v.shape
    mo, ms = gc.parity(o, o_ref), gc.parity(st, s_ref)
    print(f"    o: {gc.fmt(mo)}\n    S: {gc.fmt(ms)}", flush=True)
    gc.assert_abs(mo, what=f"{tag} o")
    gc.assert_abs(ms, what=f"{tag} state")
    if ref_bar:
        gc.assert_ref_bar(mo, what=f"{tag} o")
        gc.assert_ref_bar(ms, what=f"{tag} state")
    return o, st


def test_fused_fp16_T1141_HV32(ops, dev):
    """The plugin's shape and dtypes: B1 T1141 HK16 HV32, fp16 I/O."""
    _fused(ops, dev, *gc.fused_inputs(20, B=1, T=1141, HK=16, HV=32), tag="fp16 T1141 HV32")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 65, 150])
def test_fused_small(ops, dev, dtype, T):
    _fused(ops, dev, *gc.fused_inputs(21 + T, B=2, T=T, HK=2, HV=4, dtype=dtype),
           tag=f"{dtype} B2 T{T}", ref_bar=T > 1)


def test_fused_batch_gqa(ops, dev):
    """B=2 with the plugin's head layout (HK=16, HV=32) and a ragged tail."""
    _fused(ops, dev, *gc.fused_inputs(24, B=2, T=200, HK=16, HV=32), tag="fp16 B2 T200 HV32")


def test_fused_empty_sequence_keeps_state(ops, dev):
    q, k, v, a, b, A_log, dt_bias, s0 = gc.fused_inputs(22, B=1, T=0, HK=2, HV=4)
    st = s0.to(dev).contiguous()
    o = ops.chunk_prefill_fused(*[t.to(dev) for t in (q, k, v, a, b, A_log, dt_bias)], st)
    torch.cuda.synchronize()
    assert o.shape == v.shape and torch.equal(st.cpu(), s0)


def test_fused_matches_unfused_path(ops, dev):
    """Fused == adapter preprocessing (torch on the GPU) + chunk_prefill, up
    to the last bits of the norm and gate arithmetic (a bf16 rounding of a q
    or k element can flip)."""
    q, k, v, a, b, A_log, dt_bias, s0 = gc.fused_inputs(23, B=1, T=300, HK=4, HV=8)
    d = [t.to(dev) for t in (q, k, v, a, b, A_log, dt_bias, s0)]
    print("[fused] fused vs adapter preprocessing + chunk_prefill, B1 T300 HK4 HV8", flush=True)
    st = d[7].clone()
    o_f = ops.chunk_prefill_fused(*d[:7], st)
    qn = orc.l2norm(d[0].float()).to(torch.bfloat16)
    kn = orc.l2norm(d[1].float()).to(torch.bfloat16)
    g, beta = orc.gdn_gate(d[3], d[4], d[5], d[6])
    o_u, s_u = ops.chunk_prefill(qn, kn, d[2].to(torch.bfloat16), g, beta, d[7])
    torch.cuda.synchronize()
    o_u16 = o_u.to(torch.float16)
    same = (o_f == o_u16).float().mean().item()
    do = (o_f.float() - o_u16.float()).abs().max().item()
    ds = (st - s_u).abs().max().item()
    print(f"    o identical {same * 100:.3f}%  max|do|={do:.3e}  max|dS|={ds:.3e}", flush=True)
    assert same > 0.99 and do < 1e-2 and ds < 1e-3


@pytest.mark.parametrize("varlen", [False, True])
def test_in_kernel_l2norm_matches_normalised_inputs(ops, dev, varlen):
    """chunk_prefill(..., qk_l2norm=True) on raw bf16 q/k == chunk_prefill on
    rows normalised by torch (fp32, eps 1e-6, rounded to bf16), up to the
    last bits of the norm (a bf16 rounding of a q or k element can flip)."""
    gen = torch.Generator().manual_seed(31)
    T, HK, HV = 300, 4, 8
    q = torch.randn(1, T, HK, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, T, HK, 128, generator=gen).to(torch.bfloat16)
    _, _, v, g, beta, s0 = gc.make_gdn_inputs(32, B=1, T=T, HK=HK, HV=HV)
    cu = torch.tensor([0, 120, 121, 300], dtype=torch.int32) if varlen else None
    if varlen:
        s0 = 0.02 * torch.randn(3, HV, 128, 128, generator=gen)
    d = [t.to(dev) for t in (q, k, v, g, beta, s0)]
    kw = {"cu_seqlens": cu.to(dev)} if varlen else {}
    print(f"[l2norm] in-kernel vs torch-normalised, T{T} HK{HK} HV{HV} varlen={varlen}", flush=True)
    o_k, s_k = ops.chunk_prefill(*d, qk_l2norm=True, **kw)
    qn = orc.l2norm(d[0].float()).to(torch.bfloat16)
    kn = orc.l2norm(d[1].float()).to(torch.bfloat16)
    o_t, s_t = ops.chunk_prefill(qn, kn, *d[2:], **kw)
    torch.cuda.synchronize()
    same = (o_k == o_t).float().mean().item()
    do = (o_k.float() - o_t.float()).abs().max().item()
    ds = (s_k - s_t).abs().max().item()
    print(f"    o identical {same * 100:.3f}%  max|do|={do:.3e}  max|dS|={ds:.3e}", flush=True)
    assert same > 0.99 and do < 1e-2 and ds < 1e-3
