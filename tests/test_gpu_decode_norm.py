"""GPU parity of the recurrent decode step and the gated RMSNorm."""
import pytest
import torch

import gdn_cases as gc
from oracle import gdn_oracle as orc

pytestmark = pytest.mark.gpu


def _decode_check(ops, dev, q, k, v, g, beta, s0, tag):
    print(f"[decode] {tag} q={tuple(q.shape)} v={tuple(v.shape)}", flush=True)
    state = s0.to(dev).clone()
    o = ops.recurrent_step(q.to(dev), k.to(dev), v.to(dev), g.to(dev), beta.to(dev), state)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    mo, ms = gc.parity(o, o_ref), gc.parity(state, s_ref)
    print(f"    o: {gc.fmt(mo)}\n    S: {gc.fmt(ms)}", flush=True)
    gc.assert_abs(mo, what=f"{tag} o")
    gc.assert_abs(ms, what=f"{tag} state")
    gc.assert_ref_bar(mo, what=f"{tag} o")
    gc.assert_ref_bar(ms, what=f"{tag} state")
    return o, state


def test_decode_B64_HV32(ops, dev):
    """B64 T1 HV32 HK16 d128, fp32 state updated in place."""
    _decode_check(ops, dev, *gc.decode_inputs(), tag="decode B64 HV32")


@pytest.mark.parametrize("T", [2, 5])
@pytest.mark.parametrize("hk,hv", [(2, 4), (4, 4)])
def test_multi_token(ops, dev, T, hk, hv):
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(40 + T + hk, B=3, T=T, HK=hk, HV=hv, s0_scale=0.5)
    _decode_check(ops, dev, q, k, v, g, beta, s0, tag=f"T{T} hk{hk} hv{hv}")


@pytest.mark.parametrize("g_shift", [0.0, 4.0])
def test_multi_token_long(ops, dev, g_shift):
    """512 tokens in one call (the kernel's token loop keeps the state in
    registers throughout): no error growth over the steps, with fast and with
    slow decay."""
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(77 + int(g_shift), B=4, T=512, HK=2, HV=4,
                                              g_shift=g_shift, s0_scale=0.5)
    _decode_check(ops, dev, q, k, v, g, beta, s0, tag=f"T512 g+{g_shift:g}")


def test_decode_matches_prefill_t1(ops, dev):
    """A T=1 prefill and a decode step compute the same token."""
    q, k, v, g, beta, s0 = [t.to(dev) for t in gc.make_gdn_inputs(9, B=4, T=1, HK=2, HV=4)]
    o_p, s_p = ops.chunk_prefill(q, k, v, g, beta, s0)
    st = s0.clone()
    o_d = ops.recurrent_step(q, k, v, g, beta, st)
    assert (o_p.float() - o_d.float()).abs().max().item() < 2e-3
    assert (s_p - st).abs().max().item() < 2e-3


def _norm_check(ops, dev, x, z, w, eps, tag):
    print(f"[rmsnorm] {tag} x={tuple(x.shape)} {x.dtype} w={w.dtype}", flush=True)
    y = ops.gated_rmsnorm(x.to(dev), z.to(dev), w.to(dev), eps)
    torch.cuda.synchronize()
    y_ref = orc.gated_rmsnorm(x, z, w, eps)
    y = y.cpu()
    exact = (y == y_ref).float().mean().item()
    d = (y.float() - y_ref.float()).abs()
    # The GPU and CPU differ only in fp32 summation order and exp/sqrt last
    # bits, which can flip one of the three roundings (n, w*n, y).  A flip in
    # n moves y by ulp(n)|w||silu z|, so bound by one rounding step of each
    # stage at its own magnitude (2^-8 relative for bf16, 2^-11 for fp16).
    u = 2 ** -8 if x.dtype == torch.bfloat16 else 2 ** -11
    xf, zf = x.float(), z.float()
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    stage = (w.float() * n * torch.nn.functional.silu(zf)).abs()
    bound = 2 * u * (2 * stage + y_ref.float().abs()) + 1e-6
    print(f"    bitwise={exact * 100:.4f}% max_abs={d.max().item():.3e} "
          f"cos={gc.row_cos_min(y, y_ref):.8f}", flush=True)
    assert not torch.isnan(y).any()
    assert (d <= bound).all(), "more than one rounding step per stage off"
    assert exact >= 0.999
    return y


def test_gated_rmsnorm_1141x32(ops, dev):
    """rows 1141x32, d128, bf16 o/z/w, eps 1e-6 (HF Qwen3_5RMSNormGated rounding)."""
    _norm_check(ops, dev, *gc.rmsnorm_inputs(), tag="rmsnorm 1141x32x128")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wdt", ["io", "fp32"])
@pytest.mark.parametrize("dv", [64, 128, 256, 512])
def test_rmsnorm_variants(ops, dev, dtype, wdt, dv):
    gen = torch.Generator().manual_seed(dv)
    x = torch.randn(37, 3, dv, generator=gen).to(dtype)
    z = torch.randn(37, 3, dv, generator=gen).to(dtype)
    w = 1 + 0.1 * torch.randn(dv, generator=gen)
    w = w.to(dtype) if wdt == "io" else w
    _norm_check(ops, dev, x, z, w, 1e-6, tag=f"{dtype} w={wdt} dv={dv}")


def test_decode_in_kernel_l2norm_matches_normalised_inputs(ops, dev):
    """recurrent_step(..., qk_l2norm=True) on raw bf16 q/k == recurrent_step
    on rows normalised by torch (fp32, eps 1e-6, rounded to bf16), up to the
    last bits of the norm."""
    gen = torch.Generator().manual_seed(41)
    B, T, HK, HV = 4, 3, 2, 4
    q = torch.randn(B, T, HK, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, T, HK, 128, generator=gen).to(torch.bfloat16)
    _, _, v, g, beta, s0 = gc.make_gdn_inputs(42, B=B, T=T, HK=HK, HV=HV)
    d = [t.to(dev) for t in (q, k, v, g, beta)]
    print(f"[decode] in-kernel l2norm B{B} T{T} HK{HK} HV{HV}", flush=True)
    st_k, st_t = s0.to(dev), s0.to(dev)
    o_k = ops.recurrent_step(*d, st_k, qk_l2norm=True)
    qn = orc.l2norm(d[0].float()).to(torch.bfloat16)
    kn = orc.l2norm(d[1].float()).to(torch.bfloat16)
    o_t = ops.recurrent_step(qn, kn, *d[2:], st_t)
    torch.cuda.synchronize()
    same = (o_k == o_t).float().mean().item()
    do = (o_k.float() - o_t.float()).abs().max().item()
    ds = (st_k - st_t).abs().max().item()
    print(f"    o identical {same * 100:.3f}%  max|do|={do:.3e}  max|dS|={ds:.3e}", flush=True)
    assert same > 0.99 and do < 1e-2 and ds < 1e-3
