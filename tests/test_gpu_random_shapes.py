"""Seeded random shapes against the CPU oracle: the chunked prefill (fixed
length and packed batches, GQA ratios 1/2/4, with and without an initial
state, so that both scan instances and every chunk-tail case come up), the
recurrent decode step (batch, tokens per call, GQA ratio, state scale and
gate range), the fused raw-input prefill (gate pre-op and in-kernel q/k norm; fp16 and
bf16 I/O), the causal conv1d prefill (widths with partial channel tiles,
K = 2..4, both I/O dtypes, bias, both launch regimes), the conv1d decode
update (the 4-channel vector path and the per-channel path: state lengths
K-1..8, several tokens per call) and the gated RMSNorm (row counts, head
widths, dtypes, fp32 or I/O-dtype weights).  The cases are drawn once from a
fixed seed; each prints its shape before it runs.

Bars as in test_gpu_prefill.py and test_gpu_decode_norm.py (max |err| <= 2e-2
on o and the final state, the reference harness's random-case bar; the
RMSNorm within one rounding step per stage, >= 99.9 % bitwise) and
test_gpu_conv.py (bit-identical without activation; with SiLU every element
within 1 ulp and at most 1e-3 of them different; the carried state
bit-identical).
"""
import pytest
import torch

import gdn_cases as gc
from oracle import gdn_oracle as orc
from test_gpu_decode_norm import _decode_check, _norm_check
from test_gpu_fused import _fused

pytestmark = pytest.mark.gpu


def _prefill_cases(n=16, seed=2024):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    cases = []
    for i in range(n):
        hk = pick([1, 2, 4, 8, 16])
        hv = hk * pick([1, 2, 4])
        if hv > 32:
            hv = hk
        varlen = i % 2 == 1
        if varlen:
            nseq = int(torch.randint(1, 13, (1,), generator=gen))
            lens = torch.randint(0, 400, (nseq,), generator=gen)
            lens[0] = max(int(lens[0]), 1)
            cases.append(dict(seed=100 + i, varlen=True, lens=lens.tolist(), hk=hk, hv=hv,
                              s0=pick([True, False]), g_shift=pick([0.0, 2.0])))
        else:
            cases.append(dict(seed=100 + i, varlen=False, B=int(torch.randint(1, 4, (1,), generator=gen)),
                              T=int(torch.randint(1, 600, (1,), generator=gen)), hk=hk, hv=hv,
                              s0=pick([True, False]), g_shift=pick([0.0, 2.0])))
    return cases


PREFILL_CASES = _prefill_cases()


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[f"p{i}" for i in range(len(PREFILL_CASES))])
def test_prefill_random_shape(ops, dev, case):
    if case["varlen"]:
        lens = torch.tensor(case["lens"])
        total = int(lens.sum())
        q, k, v, g, beta, s0 = gc.make_gdn_inputs(case["seed"], B=1, T=total, HK=case["hk"],
                                                  HV=case["hv"], g_shift=case["g_shift"],
                                                  n_states=len(lens), with_s0=case["s0"])
        cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(lens, 0)
        print(f"[random prefill] varlen lens={case['lens']} HK={case['hk']} HV={case['hv']} "
              f"s0={case['s0']} g_shift={case['g_shift']}", flush=True)
        args = [t.to(dev) if t is not None else None for t in (q, k, v, g, beta, s0)]
        o, sf = ops.chunk_prefill(*args, cu_seqlens=cu.to(dev))
        o_ref, s_ref = orc.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, s0,
                                                         dtype=torch.float64)
    else:
        q, k, v, g, beta, s0 = gc.make_gdn_inputs(case["seed"], B=case["B"], T=case["T"],
                                                  HK=case["hk"], HV=case["hv"],
                                                  g_shift=case["g_shift"], with_s0=case["s0"])
        print(f"[random prefill] B={case['B']} T={case['T']} HK={case['hk']} HV={case['hv']} "
              f"s0={case['s0']} g_shift={case['g_shift']}", flush=True)
        args = [t.to(dev) if t is not None else None for t in (q, k, v, g, beta, s0)]
        o, sf = ops.chunk_prefill(*args)
        o_ref, s_ref = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    torch.cuda.synchronize()
    mo, ms = gc.parity(o, o_ref), gc.parity(sf, s_ref)
    print(f"    o: {gc.fmt(mo)}\n    S: {gc.fmt(ms)}", flush=True)
    gc.assert_abs(mo, what="o")
    gc.assert_abs(ms, what="state")
    gc.assert_ref_bar(mo, what="o")
    gc.assert_ref_bar(ms, what="state")


def _conv_cases(n=10, seed=77):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    return [dict(seed=300 + i, B=int(torch.randint(1, 5, (1,), generator=gen)),
                 T=int(torch.randint(1, 2500, (1,), generator=gen)),
                 D=pick([264, 1032, 2312, 4104, 8192]), K=pick([2, 3, 4]),
                 io=pick([torch.bfloat16, torch.float16]), bias=pick([True, False]))
            for i in range(n)]


CONV_CASES = _conv_cases()


def _ulps(a, r, io):
    mant = 7 if io == torch.bfloat16 else 10
    a, r = a.float(), r.float()
    unit = torch.maximum(a.abs(), r.abs()).clamp_min(1e-30) * 2.0 ** -mant
    return (a - r).abs() / unit


@pytest.mark.parametrize("case", CONV_CASES, ids=[f"c{i}" for i in range(len(CONV_CASES))])
def test_conv_random_shape(ops, dev, case):
    B, T, D, K, io = case["B"], case["T"], case["D"], case["K"], case["io"]
    gen = torch.Generator().manual_seed(case["seed"])
    x = torch.randn(B, T, D, generator=gen).to(io).transpose(1, 2)   # transformers' view
    w = (0.5 * torch.randn(D, K, generator=gen)).to(io)
    bias = (0.1 * torch.randn(D, generator=gen)).to(io) if case["bias"] else None
    xd, wd, bd = x.to(dev), w.to(dev), bias.to(dev) if bias is not None else None
    print(f"[random conv] B={B} T={T} D={D} K={K} {io} bias={case['bias']}", flush=True)
    y = ops.causal_conv1d_fwd(xd, wd, bd, False)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), orc.causal_conv1d(x, w, bias, None))
    y = ops.causal_conv1d_fwd(xd, wd, bd, True)
    torch.cuda.synchronize()
    ref = orc.causal_conv1d(x, w, bias, "silu")
    y = y.cpu()
    n_diff = (y != ref).sum().item()
    assert _ulps(y, ref, io).max().item() <= 1.0
    assert n_diff <= 1e-3 * ref.numel(), n_diff


def _decode_cases(n=8, seed=4242):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    cases = []
    for i in range(n):
        hk = pick([1, 2, 4, 8, 16])
        hv = min(hk * pick([1, 2, 4]), 32)
        hv -= hv % hk
        cases.append(dict(seed=500 + i, B=int(torch.randint(1, 41, (1,), generator=gen)),
                          T=int(torch.randint(1, 9, (1,), generator=gen)), hk=hk, hv=hv,
                          s0_scale=pick([0.02, 0.5]), g_offset=pick([0.0, -1.0]),
                          g_shift=pick([0.0, 2.0])))
    return cases


DECODE_CASES = _decode_cases()


@pytest.mark.parametrize("case", DECODE_CASES, ids=[f"d{i}" for i in range(len(DECODE_CASES))])
def test_decode_random_shape(ops, dev, case):
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(case["seed"], B=case["B"], T=case["T"],
                                              HK=case["hk"], HV=case["hv"],
                                              g_shift=case["g_shift"], g_offset=case["g_offset"],
                                              s0_scale=case["s0_scale"])
    _decode_check(ops, dev, q, k, v, g, beta, s0,
                  tag=f"random B={case['B']} T={case['T']} HK={case['hk']} HV={case['hv']} "
                      f"s0={case['s0_scale']} g_off={case['g_offset']} g_shift={case['g_shift']}")


def _update_cases(n=10, seed=91):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    cases = []
    for i in range(n):
        K = pick([2, 3, 4])
        # every other case on the vector path's shape (K = 4, 4-token state)
        L = 4 if i % 2 == 0 else int(torch.randint(K - 1, 9, (1,), generator=gen))
        cases.append(dict(seed=700 + i, B=int(torch.randint(1, 71, (1,), generator=gen)),
                          T=int(torch.randint(1, 5, (1,), generator=gen)),
                          D=pick([264, 1032, 2312, 8192]), K=4 if i % 2 == 0 else K, L=L,
                          io=pick([torch.bfloat16, torch.float16]), bias=pick([True, False])))
    return cases


UPDATE_CASES = _update_cases()


@pytest.mark.parametrize("case", UPDATE_CASES, ids=[f"u{i}" for i in range(len(UPDATE_CASES))])
def test_conv_update_random_shape(ops, dev, case):
    B, T, D, K, L, io = case["B"], case["T"], case["D"], case["K"], case["L"], case["io"]
    gen = torch.Generator().manual_seed(case["seed"])
    x = torch.randn(B, T, D, generator=gen).to(io).transpose(1, 2)   # transformers' view
    st = torch.randn(B, D, L, generator=gen).to(io)
    w = (0.5 * torch.randn(D, K, generator=gen)).to(io)
    bias = (0.1 * torch.randn(D, generator=gen)).to(io) if case["bias"] else None
    print(f"[random conv update] B={B} T={T} D={D} K={K} L={L} {io} bias={case['bias']}",
          flush=True)
    for act in (None, "silu"):
        ref, ref_st = orc.causal_conv1d_update(x, st, w, bias, act)
        st_d = st.to(dev)
        y = ops.causal_conv1d_update(x.to(dev), st_d, w.to(dev),
                                     bias.to(dev) if bias is not None else None, act is not None)
        torch.cuda.synchronize()
        y = y.cpu()
        assert torch.equal(st_d.cpu(), ref_st)
        if act is None:
            assert torch.equal(y, ref)
        else:
            assert _ulps(y, ref, io).max().item() <= 1.0
            assert (y != ref).sum().item() <= max(1, 1e-3 * ref.numel())


def _norm_cases(n=6, seed=313):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    return [dict(seed=900 + i, rows=int(torch.randint(1, 3000, (1,), generator=gen)),
                 heads=int(torch.randint(1, 9, (1,), generator=gen)), dv=pick([64, 128, 256, 512]),
                 io=pick([torch.bfloat16, torch.float16]), wdt=pick(["io", "fp32"]))
            for i in range(n)]


NORM_CASES = _norm_cases()


@pytest.mark.parametrize("case", NORM_CASES, ids=[f"n{i}" for i in range(len(NORM_CASES))])
def test_gated_rmsnorm_random_shape(ops, dev, case):
    gen = torch.Generator().manual_seed(case["seed"])
    shape = (case["rows"], case["heads"], case["dv"])
    x = torch.randn(*shape, generator=gen).to(case["io"])
    z = torch.randn(*shape, generator=gen).to(case["io"])
    w = 1 + 0.1 * torch.randn(case["dv"], generator=gen)
    w = w.to(case["io"]) if case["wdt"] == "io" else w
    _norm_check(ops, dev, x, z, w, 1e-6, tag=f"random {shape} w={case['wdt']}")


def _fused_cases(n=8, seed=515):
    gen = torch.Generator().manual_seed(seed)

    def pick(seq):
        return seq[int(torch.randint(len(seq), (1,), generator=gen))]

    cases = []
    for i in range(n):
        hk = pick([1, 2, 4, 8, 16])
        hv = min(hk * pick([1, 2, 4]), 32)
        hv -= hv % hk
        cases.append(dict(seed=600 + i, B=int(torch.randint(1, 4, (1,), generator=gen)),
                          T=int(torch.randint(2, 600, (1,), generator=gen)), hk=hk, hv=hv,
                          dtype=pick([torch.float16, torch.bfloat16])))
    return cases


FUSED_CASES = _fused_cases()


@pytest.mark.parametrize("case", FUSED_CASES, ids=[f"f{i}" for i in range(len(FUSED_CASES))])
def test_fused_random_shape(ops, dev, case):
    _fused(ops, dev, *gc.fused_inputs(case["seed"], B=case["B"], T=case["T"], HK=case["hk"],
                                      HV=case["hv"], dtype=case["dtype"]),
           tag=f"random B={case['B']} T={case['T']} HK={case['hk']} HV={case['hv']}")
