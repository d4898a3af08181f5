"""GPU parity of the causal conv1d ops (gdn_causal_conv1d_fwd / _update
through the torch extension and the transformers adapter) against the CPU
oracle, which reproduces transformers' torch functions bit for bit
(models/qwen3_5/modeling_qwen3_5.py:199-240).

Bar: without activation the outputs are bit-identical (same fp32 fused
multiply-add order, same roundings).  With SiLU, the device expf may differ
from the host's by an fp32 unit, so an output may differ by one unit of the
I/O dtype in rare elements: every element within 1 ulp of the I/O dtype and
at most 1e-3 of them different.  The carried state is bit-identical.
Shapes follow a Qwen3.5 layer with 16 key heads and 32 value heads of 128:
conv channels D = 2 * 16 * 128 + 32 * 128 = 8192, kernel size 4.
"""
import sys
from pathlib import Path

import pytest
import torch

from oracle import gdn_oracle as orc

pytestmark = pytest.mark.gpu

HF_DIR = Path(__file__).resolve().parent.parent / "qwen-drive-edge-orin_amd" / "hf"
D_QWEN = 8192


def _ulps(a, r, io):
    mant = 7 if io == torch.bfloat16 else 10
    a, r = a.float(), r.float()
    unit = torch.maximum(a.abs(), r.abs()).clamp_min(1e-30) * 2.0 ** -mant
    return ((a - r).abs() / unit)


def _check(y, ref, act, tag):
    y = y.cpu()
    assert y.shape == ref.shape and y.dtype == ref.dtype
    n_diff = (y != ref).sum().item()
    print(f"{tag}: {n_diff} of {ref.numel()} differ", flush=True)
    if act is None:
        assert n_diff == 0, tag
    else:
        assert _ulps(y, ref, ref.dtype).max().item() <= 1.0, tag
        assert n_diff <= 1e-3 * ref.numel(), tag


def _inputs(seed, B, T, D, K, io, wd, transposed=True):
    gen = torch.Generator().manual_seed(seed)
    if transposed:   # the view transformers hands over: [B, T, D] buffer, [B, D, T] view
        x = torch.randn(B, T, D, generator=gen).to(io).transpose(1, 2)
    else:
        x = torch.randn(B, D, T, generator=gen).to(io)
    w = (0.5 * torch.randn(D, K, generator=gen)).to(wd)
    bias = (0.1 * torch.randn(D, generator=gen)).to(wd)
    return x, w, bias


@pytest.mark.parametrize("T", [1, 3, 64, 1141])
def test_fwd_qwen_shape(ops, dev, T):
    x, w, _ = _inputs(T, 1, T, D_QWEN, 4, torch.bfloat16, torch.bfloat16)
    ref = orc.causal_conv1d(x, w, None, "silu")
    print(f"fwd B=1 T={T} D={D_QWEN} K=4 bf16 silu", flush=True)
    y = ops.causal_conv1d_fwd(x.to(dev), w.to(dev), None, True)
    torch.cuda.synchronize()
    assert y.transpose(1, 2).is_contiguous()
    _check(y, ref, "silu", f"fwd T={T}")


# Lengths at D = 8192 (4 channel tiles) that give, on a 256-CU device, runs
# of ceil(T / 64) tokens in one round up to T = 1536 (40 .. 1500: runs 1, 2,
# 3, 4, 5, 6, 8, 10, 11, 15, 18, 20, 21, 24, i.e. every slot count of that
# launch, with and without a slot past the run), ceil(T / 128) in two rounds
# up to 3072 (1600, 2048, 3000) and the many-rounds launch past that (3100).
RUN_LENGTHS = [40, 100, 150, 250, 300, 380, 500, 600, 700, 900, 1141, 1250, 1300, 1500, 1600,
               2048, 3000, 3100]


@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
def test_fwd_run_lengths(ops, dev, io):
    """Every launch shape of the K = 4 prefill at the Qwen3.5 width: without
    activation bit-identical to the oracle, with a bias; with SiLU at the
    tolerance above."""
    for T in RUN_LENGTHS:
        x, w, bias = _inputs(T + 1, 1, T, D_QWEN, 4, io, io)
        xd, wd_, bd = x.to(dev), w.to(dev), bias.to(dev)
        print(f"fwd run lengths T={T} {io}", flush=True)
        y = ops.causal_conv1d_fwd(xd, wd_, bd, False)
        torch.cuda.synchronize()
        _check(y, orc.causal_conv1d(x, w, bias, None), None, f"fwd T={T} {io} bias")
        y = ops.causal_conv1d_fwd(xd, wd_, None, True)
        torch.cuda.synchronize()
        _check(y, orc.causal_conv1d(x, w, None, "silu"), "silu", f"fwd T={T} {io} silu")


def test_fwd_run_lengths_batch_and_partial_tile(ops, dev):
    """Batches (B = 2, 5) and a width with a partial last channel tile
    (D = 2048 + 264), so that runs, batches and channel tiles share the
    grid, bit-identical to the oracle."""
    for B, T, D in [(2, 1141, D_QWEN), (5, 300, D_QWEN), (3, 700, 2312), (2, 2000, 2312)]:
        x, w, bias = _inputs(B * T, B, T, D, 4, torch.bfloat16, torch.bfloat16)
        print(f"fwd B={B} T={T} D={D}", flush=True)
        y = ops.causal_conv1d_fwd(x.to(dev), w.to(dev), bias.to(dev), False)
        torch.cuda.synchronize()
        _check(y, orc.causal_conv1d(x, w, bias, None), None, f"fwd B={B} T={T} D={D}")


@pytest.mark.parametrize("io,wd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.bfloat16, torch.float32), (torch.float16, torch.float32)])
@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("act", [None, "silu"])
def test_fwd_dtypes_taps_bias(ops, dev, io, wd, K, act):
    x, w, bias = _inputs(K, 3, 77, 264, K, io, wd)
    for bb in (None, bias):
        ref = orc.causal_conv1d(x, w, bb, act)
        print(f"fwd B=3 T=77 D=264 K={K} {io} w={wd} act={act} bias={bb is not None}", flush=True)
        y = ops.causal_conv1d_fwd(x.to(dev), w.to(dev), None if bb is None else bb.to(dev),
                                  act is not None)
        torch.cuda.synchronize()
        _check(y, ref, act, f"fwd K={K} {io} {wd} {act}")


def test_fwd_layouts(ops, dev):
    # contiguous [B, D, T] input (copied into the channel-contiguous layout)
    # and a channel slice of a wider buffer (strided rows, used in place)
    x, w, bias = _inputs(5, 2, 50, 128, 4, torch.bfloat16, torch.bfloat16, transposed=False)
    ref = orc.causal_conv1d(x, w, bias, None)
    print("fwd contiguous [B, D, T]", flush=True)
    y = ops.causal_conv1d_fwd(x.to(dev), w.to(dev), bias.to(dev), False)
    torch.cuda.synchronize()
    _check(y, ref, None, "fwd contiguous BDT")
    wide = torch.randn(2, 50, 384, generator=torch.Generator().manual_seed(6)).bfloat16()
    xs = wide[:, :, 128:256].transpose(1, 2)
    ref = orc.causal_conv1d(xs, w, bias, "silu")
    print("fwd channel slice of a wider [B, T, 384] buffer", flush=True)
    y = ops.causal_conv1d_fwd(wide.to(dev)[:, :, 128:256].transpose(1, 2), w.to(dev),
                              bias.to(dev), True)
    torch.cuda.synchronize()
    _check(y, ref, "silu", "fwd slice")


@pytest.mark.parametrize("B,T,L", [(1, 1, 4), (4, 1, 4), (2, 2, 4), (2, 1, 3), (2, 5, 6)])
def test_update_matches_oracle(ops, dev, B, T, L):
    gen = torch.Generator().manual_seed(100 * B + 10 * T + L)
    x = torch.randn(B, T, D_QWEN, generator=gen).bfloat16().transpose(1, 2)
    st = torch.randn(B, D_QWEN, L, generator=gen).bfloat16()
    w = (0.5 * torch.randn(D_QWEN, 4, generator=gen)).bfloat16()
    ref, ref_st = orc.causal_conv1d_update(x, st, w, None, "silu")
    print(f"update B={B} T={T} L={L} D={D_QWEN}", flush=True)
    st_d = st.to(dev)
    y = ops.causal_conv1d_update(x.to(dev), st_d, w.to(dev), None, True)
    torch.cuda.synchronize()
    _check(y, ref, "silu", f"update B={B} T={T} L={L}")
    assert torch.equal(st_d.cpu(), ref_st)


@pytest.mark.parametrize("io,wd", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                   (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("T", [1, 3])
def test_update_vector_path_dtypes_and_bias(ops, dev, io, wd, T):
    """The 4-channel update path (K = 4, 4-token state rows) with every
    weight dtype, a bias and B > 1, against the oracle."""
    gen = torch.Generator().manual_seed(7 + T)
    B, D = 3, 1024
    x = torch.randn(B, T, D, generator=gen).to(io).transpose(1, 2)
    st = torch.randn(B, D, 4, generator=gen).to(io)
    w = (0.5 * torch.randn(D, 4, generator=gen)).to(wd)
    bias = (0.1 * torch.randn(D, generator=gen)).to(wd)
    for act in (None, "silu"):
        ref, ref_st = orc.causal_conv1d_update(x, st, w, bias, act)
        print(f"update4 B={B} T={T} D={D} {io} w={wd} act={act}", flush=True)
        st_d = st.to(dev)
        y = ops.causal_conv1d_update(x.to(dev), st_d, w.to(dev), bias.to(dev), act is not None)
        torch.cuda.synchronize()
        _check(y, ref, act, f"update4 {io} {wd} {act} T={T}")
        assert torch.equal(st_d.cpu(), ref_st)


def test_prefill_then_decode_chain(ops, dev):
    """Prefill 40 tokens, then 6 single-token updates from the state the
    prefill leaves: the outputs equal one pass over all 46 tokens."""
    x, w, bias = _inputs(9, 2, 46, 512, 4, torch.bfloat16, torch.bfloat16)
    full = orc.causal_conv1d(x, w, bias, None)
    xd, wd_, bd = x.to(dev), w.to(dev), bias.to(dev)
    print("prefill 40 + 6 updates, B=2 D=512", flush=True)
    outs = [ops.causal_conv1d_fwd(xd[:, :, :40], wd_, bd, False)]
    state = xd[:, :, 36:40].contiguous()
    for t in range(40, 46):
        outs.append(ops.causal_conv1d_update(xd[:, :, t:t + 1], state, wd_, bd, False))
    torch.cuda.synchronize()
    _check(torch.cat([o.cpu() for o in outs], dim=-1), full, None, "chain")
    assert torch.equal(state.cpu(), x[:, :, 42:46])


def test_adapter_matches_transformers_fallback(ops, dev):
    """The adapter as transformers calls it (transposed in_proj output,
    weight squeezed from nn.Conv1d's [D, 1, K], no bias, 'silu') against the
    undecorated transformers functions run on the host."""
    import importlib

    import transformers.models.qwen3_5.modeling_qwen3_5 as mq

    fn = getattr(mq.causal_conv1d_fn, "__wrapped__", mq.causal_conv1d_fn)
    up = getattr(mq.causal_conv1d_update, "__wrapped__", mq.causal_conv1d_update)
    before = set(sys.modules)
    sys.path.insert(0, str(HF_DIR))
    try:
        ad = importlib.import_module("causal_conv1d")
    finally:
        sys.path.remove(str(HF_DIR))
        for name in set(sys.modules) - before:
            if name == "causal_conv1d" or name.startswith("causal_conv1d."):
                del sys.modules[name]
    gen = torch.Generator().manual_seed(11)
    mixed = torch.randn(1, 300, D_QWEN, generator=gen).bfloat16()
    w3 = (0.5 * torch.randn(D_QWEN, 1, 4, generator=gen)).bfloat16()
    ref = fn(mixed.transpose(1, 2), w3.squeeze(1), None, activation="silu")
    print("adapter fwd T=300", flush=True)
    y = ad.causal_conv1d_fn(mixed.to(dev).transpose(1, 2), w3.to(dev).squeeze(1), None,
                            activation="silu")
    torch.cuda.synchronize()
    _check(y, ref, "silu", "adapter fwd")
    st = torch.randn(1, D_QWEN, 4, generator=gen).bfloat16()
    tok = torch.randn(1, 1, D_QWEN, generator=gen).bfloat16()
    st_ref = st.clone()
    ref = up(tok.transpose(1, 2), st_ref, w3.squeeze(1), None, "silu")
    print("adapter update", flush=True)
    st_d = st.to(dev)
    y = ad.causal_conv1d_update(tok.to(dev).transpose(1, 2), st_d, w3.to(dev).squeeze(1), None,
                                "silu")
    torch.cuda.synchronize()
    _check(y, ref, "silu", "adapter update")
    assert torch.equal(st_d.cpu(), st_ref)
