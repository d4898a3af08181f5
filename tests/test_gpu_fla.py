"""GPU parity of the fla adapter against transformers' own torch fallback
(models/qwen3_5/modeling_qwen3_5.py:249-327 chunked, 331-380 recurrent), with
the inputs a Qwen3.5 layer builds (modeling_qwen3_5.py:494-499): raw q/k
normalised in the op, GQA heads expanded by repeat_interleave,
g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b).  The reference
runs in fp32 on the same (bf16-valued) inputs.  Bar: max |err| <= 2e-2 on o
and on the final state, plus tensor l2-relative error < 1e-2.
"""
import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import gdn_cases as gc

pytestmark = pytest.mark.gpu

HF_DIR = Path(__file__).resolve().parent.parent / "qwen-drive-edge-orin_amd" / "hf"


@pytest.fixture(scope="module")
def fla_ops(ops):
    import importlib

    before = set(sys.modules)
    sys.path.insert(0, str(HF_DIR))
    try:
        m = importlib.import_module("fla.ops.gated_delta_rule")
    finally:
        sys.path.remove(str(HF_DIR))
        for name in set(sys.modules) - before:
            if name == "fla" or name.startswith("fla."):
                del sys.modules[name]
    return m


@pytest.fixture(scope="module")
def torch_ref():
    import transformers.models.qwen3_5.modeling_qwen3_5 as mq

    chunk = getattr(mq.torch_chunk_gated_delta_rule, "__wrapped__", mq.torch_chunk_gated_delta_rule)
    rec = getattr(mq.torch_recurrent_gated_delta_rule, "__wrapped__",
                  mq.torch_recurrent_gated_delta_rule)
    return chunk, rec


def _layer_inputs(B, T, HK, HV, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, HK, 128, generator=gen).bfloat16()
    k = torch.randn(B, T, HK, 128, generator=gen).bfloat16()
    v = torch.randn(B, T, HV, 128, generator=gen).bfloat16()
    a = torch.randn(B, T, HV, generator=gen).bfloat16()
    b = torch.randn(B, T, HV, generator=gen).bfloat16()
    A_log = torch.rand(HV, generator=gen) * 2 - 1
    dt_bias = torch.randn(HV, generator=gen) * 0.5
    beta = b.sigmoid()
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
    rep = HV // HK
    q, k = q.repeat_interleave(rep, dim=2), k.repeat_interleave(rep, dim=2)
    s0 = torch.randn(B, HV, 128, 128, generator=gen) * 0.02
    return q, k, v, g, beta, s0


def _check(o, o_ref, s, s_ref, tag):
    """max |err| <= 2e-2 and tensor l2-relative error < 1e-2.  Per-row cosine is
    printed, not asserted: the layer's gates decay up to e^-8 per token, so
    some output rows are 1e-4-sized remainders whose direction bf16/fp16
    rounding moves by more than the 0.999 row bar meant for the reference
    harness's mild gates (those cases are asserted in test_gpu_prefill.py)."""
    o, s = o.float().cpu(), s.float().cpu()
    mo, ms = gc.parity(o, o_ref.float()), gc.parity(s, s_ref.float())
    rn = o_ref.float().flatten(0, -2).norm(dim=-1)
    print(f"[fla] {tag}\n    o: {gc.fmt(mo)} (row norms {rn.min():.2e}..{rn.max():.2e})"
          f"\n    S: {gc.fmt(ms)}", flush=True)
    gc.assert_abs(mo, what=f"{tag} o")
    gc.assert_abs(ms, what=f"{tag} state")
    assert mo["l2_rel"] < 1e-2 and ms["l2_rel"] < 1e-2, f"{tag}: {gc.fmt(mo)} | {gc.fmt(ms)}"


@pytest.mark.parametrize("B,T,HK,HV", [(1, 150, 2, 4), (2, 64, 1, 2), (1, 1141, 2, 4),
                                       (1, 1141, 16, 32), (2, 300, 16, 32)])
def test_chunk_matches_transformers(fla_ops, torch_ref, dev, B, T, HK, HV):
    """(1, 1141, 16, 32) is the planner's layer: 16 k-heads expanded to the 32
    v-heads before the call (modeling_qwen3_5.py:500-502), as transformers
    hands them to fla.  (2, 300, 16, 32) has more (sequence, head) pairs than
    one 16-column scan group per CU covers, so it runs the paired scan's
    raw-bf16 instance."""
    q, k, v, g, beta, s0 = _layer_inputs(B, T, HK, HV, seed=T + HV)
    o_ref, s_ref = torch_ref[0](q.float(), k.float(), v.float(), g, beta, initial_state=s0,
                                output_final_state=True, use_qk_l2norm_in_kernel=True)
    args = [t.to(dev) for t in (q, k, v, g, beta)]
    o, s = fla_ops.chunk_gated_delta_rule(*args, initial_state=s0.to(dev), output_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16 and o.shape == v.shape
    _check(o, o_ref, s, s_ref, f"chunk B{B} T{T} HK{HK} HV{HV}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_output_dtype_follows_input(fla_ops, torch_ref, dev, dtype):
    """fp16 / fp32 layers: o comes back in q's dtype, as transformers' fallback
    returns it (.to(initial_dtype)), with the same values as the bf16 path."""
    q, k, v, g, beta, s0 = _layer_inputs(1, 150, 2, 4, seed=21)
    o_ref, s_ref = torch_ref[0](q.float(), k.float(), v.float(), g, beta, initial_state=s0,
                                output_final_state=True, use_qk_l2norm_in_kernel=True)
    args = [t.to(dev, dtype) for t in (q, k, v)] + [t.to(dev) for t in (g, beta)]
    o, s = fla_ops.chunk_gated_delta_rule(*args, initial_state=s0.to(dev), output_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert o.dtype == dtype and o.shape == v.shape
    _check(o, o_ref, s, s_ref, f"chunk {dtype}")
    o1, s1 = fla_ops.recurrent_gated_delta_rule(*[t[:, :1] for t in args], initial_state=s0.to(dev),
                                                output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    assert o1.dtype == dtype


def test_chunk_varlen_matches_per_sequence(fla_ops, torch_ref, dev):
    lens = [70, 1, 129]
    q, k, v, g, beta, _ = _layer_inputs(1, sum(lens), 2, 4, seed=3)
    s0 = torch.randn(len(lens), 4, 128, 128) * 0.02
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    o, s = fla_ops.chunk_gated_delta_rule(*[t.to(dev) for t in (q, k, v, g, beta)],
                                          initial_state=s0.to(dev), output_final_state=True,
                                          use_qk_l2norm_in_kernel=True, cu_seqlens=cu.to(dev))
    torch.cuda.synchronize()
    for i in range(len(lens)):
        a, b = int(cu[i]), int(cu[i + 1])
        o_ref, s_ref = torch_ref[0](q[:, a:b].float(), k[:, a:b].float(), v[:, a:b].float(),
                                    g[:, a:b], beta[:, a:b],
                                    initial_state=s0[i:i + 1], output_final_state=True,
                                    use_qk_l2norm_in_kernel=True)
        _check(o[:, a:b], o_ref, s[i:i + 1], s_ref, f"varlen seq {i} (T={b - a})")


@pytest.mark.parametrize("T", [1, 3])
def test_recurrent_matches_transformers(fla_ops, torch_ref, dev, T):
    q, k, v, g, beta, s0 = _layer_inputs(4, T, 2, 4, seed=11 + T)
    o_ref, s_ref = torch_ref[1](q.float(), k.float(), v.float(), g, beta, initial_state=s0,
                                output_final_state=True, use_qk_l2norm_in_kernel=True)
    s0d = s0.to(dev)
    o, s = fla_ops.recurrent_gated_delta_rule(*[t.to(dev) for t in (q, k, v, g, beta)],
                                              initial_state=s0d, output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert torch.equal(s0d.cpu(), s0), "initial_state must not be modified"
    _check(o, o_ref, s, s_ref, f"recurrent T{T}")


def test_scale_and_shape_checks(fla_ops, torch_ref, dev):
    q, k, v, g, beta, s0 = _layer_inputs(1, 80, 2, 2, seed=5)
    # an explicit scale on l2-normalised q/k (the kernels' operand range
    # assumes |k| of order 1, as l2-normalised or the reference harness's
    # randn/8 inputs are)
    sc = 0.05
    qn, kn = fla_ops._l2norm(q), fla_ops._l2norm(k)
    o_ref, s_ref = torch_ref[0](qn * (sc * 128 ** 0.5), kn, v.float(), g, beta,
                                initial_state=s0, output_final_state=True)
    o, s = fla_ops.chunk_gated_delta_rule(*[t.to(dev) for t in (q, k, v, g, beta)], scale=sc,
                                          initial_state=s0.to(dev), output_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    _check(o, o_ref, s, s_ref, "scale 0.05")
    o2, s2 = fla_ops.chunk_gated_delta_rule(*[t.to(dev) for t in (q, k, v, g, beta)])
    assert s2 is None and o2.shape == v.shape
    with pytest.raises(NotImplementedError):
        fla_ops.chunk_gated_delta_rule(*[t[..., :64].contiguous().to(dev) if t.dim() == 4 else t.to(dev)
                                         for t in (q, k, v, g, beta)])
