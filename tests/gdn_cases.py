"""Seeded inputs and parity metrics shared by the tests, smoke() and bench.py.

Input generators for the five workloads of this path (all CPU
``torch.Generator`` draws, in the order q, k, v, beta, g, state, so the same
tensors can be moved to the GPU and handed to the oracle):

  plumbing_inputs  CPU plumbing      B1 T256 H4 d64 fp32, chunk 64, seed 0
  rmsnorm_inputs   gated RMSNorm     rows 1141x32, d128 bf16, seed 1
  decode_inputs    decode step       B64 T1 HV32 HK16 d128, seed 3
  prefill_inputs   chunked prefill   B1 T1141 HV32 HK16 d128, seed 4
  varlen_inputs    varlen prefill    8 sequences, lengths from seed 7, seed 5 for tensors

``make_reference_inputs`` restates the reference harness's random grid
(kernels/harness/parity_test.py:102-121) on a CPU generator.

Metrics restate kernels/harness/parity_test.py:124-153 (row_cos_min,
max_rel with denominator floor 0.1, tensor_l2_rel) plus max/mean absolute
error, the bar these kernels are held to (max |err| <= 2e-2 on o and state).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

ABS_TOL = 2e-2          # max |err| bar on o and final state (fp32-accumulated bf16)
REF_COS_MIN = 0.999     # reference harness random-case bar (parity_test.py:188-189)
REF_REL_MAX = 1e-2

VARLEN_LENGTHS_SEED = 7


def l2norm(x, eps=1e-6):
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def make_gdn_inputs(seed, B, T, HK, HV, D=128, g_shift=0.0, g_offset=0.0, s0_scale=0.02,
                    with_s0=True, n_states=None):
    """l2-normalised bf16 q/k, bf16 v, sigmoid beta, logsigmoid g (the
    production value domain: gdnChunkPrefillSm87.cu:113-125)."""
    gen = _gen(seed)
    q = l2norm(torch.randn(B, T, HK, D, generator=gen)).to(torch.bfloat16)
    k = l2norm(torch.randn(B, T, HK, D, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, HV, D, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, HV, generator=gen))
    g = F.logsigmoid(torch.randn(B, T, HV, generator=gen) + g_shift) + g_offset
    ns = B if n_states is None else n_states
    s0 = s0_scale * torch.randn(ns, HV, D, D, generator=gen) if with_s0 else None
    return q, k, v, g, beta, s0


def plumbing_inputs():
    gen = _gen(0)
    B, T, H, D = 1, 256, 4, 64
    q = l2norm(torch.randn(B, T, H, D, generator=gen))
    k = l2norm(torch.randn(B, T, H, D, generator=gen))
    v = torch.randn(B, T, H, D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = F.logsigmoid(torch.randn(B, T, H, generator=gen))
    s0 = torch.zeros(B, H, D, D)
    return q, k, v, g, beta, s0


def rmsnorm_inputs(rows_t=1141, heads=32, dv=128):
    gen = _gen(1)
    x = torch.randn(rows_t, heads, dv, generator=gen).to(torch.bfloat16)
    z = torch.randn(rows_t, heads, dv, generator=gen).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(dv, generator=gen)).to(torch.bfloat16)
    return x, z, w, 1e-6


def decode_inputs():
    return make_gdn_inputs(3, B=64, T=1, HK=16, HV=32, g_offset=-1.0)


def prefill_inputs():
    return make_gdn_inputs(4, B=1, T=1141, HK=16, HV=32, g_shift=2.0)


def varlen_lengths():
    return torch.randint(512, 4097, (8,), generator=_gen(VARLEN_LENGTHS_SEED))


def varlen_inputs(lengths=None):
    lengths = varlen_lengths() if lengths is None else torch.as_tensor(lengths)
    total = int(lengths.sum())
    q, k, v, g, beta, s0 = make_gdn_inputs(5, B=1, T=total, HK=16, HV=32, g_shift=2.0,
                                           n_states=len(lengths))
    cu = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    return q, k, v, g, beta, s0, cu


def make_reference_inputs(B, S, seed, l2_pre=False, with_init_state=False, H=32, D=128):
    """The reference harness's random grid distributions
    (kernels/harness/parity_test.py:109-120), drawn on a CPU generator."""
    gen = _gen(seed)
    q = (torch.randn(B, S, H, D, generator=gen) / 8.0).to(torch.bfloat16)
    k = (torch.randn(B, S, H, D, generator=gen) / 8.0).to(torch.bfloat16)
    v = torch.randn(B, S, H, D, generator=gen).to(torch.bfloat16)
    g = -(torch.rand(B, S, H, generator=gen) * 0.3)
    beta = torch.rand(B, S, H, generator=gen)
    if l2_pre:
        q = l2norm(q.float()).to(torch.bfloat16)
        k = l2norm(k.float()).to(torch.bfloat16)
    s0 = torch.randn(B, H, D, D, generator=gen) * 0.5 if with_init_state else None
    return q, k, v, g, beta, s0


# ---------------------------------------------------------------- metrics
def row_cos_min(a, b):
    a = a.double().reshape(-1, a.shape[-1])
    b = b.double().reshape(-1, b.shape[-1])
    return F.cosine_similarity(a, b, dim=-1).min().item()


def max_rel(a, b, floor=0.1):
    d = (a.double() - b.double()).abs()
    return (d / b.double().abs().clamp_min(floor)).max().item()


def tensor_l2_rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def parity(out, ref):
    """All metrics for one output tensor vs its reference (both moved to CPU)."""
    out = out.detach().cpu().double()
    ref = ref.detach().cpu().double()
    d = (out - ref).abs()
    return {
        "max_abs": d.max().item() if d.numel() else 0.0,
        "mean_abs": d.mean().item() if d.numel() else 0.0,
        "row_cos_min": row_cos_min(out, ref) if d.numel() else 1.0,
        "max_rel": max_rel(out, ref) if d.numel() else 0.0,
        "l2_rel": tensor_l2_rel(out, ref) if d.numel() and ref.norm() > 0 else 0.0,
        "nan": bool(torch.isnan(out).any()),
        "first_nan": first_nan_token(out) if out.dim() == 4 and bool(torch.isnan(out).any()) else None,
    }


def fmt(m):
    return (f"max_abs={m['max_abs']:.3e} mean_abs={m['mean_abs']:.3e} "
            f"cos={m['row_cos_min']:.6f} rel={m['max_rel']:.2e} l2={m['l2_rel']:.2e}")


def assert_abs(m, tol=ABS_TOL, what=""):
    assert not m["nan"], f"{what}: NaN in output (first bad token {m.get('first_nan')})"
    assert m["max_abs"] <= tol, f"{what}: max |err| {m['max_abs']:.3e} > {tol} ({fmt(m)})"


def assert_ref_bar(m, what=""):
    """The reference harness's random-case bar (parity_test.py:188-189)."""
    assert not m["nan"], f"{what}: NaN in output"
    assert m["row_cos_min"] >= REF_COS_MIN and m["max_rel"] < REF_REL_MAX, f"{what}: {fmt(m)}"


# The reference's fixture bar (kernels/harness/parity_test.py:272-280): o
# tensor-L2 relative error < 3e-3 and row-cos >= 0.9999 over rows whose norm
# is not degenerate (> 1e-3 of the largest), final state row-cos >= 0.9999 and
# max-rel < 1e-3 -- the "24-layer drift budget".
FIX_O_L2 = 3e-3
FIX_COS = 0.9999
FIX_S_REL = 1e-3


def row_cos_min_masked(a, b, floor_ratio=1e-3):
    """Min cosine over rows whose reference norm exceeds floor_ratio of the
    largest (kernels/harness/parity_test.py:139-153)."""
    a = a.detach().cpu().double().reshape(-1, a.shape[-1])
    b = b.detach().cpu().double().reshape(-1, b.shape[-1])
    rn = b.norm(dim=-1)
    mask = rn > rn.max() * floor_ratio
    if not mask.any():
        return 1.0
    return F.cosine_similarity(a[mask], b[mask], dim=-1).min().item()


def assert_fixture_bar(o, o_ref, s, s_ref, what=""):
    l2 = tensor_l2_rel(o.detach().cpu(), o_ref)
    oc = row_cos_min_masked(o, o_ref)
    sc = row_cos_min(s.detach().cpu(), s_ref)
    sr = max_rel(s.detach().cpu(), s_ref)
    print(f"    fixture bar {what}: o l2={l2:.2e} cos={oc:.6f} | state cos={sc:.7f} rel={sr:.2e}",
          flush=True)
    assert l2 < FIX_O_L2 and oc >= FIX_COS, f"{what}: o l2 {l2:.2e} cos {oc:.6f}"
    assert sc >= FIX_COS and sr < FIX_S_REL, f"{what}: state cos {sc:.7f} max-rel {sr:.2e}"


def first_nan_token(o):
    """First token index whose output row holds a NaN in any head (o is
    [B, T, H, D]), or None: the localisation the reference does by bisecting
    prefixes (parity_test.py:231-249); chunk = index // 64."""
    bad = torch.isnan(o.detach().float()).flatten(2).any(-1).any(0)
    idx = torch.nonzero(bad)
    return int(idx[0]) if idx.numel() else None


def flops_prefill(total_tokens, hv):
    """Dense chunked-algorithm FLOP convention: 182.95 kFLOP per token per
    v-head (five C x C x 128, three 64 x 128 x 128 products and C^3/3 for the
    inverse per 64-token chunk)."""
    C, d = 64, 128
    per_chunk = 2 * (5 * C * C * d + 3 * C * d * d + C ** 3 / 3)
    return total_tokens * hv * per_chunk / C


assert math.isclose(flops_prefill(1, 1), 182954.67, rel_tol=1e-6)


def fused_inputs(seed, B, T, HK, HV, D=128, dtype=torch.float16, s0_scale=0.02):
    """Raw inputs of the fused prefill (gdnChunkPrefillSm87.cu:189-316): raw
    (unnormalised) q/k rows, v, gate inputs a, b, per-head A_log and dt_bias,
    an initial state.  A = e^{A_log} in U(0.02, 1) and dt_bias in N(0, 0.5)
    keep the per-token decay g in the range of the other prefill cases
    (mostly -0.05 .. -2); a freshly initialised layer's A = U(0, 16) would
    decay every state to ~0 within a token."""
    gen = _gen(seed)
    q = torch.randn(B, T, HK, D, generator=gen).to(dtype)
    k = torch.randn(B, T, HK, D, generator=gen).to(dtype)
    v = torch.randn(B, T, HV, D, generator=gen).to(dtype)
    a = torch.randn(B, T, HV, generator=gen).to(dtype)
    b = torch.randn(B, T, HV, generator=gen).to(dtype)
    A_log = torch.log(0.02 + 0.98 * torch.rand(HV, generator=gen))
    dt_bias = (0.5 * torch.randn(HV, generator=gen)).to(dtype)
    s0 = s0_scale * torch.randn(B, HV, D, D, generator=gen)
    return q, k, v, a, b, A_log, dt_bias, s0
