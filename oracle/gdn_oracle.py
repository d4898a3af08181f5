"""CPU oracle for the gated-delta-rule (GDN) hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the reference that results are compared with
(or as the timed CPU baseline).

It restates, in plain torch CPU code (fp32 or fp64), the algorithm the
reference's kernels are gated against.  The defining code is the third-party
transformers function the reference imports as its parity reference
(``kernels/harness/parity_test.py:22-27``; a verbatim copy of the same math at
``kernels/harness/parity_test.py:35-96``), i.e.
transformers 5.14.1 ``models/qwen3_5/modeling_qwen3_5.py``:

* ``l2norm``                 -> modeling_qwen3_5.py:242-245
* ``chunk_gated_delta_rule`` -> modeling_qwen3_5.py:249-327 (== parity_test.py:35-96)
* ``chunk_debug_views``      -> the per-chunk A, T, M, cumsum(g) and entry states of the
                                same computation, as kernels/torch_binding.cpp:58-86 exposes them
* ``recurrent_gated_delta_rule`` -> modeling_qwen3_5.py:331-380
* ``gated_rmsnorm``          -> modeling_qwen3_5.py:168-184 (Qwen3_5RMSNormGated)
* ``causal_conv1d``          -> modeling_qwen3_5.py:219-240 (causal_conv1d_fn)
* ``causal_conv1d_update``   -> modeling_qwen3_5.py:199-216
* ``gdn_gate``               -> export/patches/orin_text_engine/files/cpp/kernels/
                                gdnKernels/gdnChunkPrefillSm87.cu:113-125
* ``fused_prefill``          -> gdnChunkPrefillSm87.cu:189-316 (runGdnChunkPrefillSm87:
                                l2norm + conversions + gates + prefill + o / state out)
* GQA head map               -> kernels/chunk_delta_cuda.h:12-14 (repeat_interleave)
* tail padding               -> kernels/chunk_delta_cuda.cu:17-19

Layouts follow the reference C ABI (``kernels/chunk_delta_cuda.h:12-20``):
q, k ``[B, T, HK, DK]``; v ``[B, T, HV, DV]``; g, beta ``[B, T, HV]``;
state ``[B, HV, DK, DV]``.  Varlen (``cu_seqlens``) is new relative to the
reference kernel (its torch fallback swallows the argument); the oracle
defines it as a per-sequence loop over a packed ``[1, sum(T), H, D]`` batch,
each sequence with its own initial and final state (FLA convention).

Every function here is pinned by tests in ``tests/test_oracle.py``:
an independent fp64 token recurrence (``recurrence_fp64``), closed forms,
library routines (``torch.linalg.solve_triangular``, ``F.rms_norm``), the
installed transformers functions, and invariances (chunk size, resume, GQA,
padding).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "l2norm",
    "gdn_gate",
    "expand_kv_heads",
    "chunk_gated_delta_rule",
    "chunk_gated_delta_rule_varlen",
    "chunk_debug_views",
    "recurrent_gated_delta_rule",
    "recurrence_fp64",
    "gated_rmsnorm",
    "unit_lower_inverse",
    "causal_conv1d",
    "causal_conv1d_update",
    "fused_prefill",
]


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Row L2 normalisation, eps inside the rsqrt (modeling_qwen3_5.py:242-245)."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def gdn_gate(a, b, A_log, dt_bias):
    """Gate pre-op: g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b).

    Follows gdnChunkPrefillSm87.cu:113-125 and modeling_qwen3_5.py:497-499.
    Returns fp32 (g, beta) with the [.., HV] layout of ``a`` / ``b``.
    """
    a = a.float()
    b = b.float()
    g = -torch.exp(A_log.float()) * F.softplus(a + dt_bias.float())
    return g, torch.sigmoid(b)


def expand_kv_heads(x: torch.Tensor, hv: int) -> torch.Tensor:
    """[B, T, HK, D] -> [B, T, HV, D]: v-head h reads k-head h // (HV // HK)
    (repeat_interleave semantics, kernels/chunk_delta_cuda.h:12-14)."""
    hk = x.shape[2]
    if hk == hv:
        return x
    assert hv % hk == 0, "HV must be a multiple of HK"
    return x.repeat_interleave(hv // hk, dim=2)


def unit_lower_inverse(A: torch.Tensor) -> torch.Tensor:
    """(I - A)^-1 for strictly lower triangular A (batched over leading dims).

    Row-by-row forward substitution, the scheme of modeling_qwen3_5.py:294-297:
    row i of the inverse is e_i + sum_{j<i} A[i, j] * row_j(inverse), done in
    place on the strictly lower part before the identity is added.
    """
    C = A.shape[-1]
    X = A.clone()
    for i in range(1, C):
        row = X[..., i, :i].clone()
        sub = X[..., :i, :i].clone()
        X[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
    return X + torch.eye(C, dtype=A.dtype)


def _chunk_core(q, k, v, g, beta, chunk_size, s0, dtype, views=None):
    """Chunked gated delta rule on [B, H, T, D] fp tensors (heads already
    expanded).  Restates modeling_qwen3_5.py:262-327 term by term:

        c   = cumsum_chunk(g)                 Gamma_rj = exp(c_r - c_j), r >= j
        A   = -(diag(beta) K K^T o Gamma)     strictly lower
        T   = (I - A)^-1
        U   = T diag(beta) V                  W = T diag(beta e^c) K
        per chunk n:  V_new = U - W S
                      O     = (Q e^c) S + (Q K^T o Gamma) V_new
                      S     = e^{c_last} S + (K e^{c_last - c})^T V_new
    """
    B, H, T, DK = k.shape
    DV = v.shape[-1]
    pad = (chunk_size - T % chunk_size) % chunk_size
    # zero padding with g = beta = 0 leaves cumsum, decay and state unchanged
    # (kernels/chunk_delta_cuda.cu:17-19)
    q = F.pad(q, (0, 0, 0, pad))
    k = F.pad(k, (0, 0, 0, pad))
    v = F.pad(v, (0, 0, 0, pad))
    g = F.pad(g, (0, pad))
    beta = F.pad(beta, (0, pad))
    Tp = T + pad
    n = Tp // chunk_size
    scale = 1.0 / math.sqrt(DK)
    q = q * scale
    qc = q.reshape(B, H, n, chunk_size, DK)
    kc = k.reshape(B, H, n, chunk_size, DK)
    vc = v.reshape(B, H, n, chunk_size, DV)
    bc = beta.reshape(B, H, n, chunk_size)
    c = g.reshape(B, H, n, chunk_size).cumsum(-1)

    lower_incl = torch.tril(torch.ones(chunk_size, chunk_size, dtype=torch.bool))
    strict = torch.tril(torch.ones(chunk_size, chunk_size, dtype=torch.bool), -1)
    diff = c.unsqueeze(-1) - c.unsqueeze(-2)
    gamma = torch.where(lower_incl, diff, torch.zeros((), dtype=dtype)).exp() * lower_incl

    kb = kc * bc.unsqueeze(-1)
    A = -(kb @ kc.transpose(-1, -2)) * gamma
    A = torch.where(strict, A, torch.zeros((), dtype=dtype))
    Tm = unit_lower_inverse(A)
    U = Tm @ (vc * bc.unsqueeze(-1))
    W = Tm @ (kb * c.exp().unsqueeze(-1))

    S = torch.zeros(B, H, DK, DV, dtype=dtype) if s0 is None else s0.to(dtype).clone()
    out = torch.empty(B, H, n, chunk_size, DV, dtype=dtype)
    if views is not None:
        views.update(A=A, T=Tm, c=c, M=[], S=[])
    for i in range(n):
        qi, ki = qc[:, :, i], kc[:, :, i]
        ci = c[:, :, i]
        M = (qi @ ki.transpose(-1, -2)) * gamma[:, :, i]
        if views is not None:
            views["M"].append(M)
            views["S"].append(S.clone())
        v_new = U[:, :, i] - W[:, :, i] @ S
        out[:, :, i] = (qi * ci.exp().unsqueeze(-1)) @ S + M @ v_new
        last = ci[..., -1:]
        kd = ki * (last - ci).exp().unsqueeze(-1)
        S = S * last.exp().unsqueeze(-1) + kd.transpose(-1, -2) @ v_new
    out = out.reshape(B, H, Tp, DV)[:, :, :T]
    return out, S


def chunk_gated_delta_rule(q, k, v, g, beta, initial_state=None, chunk_size=64,
                           dtype=torch.float32, use_qk_l2norm=False):
    """Chunked GDN prefill, reference layout.

    q, k: [B, T, HK, DK]; v: [B, T, HV, DV]; g, beta: [B, T, HV];
    initial_state: [B, HV, DK, DV] or None (zeros).
    Returns (o [B, T, HV, DV] in ``dtype``, final_state [B, HV, DK, DV] in ``dtype``).
    """
    HV = v.shape[2]
    q = q.to(dtype)
    k = k.to(dtype)
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    q = expand_kv_heads(q, HV)
    k = expand_kv_heads(k, HV)
    tr = lambda x: x.transpose(1, 2).contiguous().to(dtype)  # noqa: E731
    o, S = _chunk_core(tr(q), tr(k), tr(v), tr(g), tr(beta), chunk_size,
                       initial_state, dtype)
    return o.transpose(1, 2).contiguous(), S


def chunk_debug_views(q, k, v, g, beta, initial_state=None, chunk_size=64,
                      dtype=torch.float64):
    """Per-chunk quantities of ``chunk_gated_delta_rule`` for one sequence
    (B = 1), as the reference's debug workspace exposes them
    (kernels/torch_binding.cpp:58-86): A, T = (I - A)^-1, M = s (Q K^T o
    Gamma), the in-chunk cumsum of g, and the state at each chunk's start.
    Returns a dict of tensors [NC, HV, ...] (A, T, M: [..., C, C]; c: [..., C];
    S: [..., DK, DV]), padded rows included as the kernels pad them."""
    assert q.shape[0] == 1, "one sequence"
    HV = v.shape[2]
    qx = expand_kv_heads(q.to(dtype), HV)
    kx = expand_kv_heads(k.to(dtype), HV)
    tr = lambda x: x.transpose(1, 2).contiguous().to(dtype)  # noqa: E731
    views = {}
    _chunk_core(tr(qx), tr(kx), tr(v), tr(g), tr(beta), chunk_size, initial_state, dtype,
                views=views)
    first = lambda x: x[0].transpose(0, 1).contiguous()  # noqa: E731  [H, n, ...] -> [n, H, ...]
    return dict(A=first(views["A"]), T=first(views["T"]), c=first(views["c"]),
                M=torch.stack([m[0] for m in views["M"]], 0),
                S=torch.stack([x[0] for x in views["S"]], 0))


def chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu_seqlens, initial_state=None,
                                  chunk_size=64, dtype=torch.float32):
    """Varlen prefill: packed [1, sum(T), H, D] inputs, ``cu_seqlens`` [N+1],
    initial_state [N, HV, DK, DV] (or None).  A per-sequence loop of
    ``chunk_gated_delta_rule``; chunks never straddle sequence boundaries."""
    cu = [int(x) for x in torch.as_tensor(cu_seqlens).tolist()]
    N = len(cu) - 1
    HV, DV = v.shape[2], v.shape[3]
    DK = k.shape[3]
    o = torch.zeros(1, cu[-1], HV, DV, dtype=dtype)
    sf = torch.zeros(N, HV, DK, DV, dtype=dtype)
    for i in range(N):
        a, b = cu[i], cu[i + 1]
        s0 = None if initial_state is None else initial_state[i:i + 1]
        if b == a:
            sf[i] = 0 if s0 is None else s0[0].to(dtype)
            continue
        oi, si = chunk_gated_delta_rule(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b],
                                        beta[:, a:b], s0, chunk_size, dtype)
        o[:, a:b] = oi
        sf[i] = si[0]
    return o, sf


def recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=None, dtype=torch.float32):
    """Token recurrence / decode step (modeling_qwen3_5.py:331-380):

        S <- e^{g_t} S;  delta = beta_t (v_t - S^T k_t);  S <- S + k_t delta^T;
        o_t = (q_t / sqrt(DK))^T S        (o uses the updated state)

    Same layouts as ``chunk_gated_delta_rule``.  Returns (o, final_state).
    """
    B, T, HK, DK = q.shape
    HV, DV = v.shape[2], v.shape[3]
    q = expand_kv_heads(q.to(dtype), HV) / math.sqrt(DK)
    k = expand_kv_heads(k.to(dtype), HV)
    v = v.to(dtype)
    g = g.to(dtype)
    beta = beta.to(dtype)
    S = torch.zeros(B, HV, DK, DV, dtype=dtype) if initial_state is None \
        else initial_state.to(dtype).clone()
    o = torch.empty(B, T, HV, DV, dtype=dtype)
    for t in range(T):
        S = S * g[:, t].exp()[..., None, None]
        kv = (S * k[:, t, :, :, None]).sum(-2)
        delta = (v[:, t] - kv) * beta[:, t, :, None]
        S = S + k[:, t, :, :, None] * delta[:, :, None, :]
        o[:, t] = (S * q[:, t, :, :, None]).sum(-2)
    return o, S


def recurrence_fp64(q, k, v, g, beta, s0=None):
    """Independent brute-force fp64 numpy token recurrence, one head at a time,
    written directly from the delta-rule update (Yang et al. 2024, "Gated
    Delta Networks"): S_t = a_t (I - b_t k_t k_t^T) S_{t-1} + b_t k_t v_t^T,
    o_t = S_t^T q_t / sqrt(DK) with a_t = exp(g_t).

    This form multiplies the projector explicitly, so it shares no code path
    with the chunked form or with ``recurrent_gated_delta_rule``.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    beta = np.asarray(beta, dtype=np.float64)
    B, T, HK, DK = q.shape
    HV, DV = v.shape[2], v.shape[3]
    rep = HV // HK
    o = np.zeros((B, T, HV, DV))
    S_out = np.zeros((B, HV, DK, DV))
    eye = np.eye(DK)
    for b in range(B):
        for h in range(HV):
            S = np.zeros((DK, DV)) if s0 is None else np.asarray(s0[b, h], dtype=np.float64).copy()
            for t in range(T):
                kt = k[b, t, h // rep]
                qt = q[b, t, h // rep]
                P = eye - beta[b, t, h] * np.outer(kt, kt)
                S = np.exp(g[b, t, h]) * (P @ S) + beta[b, t, h] * np.outer(kt, v[b, t, h])
                o[b, t, h] = S.T @ qt / math.sqrt(DK)
            S_out[b, h] = S
    return o, S_out


def gated_rmsnorm(x, z, weight, eps=1e-6):
    """Qwen3_5RMSNormGated.forward (modeling_qwen3_5.py:175-184) with its
    dtype steps: normalise in fp32, round to the input dtype, multiply by the
    weight (in the weight's dtype promotion), multiply by silu(z) in fp32,
    round to the input dtype.
    """
    in_dtype = x.dtype
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    n = (xf * torch.rsqrt(var + eps)).to(in_dtype)
    h = weight * n
    h = h * F.silu(z.to(torch.float32))
    return h.to(in_dtype)


def _conv_valid(win, weight, bias, activation, t_out):
    """Last ``t_out`` outputs of the valid depthwise correlation over ``win``
    ([B, D, L] already in the weight dtype), with the dtype steps of the
    transformers functions: the sum in fp32 (taps oldest first, each tap a
    multiply-add rounded once to fp32, as a fused multiply-add, then the bias
    added -- the order of torch's CPU convolution, which this reproduces bit
    for bit), the result rounded to the weight dtype (F.conv1d runs in that
    dtype), SiLU in fp32 on the rounded value and rounded again.
    """
    wd = weight.dtype
    B, D, L = win.shape
    K = weight.shape[-1]
    n = L - K + 1
    xw = win.to(torch.float64)
    w64 = weight.to(torch.float64)
    acc = torch.zeros(B, D, n, dtype=torch.float32)
    for j in range(K):
        # fp32 * fp32 is exact in fp64, so one rounding to fp32 per tap
        acc = (acc.to(torch.float64) + w64[None, :, j:j + 1] * xw[:, :, j:j + n]).to(torch.float32)
    if bias is not None:
        acc = acc + bias.to(torch.float32)[None, :, None]
    out = acc.to(wd)
    if activation is not None:
        if activation not in ("silu", "swish"):
            raise ValueError(f"unsupported activation {activation!r}")
        out = F.silu(out.to(torch.float32)).to(wd)
    return out[:, :, n - t_out:]


def causal_conv1d(x, weight, bias=None, activation=None):
    """causal_conv1d_fn (modeling_qwen3_5.py:219-240): depthwise conv over
    time with K-1 zero tokens before the first, x [B, D, T], weight [D, K],
    bias [D] or None; returns [B, D, T] in x's dtype."""
    K = weight.shape[-1]
    T = x.shape[-1]
    win = F.pad(x.to(weight.dtype), (K - 1, 0))
    return _conv_valid(win, weight, bias, activation, T).to(x.dtype)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None):
    """causal_conv1d_update (modeling_qwen3_5.py:199-216) without the in-place
    write: the window is conv_state [B, D, L] followed by x [B, D, T];
    returns (y [B, D, T] in x's dtype, the new state = the window's last L
    tokens in conv_state's dtype)."""
    L = conv_state.shape[-1]
    T = x.shape[-1]
    win = torch.cat([conv_state, x], dim=-1).to(weight.dtype)
    new_state = win[:, :, -L:].to(conv_state.dtype)
    return _conv_valid(win, weight, bias, activation, T).to(x.dtype), new_state


def fused_prefill(q, k, v, a, b, A_log, dt_bias, state, chunk_size=64, dtype=torch.float32):
    """The reference TensorRT adapter's GDN step on raw inputs
    (gdnChunkPrefillSm87.cu:189-316): q and k rows L2-normalised in fp32
    with eps inside the rsqrt and rounded to bf16 (:52-84, :241-254), v
    rounded to bf16 (:87-97, :257-261), g and beta from the gate inputs in
    fp32 (:113-125), the prefill on those values, o rounded to bf16 and
    returned in q's dtype (:292-303), the final state in place of the
    initial one (:305-311).

    q, k: [B, T, HK, 128]; v: [B, T, HV, 128]; a, b: [B, T, HV];
    A_log, dt_bias: [HV]; state: [B, HV, 128, 128] (initial).
    Returns (o, final_state); o rounded as the adapter rounds it, the state
    in ``dtype``.
    """
    qn = l2norm(q.float()).to(torch.bfloat16)
    kn = l2norm(k.float()).to(torch.bfloat16)
    vb = v.to(torch.bfloat16)
    g, beta = gdn_gate(a, b, A_log, dt_bias)
    o, S = chunk_gated_delta_rule(qn, kn, vb, g, beta, state, chunk_size=chunk_size, dtype=dtype)
    return o.to(torch.bfloat16).to(q.dtype), S
