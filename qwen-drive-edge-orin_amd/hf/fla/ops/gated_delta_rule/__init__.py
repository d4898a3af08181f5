"""``chunk_gated_delta_rule`` / ``recurrent_gated_delta_rule`` with the
argument convention transformers passes to flash-linear-attention
(models/qwen3_5/modeling_qwen3_5.py:505-529), backed by the gfx950 ops of
``gdn_hip`` (chunked prefill and the recurrent step).

Tensors are ``[B, T, H, D]`` (q, k with H = the v-head count or a divisor of
it, v with the v-head count), g and beta ``[B, T, HV]``, states
``[B, HV, 128, 128]``.  With ``cu_seqlens`` the batch is one packed row
(B = 1) and states are per sequence.  Differences from the torch fallback
(modeling_qwen3_5.py:249-327,331-380) are only in rounding: the kernels take
bf16 q/k/v and fp32 g/beta/state and return bf16 outputs.

Only what the kernels implement is accepted: head dims of 128, any scale (q
is rescaled), l2-normalised or raw q/k.  Anything else raises; there is no
silent fallback to another implementation.

The prefill's scan waits on its own stages with bounded waits; one that gives
up (another process holding the device for ~0.1 s, say) leaves o and the
state incomplete and sets a status word.  With the environment variable
``GDN_HIP_CHECKED=1`` set when this module is imported, every prefill call
synchronises and raises ``RuntimeError`` on such a give-up (a debug mode:
the check costs a host synchronisation per call).
"""
from __future__ import annotations

import math
import os
import sys
from pathlib import Path

_PKG_DIR = Path(__file__).resolve().parents[4]   # .../qwen-drive-edge-orin_amd
if str(_PKG_DIR) not in sys.path:
    sys.path.insert(0, str(_PKG_DIR))

import gdn_hip  # noqa: E402

_D = 128
_KERNEL_SCALE = 1.0 / math.sqrt(_D)
_CHECKED = os.environ.get("GDN_HIP_CHECKED", "0") not in ("", "0")


def _l2norm(x, eps=1e-6):
    """x * rsqrt(sum(x^2) + eps) over the last dim in fp32, as transformers'
    l2norm (modeling_qwen3_5.py:242-245)."""
    import torch

    xf = x.float()
    return xf * torch.rsqrt((xf * xf).sum(dim=-1, keepdim=True) + eps)


def _prepare(q, k, v, g, beta, scale, use_qk_l2norm_in_kernel, kernel_norm=False):
    """Validate and convert.  With ``kernel_norm`` (the kernels can normalise
    bf16 q/k rows themselves) and the default scale, bf16 q and k are
    returned raw and the last element says the kernel must normalise them."""
    import torch

    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be on the HIP device (the ops have no CPU path)")
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4:
        raise ValueError("q, k must be [B, T, H, 128] of one shape and v [B, T, HV, 128]")
    if q.shape[-1] != _D or v.shape[-1] != _D:
        raise NotImplementedError(f"head dims must be {_D} (got {q.shape[-1]}, {v.shape[-1]})")
    B, T, HQ, _ = q.shape
    HV = v.shape[2]
    if v.shape[:2] != (B, T) or HV % HQ != 0:
        raise ValueError("v must be [B, T, HV, 128] with HV a multiple of the q/k heads")
    if g.shape != (B, T, HV) or beta.shape != (B, T, HV):
        raise ValueError("g and beta must be [B, T, HV]")
    custom_scale = scale is not None and abs(float(scale) - _KERNEL_SCALE) > 1e-12
    bf = torch.bfloat16
    in_kernel = (use_qk_l2norm_in_kernel and kernel_norm and not custom_scale
                 and q.dtype == bf and k.dtype == bf)
    if use_qk_l2norm_in_kernel and not in_kernel:
        q, k = _l2norm(q), _l2norm(k)
    if custom_scale:
        q = q.float() * (float(scale) / _KERNEL_SCALE)   # the kernels scale q by 1/sqrt(128)
    return (q.to(bf).contiguous(), k.to(bf).contiguous(), v.to(bf).contiguous(),
            g.float().contiguous(), beta.float().contiguous(), HV, in_kernel)


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                           output_final_state=False, use_qk_l2norm_in_kernel=False,
                           cu_seqlens=None, **kwargs):
    """Chunked gated delta rule (prefill).  Returns ``(o, final_state)``,
    final_state None unless ``output_final_state``; o has q's dtype, as in
    transformers' fallback (modeling_qwen3_5.py:326, ``.to(initial_dtype)``)."""
    import torch

    out_dtype = q.dtype
    q, k, v, g, beta, HV, norm = _prepare(q, k, v, g, beta, scale, use_qk_l2norm_in_kernel,
                                          kernel_norm=True)
    s0 = None
    if initial_state is not None:
        s0 = initial_state.float().contiguous()
    if cu_seqlens is not None:
        if q.shape[0] != 1:
            raise ValueError("with cu_seqlens the batch must be one packed row (B = 1)")
        o, sf = gdn_hip.chunk_prefill(q, k, v, g, beta, s0,
                                      cu_seqlens=cu_seqlens.to(torch.int32).contiguous(),
                                      qk_l2norm=norm, checked=_CHECKED)
    else:
        o, sf = gdn_hip.chunk_prefill(q, k, v, g, beta, s0, qk_l2norm=norm, checked=_CHECKED)
    return o.to(out_dtype), (sf if output_final_state else None)


def recurrent_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None,
                               output_final_state=False, use_qk_l2norm_in_kernel=False,
                               cu_seqlens=None, **kwargs):
    """Token-by-token gated delta rule (decode).  Returns ``(o, final_state)``
    with o in q's dtype (modeling_qwen3_5.py:379); the caller's initial_state
    is not modified."""
    import torch

    out_dtype = q.dtype
    if cu_seqlens is not None:
        raise NotImplementedError("recurrent_gated_delta_rule takes no cu_seqlens here")
    q, k, v, g, beta, HV, norm = _prepare(q, k, v, g, beta, scale, use_qk_l2norm_in_kernel,
                                          kernel_norm=True)
    B = q.shape[0]
    if initial_state is None:
        state = torch.zeros(B, HV, _D, _D, dtype=torch.float32, device=q.device)
    else:
        state = initial_state.float().clone().contiguous()
    o = gdn_hip.recurrent_step(q, k, v, g, beta, state, qk_l2norm=norm)
    return o.to(out_dtype), (state if output_final_state else None)
