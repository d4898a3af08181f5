"""``causal_conv1d_fn`` / ``causal_conv1d_update`` with the calling
convention transformers uses for the causal-conv1d package
(models/qwen3_5/modeling_qwen3_5.py:199-240 for the torch fallbacks,
457-476 for the calls), backed by the gfx950 conv ops of ``gdn_hip``.

transformers imports ``causal_conv1d`` and takes these two functions when the
import succeeds, so putting the directory that holds this package on
``sys.path`` routes the Qwen3.5 gated-delta layers' convolutions here.

x is ``[B, D, T]`` (the update also takes ``[B, D]``), weight ``[D, K]`` or
``[D, 1, K]`` with K in 2..4, bias ``[D]`` or None, conv_state ``[B, D, L]``
with L in K-1..8 (updated in place).  x must be bf16 or fp16 and weight/bias
of x's dtype or fp32.  Outputs match the torch fallbacks' dtype steps: the
convolution in the weight dtype with an fp32 sum, SiLU in fp32, rounded to
x's dtype.  Features the kernels do not implement (``seq_idx``, initial or
final states of the prefill form, ``cache_seqlens``, ``conv_state_indices``,
activations other than SiLU) raise; there is no silent fallback.
"""
from __future__ import annotations

import sys
from pathlib import Path

_PKG_DIR = Path(__file__).resolve().parents[2]   # .../qwen-drive-edge-orin_amd
if str(_PKG_DIR) not in sys.path:
    sys.path.insert(0, str(_PKG_DIR))

import gdn_hip  # noqa: E402

__all__ = ["causal_conv1d_fn", "causal_conv1d_update"]


def _silu(activation) -> bool:
    if activation is None:
        return False
    if activation in ("silu", "swish"):
        return True
    raise NotImplementedError(f"activation {activation!r} (only None, 'silu', 'swish')")


def _weight(weight):
    if weight.dim() == 3 and weight.shape[1] == 1:
        weight = weight.squeeze(1)
    if weight.dim() != 2:
        raise ValueError("weight must be [D, K] or [D, 1, K]")
    return weight


def _on_device(**tensors):
    for name, t in tensors.items():
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{name} must be on the HIP device (the ops have no CPU path)")


def causal_conv1d_fn(x, weight, bias=None, seq_idx=None, initial_states=None,
                     return_final_states=False, final_states_out=None, activation=None):
    """Causal depthwise conv1d over x [B, D, T]; returns [B, D, T] in x's
    dtype (a transposed view of a contiguous [B, T, D] buffer)."""
    if seq_idx is not None or initial_states is not None or return_final_states or \
            final_states_out is not None:
        raise NotImplementedError("seq_idx / initial_states / final states are not supported")
    silu = _silu(activation)
    _on_device(x=x, weight=weight, bias=bias)
    if x.dim() != 3:
        raise ValueError("x must be [B, D, T]")
    return gdn_hip.causal_conv1d_fwd(x, _weight(weight), bias, silu)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, cache_seqlens=None,
                         conv_state_indices=None):
    """Decode step: x [B, D, T] or [B, D] is appended to conv_state (updated
    in place); returns the outputs for x's tokens in x's shape and dtype."""
    if cache_seqlens is not None or conv_state_indices is not None:
        raise NotImplementedError("cache_seqlens / conv_state_indices are not supported")
    silu = _silu(activation)
    _on_device(x=x, conv_state=conv_state, weight=weight, bias=bias)
    squeeze = x.dim() == 2
    if squeeze:
        x = x.unsqueeze(-1)
    if x.dim() != 3:
        raise ValueError("x must be [B, D, T] or [B, D]")
    y = gdn_hip.causal_conv1d_update(x, conv_state, _weight(weight), bias, silu)
    return y.squeeze(-1) if squeeze else y
