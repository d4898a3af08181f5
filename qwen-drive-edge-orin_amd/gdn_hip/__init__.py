"""gdn_hip: MI355X (gfx950) gated-delta-rule ops.

The compiled pieces live next to this file:
  libgdn_hip.so            C ABI (include/gdn_hip.h)
  deltanet_chunk_hip*.so   torch extension over it, the drop-in for the
                           reference's deltanet_chunk_cuda / _tco modules
                           (kernels/torch_binding.cpp:113-131)

``load()`` returns the extension module, whose ops are

  chunk_prefill(q, k, v, g, beta, s0=None, *, cu_seqlens=None, qk_l2norm=False,
                checked=False)                         -> [o, final_state]
  chunk_prefill_debug(...)  -> [o, final_state, T, A, cumsum_g, T_post_leaf, M, S_chunk]
  recurrent_step(q, k, v, g, beta, state, *, qk_l2norm=False) -> o
                                                        (state updated in place)
  chunk_prefill_norm(q, k, v, g, beta, z, weight, s0=None, *, eps=1e-6, checked=False,
                     fused=False)
                          -> [gated_rmsnorm(o, z, weight), final_state]
  chunk_prefill_fused(q, k, v, a, b, A_log, dt_bias, state) -> o
                          raw q/k/v and gate inputs     (state updated in place)
  gated_rmsnorm(x, z, weight, eps=1e-6) -> y
  causal_conv1d_fwd(x, weight, bias=None, silu=False) -> y      x, y [B, D, T]
  causal_conv1d_update(x, conv_state, weight, bias=None, silu=False) -> y
                                                  (conv_state updated in place)

``checked=True`` synchronises after the call and raises when one of the
scan's bounded waits gave up (o and the state would then be incomplete);
the default leaves the call asynchronous.

There is no fallback: if the extension is not built, ``load()`` raises.
Build with ``python qwen-drive-edge-orin_amd/build.py``.
"""
from __future__ import annotations

import importlib
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libgdn_hip.so"
EXT_NAME = "deltanet_chunk_hip"

_mod = None


def ext_path() -> Path | None:
    hits = sorted(HERE.glob(f"{EXT_NAME}.cpython*.so"))
    return hits[0] if hits else None


def load():
    """Import the in-tree torch extension (raises ImportError when missing)."""
    global _mod
    if _mod is None:
        if not LIB_PATH.exists() or ext_path() is None:
            raise ImportError(
                f"gdn_hip native code is not built under {HERE}; run "
                "`python qwen-drive-edge-orin_amd/build.py`")
        import torch  # noqa: F401  (loads libc10/libtorch the extension links)
        _mod = importlib.import_module(f"{__name__}.{EXT_NAME}")
    return _mod


def chunk_prefill(q, k, v, g, beta, s0=None, *, cu_seqlens=None, qk_l2norm=False,
                  checked=False):
    return load().chunk_prefill(q, k, v, g, beta, s0, cu_seqlens=cu_seqlens, qk_l2norm=qk_l2norm,
                                checked=checked)


def chunk_prefill_debug(q, k, v, g, beta, s0=None, *, cu_seqlens=None):
    return load().chunk_prefill_debug(q, k, v, g, beta, s0, cu_seqlens=cu_seqlens)


def chunk_prefill_norm(q, k, v, g, beta, z, weight, s0=None, *, eps=1e-6, checked=False,
                       fused=False):
    return load().chunk_prefill_norm(q, k, v, g, beta, z, weight, s0, eps=eps, checked=checked,
                                     fused=fused)


def chunk_prefill_fused(q, k, v, a, b, A_log, dt_bias, state):
    return load().chunk_prefill_fused(q, k, v, a, b, A_log, dt_bias, state)


def recurrent_step(q, k, v, g, beta, state, *, qk_l2norm=False):
    return load().recurrent_step(q, k, v, g, beta, state, qk_l2norm=qk_l2norm)


def gated_rmsnorm(x, z, weight, eps=1e-6):
    return load().gated_rmsnorm(x, z, weight, eps)


def causal_conv1d_fwd(x, weight, bias=None, silu=False):
    return load().causal_conv1d_fwd(x, weight, bias, silu)


def causal_conv1d_update(x, conv_state, weight, bias=None, silu=False):
    return load().causal_conv1d_update(x, conv_state, weight, bias, silu)
