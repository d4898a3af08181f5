"""The causal_conv1d adapter (qwen-drive-edge-orin_amd/hf/causal_conv1d):
transformers picks it up, the calls transformers makes
(models/qwen3_5/modeling_qwen3_5.py:457-476) bind to its signature, and it
refuses host tensors and unsupported features (no CPU path, no fallback).

The resolution check runs in a child process so that this process's
transformers import (used by the oracle tests) keeps its torch fallback.
"""
import inspect
import subprocess
import sys
from pathlib import Path

import pytest

HF_DIR = Path(__file__).resolve().parent.parent / "qwen-drive-edge-orin_amd" / "hf"

_RESOLVE = r"""
import inspect, sys
sys.path.insert(0, sys.argv[1])
import transformers.models.qwen3_5.modeling_qwen3_5 as mq
for name in ("causal_conv1d_fn", "causal_conv1d_update"):
    impl = inspect.getclosurevars(getattr(mq, name)).nonlocals["implementation"]
    print(name, impl.__module__, impl.__name__)
"""


def test_transformers_resolves_the_adapter():
    out = subprocess.run([sys.executable, "-c", _RESOLVE, str(HF_DIR)], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = dict(l.split(" ", 1) for l in out.stdout.strip().splitlines())
    assert lines["causal_conv1d_fn"] == "causal_conv1d causal_conv1d_fn"
    assert lines["causal_conv1d_update"] == "causal_conv1d causal_conv1d_update"


def _adapter():
    """Import the adapter, then drop it from sys.modules again: transformers,
    imported later in this process, must not find it."""
    import importlib

    before = set(sys.modules)
    sys.path.insert(0, str(HF_DIR))
    try:
        m = importlib.import_module("causal_conv1d")
    finally:
        sys.path.remove(str(HF_DIR))
        for name in set(sys.modules) - before:
            if name == "causal_conv1d" or name.startswith("causal_conv1d."):
                del sys.modules[name]
    return m


def test_signatures_bind_transformers_calls():
    m = _adapter()
    # causal_conv1d_fn(mixed_qkv, weight, bias, activation=...) and
    # causal_conv1d_update(mixed_qkv, conv_state, weight, bias, activation)
    inspect.signature(m.causal_conv1d_fn).bind(1, 2, None, activation="silu")
    inspect.signature(m.causal_conv1d_update).bind(1, 2, 3, None, "silu")


def test_rejects_host_tensors_and_unsupported_features():
    import torch

    m = _adapter()
    x = torch.zeros(1, 64, 5, dtype=torch.bfloat16)
    w = torch.zeros(64, 4, dtype=torch.bfloat16)
    st = torch.zeros(1, 64, 4, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        m.causal_conv1d_fn(x, w, None, activation="silu")
    with pytest.raises(RuntimeError, match="HIP device"):
        m.causal_conv1d_update(x, st, w, None, "silu")
    with pytest.raises(NotImplementedError):
        m.causal_conv1d_fn(x, w, None, activation="gelu")
    with pytest.raises(NotImplementedError):
        m.causal_conv1d_fn(x, w, None, seq_idx=torch.zeros(1, 5, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        m.causal_conv1d_update(x, st, w, None, "silu", cache_seqlens=torch.zeros(1))
