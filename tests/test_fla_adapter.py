"""The fla adapter (qwen-drive-edge-orin_amd/hf/fla): transformers picks it up
and passes only arguments it accepts; it refuses host tensors (no CPU path).

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
for name in ("torch_chunk_gated_delta_rule", "torch_recurrent_gated_delta_rule"):
    impl = inspect.getclosurevars(getattr(mq, name)).nonlocals["implementation"]
    print(name, impl.__module__, impl.__name__)
"""


def test_transformers_resolves_the_adapter():
    out = subprocess.run([sys.executable, "-c", _RESOLVE, str(HF_DIR)], capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    lines = dict(l.split(" ", 1) for l in out.stdout.strip().splitlines())
    assert lines["torch_chunk_gated_delta_rule"] == "fla.ops.gated_delta_rule chunk_gated_delta_rule"
    assert lines["torch_recurrent_gated_delta_rule"] == \
        "fla.ops.gated_delta_rule recurrent_gated_delta_rule"


def _adapter():
    """Import the adapter, then drop it from sys.modules again: transformers,
    imported later in this process by the oracle tests, must not find it."""
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


def test_accepts_the_keywords_transformers_passes():
    """modeling_qwen3_5.py:506-528 passes g, beta, initial_state,
    output_final_state, use_qk_l2norm_in_kernel and cu_seqlens by keyword."""
    m = _adapter()
    for fn in (m.chunk_gated_delta_rule, m.recurrent_gated_delta_rule):
        params = inspect.signature(fn).parameters
        for kw in ("g", "beta", "initial_state", "output_final_state",
                   "use_qk_l2norm_in_kernel", "cu_seqlens", "scale"):
            assert kw in params, (fn.__name__, kw)
        assert list(params)[:3] == ["q", "k", "v"]


def test_rejects_host_tensors():
    import torch

    m = _adapter()
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    v = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    g = torch.zeros(1, 4, 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        m.chunk_gated_delta_rule(q, q, v, g, g)
    with pytest.raises(RuntimeError, match="HIP device"):
        m.recurrent_gated_delta_rule(q, q, v, g, g)


@pytest.mark.parametrize("env,expect", [(None, False), ("0", False), ("1", True)])
def test_checked_mode_reaches_the_op(monkeypatch, env, expect):
    """GDN_HIP_CHECKED=1 at import makes every prefill call ask the op to check
    the scan's status word (checked=True: synchronise and raise on a bounded
    wait that gave up); unset or 0 leaves the call asynchronous.  The op and
    the device-side conversions are stubbed: this checks the plumbing only."""
    import torch

    if env is None:
        monkeypatch.delenv("GDN_HIP_CHECKED", raising=False)
    else:
        monkeypatch.setenv("GDN_HIP_CHECKED", env)
    m = _adapter()
    assert m._CHECKED is expect
    seen = {}

    def fake_prefill(q, k, v, g, beta, s0, **kw):
        seen.update(kw)
        return torch.zeros_like(v), None

    monkeypatch.setattr(m, "_prepare", lambda q, k, v, g, beta, *a, **kw: (q, k, v, g, beta, 2,
                                                                            False))
    monkeypatch.setattr(m.gdn_hip, "chunk_prefill", fake_prefill)
    x = torch.zeros(1, 4, 2, 128)
    g = torch.zeros(1, 4, 2)
    m.chunk_gated_delta_rule(x, x, x, g, g)
    assert seen["checked"] is expect
    m.chunk_gated_delta_rule(x, x, x, g, g, cu_seqlens=torch.tensor([0, 4]))
    assert seen["checked"] is expect
