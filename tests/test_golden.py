"""Oracle and third-party reference function against the committed golden
fixtures (tests/golden/, written by tests/golden/make_golden.py)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import gdn_cases as gc
from oracle import gdn_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def _bf16(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def g128_inputs():
    z = _load("g128.npz")
    return (_bf16(z["q_bf16"]), _bf16(z["k_bf16"]), _bf16(z["v_bf16"]),
            torch.from_numpy(z["g"]), torch.from_numpy(z["beta"]), torch.from_numpy(z["s0"]),
            torch.from_numpy(z["o_fp64"]), torch.from_numpy(z["S_fp64"]))


def test_plumbing_inputs_regenerate():
    from golden.make_golden import input_digest

    z = _load("plumbing_T256_d64.npz")
    assert str(z["inputs_sha256"]) == input_digest(*gc.plumbing_inputs())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_plumbing_oracle_matches_golden(dtype):
    z = _load("plumbing_T256_d64.npz")
    q, k, v, g, beta, s0 = gc.plumbing_inputs()
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-6
    assert np.abs(o.double().numpy() - z["o_fp64"]).max() < tol
    assert np.abs(S.double().numpy() - z["S_fp64"]).max() < tol


def test_plumbing_transformers_matches_golden():
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    z = _load("plumbing_T256_d64.npz")
    q, k, v, g, beta, s0 = gc.plumbing_inputs()
    o, S = m.torch_chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0,
                                          output_final_state=True)
    assert np.abs(o.double().numpy() - z["o_fp64"]).max() < 1e-5
    assert np.abs(S.double().numpy() - z["S_fp64"]).max() < 1e-5


def test_g128_oracle_matches_golden():
    q, k, v, g, beta, s0, o_ref, S_ref = g128_inputs()
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    assert (o - o_ref.double()).abs().max().item() < 1e-6
    assert (S - S_ref.double()).abs().max().item() < 1e-6
    o_r, S_r = orc.recurrent_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float64)
    assert (o_r - o_ref.double()).abs().max().item() < 1e-6


def test_varlen_lengths_fixture():
    meta = json.loads((GOLDEN / "varlen_lengths.json").read_text())
    assert meta["lengths"] == [int(x) for x in gc.varlen_lengths().tolist()]
    assert sum(meta["lengths"]) == 19861
