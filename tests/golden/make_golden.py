"""Writes the golden fixtures of the gated-delta path (run from the repo root:
``python tests/golden/make_golden.py``).

The reference holds no golden vectors for this path (its fixture files are
referenced but not shipped: kernels/harness/parity_test.py:319-326), so the
fixtures are produced here by the brute-force fp64 projector recurrence
(oracle.recurrence_fp64, independent of the chunked form).  The tests also
check the installed transformers functions the reference gates against
(kernels/harness/parity_test.py:22-27) against the same stored outputs.

  plumbing_T256_d64.npz  B1 T256 H4 d64 fp32 (CPU plumbing case): fp64 recurrence
                outputs and the sha256 of the seeded inputs.
  g128.npz      B1 T70 HK1 HV2 d128 bf16 inputs (stored as raw bf16 bits),
                fp32 initial state, fp64 recurrence outputs; the shape the
                HIP kernels accept.
  varlen_lengths.json  the 8 varlen sequence lengths (torch.randint(512, 4097,
                (8,)) on a CPU generator seeded 7).

g128 stores its inputs; the plumbing case stores a digest of them.  Either way a change in
torch's generator cannot silently move the fixtures.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import gdn_cases as gc  # noqa: E402
from oracle import gdn_oracle as orc  # noqa: E402


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def input_digest(*ts) -> str:
    """sha256 over the raw bytes of the given CPU tensors (regeneration check)."""
    import hashlib

    h = hashlib.sha256()
    for t in ts:
        h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


def make_c1() -> None:
    """Inputs are regenerated from the seed (their digest is stored, so a
    generator change fails loudly); outputs are stored."""
    q, k, v, g, beta, s0 = gc.plumbing_inputs()
    o, S = orc.recurrence_fp64(q, k, v, g, beta, s0)
    np.savez_compressed(HERE / "plumbing_T256_d64.npz", o_fp64=o.astype(np.float32),
                        S_fp64=S.astype(np.float32),
                        inputs_sha256=np.array(input_digest(q, k, v, g, beta, s0)))


def make_g128() -> None:
    q, k, v, g, beta, s0 = gc.make_gdn_inputs(21, B=1, T=70, HK=1, HV=2, s0_scale=0.05)
    o, S = orc.recurrence_fp64(q.double(), k.double(), v.double(), g.double(), beta.double(),
                               s0.double())
    np.savez_compressed(HERE / "g128.npz", q_bf16=bf16_bits(q), k_bf16=bf16_bits(k),
                        v_bf16=bf16_bits(v), g=g.numpy(), beta=beta.numpy(), s0=s0.numpy(),
                        o_fp64=o.astype(np.float32), S_fp64=S.astype(np.float32))


def make_varlen_lengths() -> None:
    lens = [int(x) for x in gc.varlen_lengths().tolist()]
    (HERE / "varlen_lengths.json").write_text(json.dumps({"seed": 7, "lengths": lens}) + "\n")


if __name__ == "__main__":
    make_c1()
    make_g128()
    make_varlen_lengths()
    for p in sorted(HERE.glob("*.np*")) + sorted(HERE.glob("*.json")):
        print(p.name, p.stat().st_size)
