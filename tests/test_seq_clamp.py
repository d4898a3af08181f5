"""The kernels' sequence bookkeeping for packed batches, on the host
(deltanet_varlen_chunk_map runs the same code, csrc/gdn_seq.h): for any
cu_seqlens -- well-formed, non-monotone, negative, past the end -- every
token range stays inside [0, total_tokens) and every chunk id the scan forms
stays below the workspace's chunk bound.  CPU only: no kernel is launched.
"""
import ctypes as ct

import numpy as np
import pytest

from gdn_hip import capi


def _map(cu, total):
    lib = capi.lib()
    n = len(cu) - 1
    cu_a = (ct.c_int32 * len(cu))(*[int(x) for x in cu])
    outs = [(ct.c_int32 * n)() for _ in range(4)]
    bound = lib.deltanet_varlen_chunk_map(ct.cast(cu_a, ct.c_void_p), n, total,
                                          *[ct.cast(o, ct.c_void_p) for o in outs])
    return bound, [np.frombuffer(o, dtype=np.int32).astype(np.int64) for o in outs]


def _check_in_bounds(cu, total):
    bound, (c0, nc, t0, tn) = _map(cu, total)
    assert bound == (total + 63 * (len(cu) - 1)) // 64
    assert (t0 >= 0).all() and (tn >= 0).all() and (t0 + tn <= total).all()
    assert (c0 >= 0).all() and (nc >= 0).all()
    assert ((nc == 0) | (c0 + nc <= bound)).all()
    # every chunk the scan processes lies inside its sequence's token range
    assert (nc * 64 < tn + 64).all()
    return bound, c0, nc, t0, tn


def test_well_formed_matches_python():
    lengths = [1427, 3804, 2613, 3898, 660, 2279, 4069, 1111]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    bound, c0, nc, t0, tn = _check_in_bounds(cu, int(cu[-1]))
    chunks = [(L + 63) // 64 for L in lengths]
    assert list(nc) == chunks and list(c0) == list(np.concatenate([[0], np.cumsum(chunks)[:-1]]))
    assert list(t0) == list(cu[:-1]) and list(tn) == lengths


@pytest.mark.parametrize("seed", range(40))
def test_malformed_cu_stays_in_bounds(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    total = int(rng.integers(0, 5000))
    kind = seed % 4
    if kind == 0:      # arbitrary values, negatives and past the end
        cu = rng.integers(-3000, 9000, n + 1)
    elif kind == 1:    # non-monotone, inside [0, total]
        cu = rng.integers(0, total + 1, n + 1)
    elif kind == 2:    # repeated full ranges: every sequence spans all tokens
        cu = np.array([0 if i % 2 == 0 else total for i in range(n + 1)])
    else:              # well-formed prefix, last entry past the end
        cu = np.concatenate([[0], np.sort(rng.integers(0, total + 1, n - 1)), [total + 777]])
    _check_in_bounds(cu, total)


def test_extreme_values():
    big = 2 ** 31 - 1
    _check_in_bounds([-big - 1, big, -5, big], 100)
    _check_in_bounds([0, 0, 0], 0)
    # huge total: the chunk-count prefix sums saturate instead of wrapping
    cu = [0, big] * 40 + [0]
    bound, c0, nc, t0, tn = _check_in_bounds(cu, big)
    assert nc[0] == (big + 63) // 64 and (c0 >= 0).all()
