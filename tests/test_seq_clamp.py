"""The kernels' sequence bookkeeping for packed batches, on the host
(deltanet_varlen_chunk_map runs the same code, csrc/gdn_seq.h): for any
cu_seqlens -- well-formed, non-monotone, negative, past the end -- every
token range stays inside [0, total_tokens) and every chunk id the scan forms
stays below the workspace's chunk bound.  The block-cooperative lookups the
kernels actually run (the prep's locate_chunk, the scan's chunks_before) are
checked through their host twins, which run the same phases thread by
thread.  CPU only: no kernel is launched.
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


def _cu_arr(cu):
    return (ct.c_int32 * len(cu))(*[int(x) for x in cu])


def _prefix_chunks(cu, total):
    """Python restatement: clamped token ranges and saturating chunk prefix sums."""
    sat = 1 << 30
    lo = [min(max(int(x), 0), total) for x in cu]
    counts = [max(lo[i + 1] - lo[i], 0) for i in range(len(cu) - 1)]
    chunks = [(n + 63) // 64 for n in counts]
    pre, acc = [], 0
    for c in chunks:
        pre.append(acc)
        acc = min(acc + c, sat)
    return lo, counts, chunks, pre, acc


def _check_lookups(cu, total, nts=(256,), cids=None):
    lib = capi.lib()
    n = len(cu) - 1
    cu_a = _cu_arr(cu)
    lo, counts, chunks, pre, tot = _prefix_chunks(cu, total)
    for nt in (64, 256, 1024):
        for upto in sorted({0, 1, n // 2, n - 1, n}):
            got = lib.deltanet_varlen_chunks_before(ct.cast(cu_a, ct.c_void_p), n, total, upto, nt)
            want = pre[upto] if upto < n else tot
            assert got == want, (nt, upto, got, want)
    bound = (total + 63 * n) // 64
    if cids is None:
        cids = range(bound + 2)
    out = (ct.c_int32 * 3)()
    for nt in nts:
        for cid in cids:
            r = lib.deltanet_varlen_locate_chunk(ct.cast(cu_a, ct.c_void_p), n, total, cid, nt,
                                                 ct.cast(out, ct.c_void_p))
            assert r in (0, 1)
            # the Python restatement: the sequence whose chunk range holds cid
            owner = next((s for s in range(n) if chunks[s] > 0 and pre[s] + chunks[s] < (1 << 30)
                          and pre[s] <= cid < pre[s] + chunks[s]), None)
            if owner is None:
                assert r == 0, (nt, cid, list(out))
                continue
            c = cid - pre[owner]
            assert r == 1 and out[0] == owner, (nt, cid, list(out), owner)
            assert out[1] == lo[owner] + 64 * c and out[2] == min(64, counts[owner] - 64 * c)
            # in bounds: rows [tok0, tok0 + rows) inside [0, total)
            assert 0 <= out[1] and 1 <= out[2] <= 64 and out[1] + out[2] <= total


def test_lookup_twins_well_formed():
    lengths = [1427, 3804, 2613, 3898, 660, 2279, 4069, 1111]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    _check_lookups(cu, int(cu[-1]), nts=(2, 64, 256))


@pytest.mark.parametrize("seed", range(24))
def test_lookup_twins_malformed_cu(seed):
    """The twins against the Python restatement for malformed cu_seqlens, over
    every chunk id below the workspace's bound (and two past it), including
    batches wider than one block of simulated threads."""
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 300 if seed % 3 == 0 else 40))
    total = int(rng.integers(0, 3000))
    kind = seed % 4
    if kind == 0:
        cu = rng.integers(-3000, 9000, n + 1)
    elif kind == 1:
        cu = rng.integers(0, total + 1, n + 1)
    elif kind == 2:
        cu = np.array([0 if i % 2 == 0 else total for i in range(n + 1)])
    else:
        cu = np.concatenate([[0], np.sort(rng.integers(0, total + 1, n - 1)), [total + 777]])
    _check_lookups(cu, total, nts=(64, 256))


def test_lookup_twins_saturated_prefix():
    """Chunk counts whose prefix sum passes 2^30: chunk ids inside the
    saturated range have no owner, and the lookup reports none instead of
    reading a stale sequence index."""
    big = 2 ** 31 - 1
    cu = [0, big] * 40 + [0]
    n = len(cu) - 1
    per = (big + 63) // 64
    cids = [0, per - 1, per, 31 * per, 31 * per + 5, (1 << 30) - 1, 1 << 30, (1 << 30) + 7,
            big]
    _check_lookups(cu, big, nts=(64, 256), cids=cids)


def test_lookup_twins_reject_bad_args():
    lib = capi.lib()
    cu = _cu_arr([0, 5])
    out = (ct.c_int32 * 3)()
    p = ct.cast(cu, ct.c_void_p)
    assert lib.deltanet_varlen_chunks_before(p, 1, 5, 2, 256) == -1      # upto > n
    assert lib.deltanet_varlen_chunks_before(p, 1, 5, 1, 100) == -1      # nt not a multiple of 64
    assert lib.deltanet_varlen_locate_chunk(p, 1, 5, 0, 3, ct.cast(out, ct.c_void_p)) == -1
    assert lib.deltanet_varlen_locate_chunk(None, 1, 5, 0, 256, ct.cast(out, ct.c_void_p)) == -1
