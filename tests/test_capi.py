"""The C-ABI boundary on the CPU: the library loads, exports every function
include/gdn_hip.h declares, sizes workspaces, and rejects unsupported
configurations on the host (hipErrorInvalidValue, the reference's
cudaErrorInvalidValue contract, kernels/chunk_delta_cuda.cu:706-708,727)
before any launch.  No call here reaches a kernel."""
import ctypes as ct

import pytest

import gdn_hip
from gdn_hip import capi

INVALID = capi.HIP_ERROR_INVALID_VALUE


@pytest.fixture(scope="module")
def lib():
    if not gdn_hip.LIB_PATH.exists():
        pytest.fail(f"{gdn_hip.LIB_PATH} is not built")
    return capi.lib()


def test_exports_every_declared_symbol(lib):
    names = capi.declared_symbols()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/gdn_hip.h but not exported"
        assert n in capi._PROTOS, f"{n} has no ctypes prototype"


def test_workspace_size(lib):
    ws = lib.deltanet_prefill_workspace_size
    assert ws(1, 1141, 32, 128, 128, 64) > 0
    assert ws(1, 1141, 32, 64, 128, 64) == 0          # DK != 128
    assert ws(1, 1141, 32, 128, 64, 64) == 0          # DV != 128
    assert ws(1, 1141, 32, 128, 128, 32) == 0         # chunk != 64
    assert ws(0, 10, 32, 128, 128, 64) == 0
    assert ws(1, 0, 32, 128, 128, 64) > 0              # T = 0: no chunks, still a valid size
    # grows with chunks and heads; tcop twin is the same size
    assert ws(1, 1152, 32, 128, 128, 64) == ws(1, 1141, 32, 128, 128, 64)
    assert ws(1, 1153, 32, 128, 128, 64) > ws(1, 1152, 32, 128, 128, 64)
    assert ws(2, 1141, 32, 128, 128, 64) > ws(1, 1141, 32, 128, 128, 64)
    assert lib.deltanet_tcop_prefill_workspace_size(1, 1141, 32, 128, 128, 64) == \
        ws(1, 1141, 32, 128, 128, 64)
    # varlen bound covers every split of the tokens into num_seqs sequences
    vws = lib.deltanet_prefill_varlen_workspace_size
    lens = [1427, 3804, 2613, 3898, 660, 2279, 4069, 1111]
    chunks = sum((n + 63) // 64 for n in lens)
    assert vws(sum(lens), 8, 32, 128, 128, 64) >= ws(1, 64 * chunks, 32, 128, 128, 64)
    assert vws(8 * 65, 8, 32, 128, 128, 64) >= ws(1, 64 * 16, 32, 128, 128, 64)
    assert vws(100, 0, 32, 128, 128, 64) == 0
    assert vws(0, 1, 32, 128, 128, 64) > 0


def _prefill_args(**over):
    a = dict(q=1, k=1, v=1, g=1, beta=1, o=1, s0=None, sf=1, B=1, T=64, HV=4, HQK=2, DK=128,
             DV=128, chunk=64, ws=1, ws_bytes=1 << 40, stream=None, dbg=0)
    a.update(over)
    return a


def _call_prefill(lib, a):
    return lib.deltanet_chunk_prefill(a["q"], a["k"], a["v"], a["g"], a["beta"], a["o"], a["s0"],
                                      a["sf"], a["B"], a["T"], a["HV"], a["HQK"], a["DK"],
                                      a["DV"], a["chunk"], a["ws"], a["ws_bytes"], a["stream"],
                                      a["dbg"])


@pytest.mark.parametrize("bad", [dict(DK=64), dict(DV=256), dict(chunk=32), dict(HQK=3),
                                 dict(HV=0), dict(B=0), dict(T=-1), dict(ws=None),
                                 dict(sf=None), dict(q=None), dict(ws_bytes=16)])
def test_prefill_rejects_on_host(lib, bad):
    assert _call_prefill(lib, _prefill_args(**bad)) == INVALID


def test_timed_prefill_rejects_bad_events(lib):
    n = lib.deltanet_prefill_kernel_count()
    assert n >= 1
    assert all(lib.deltanet_prefill_kernel_name(i) for i in range(n))
    assert lib.deltanet_prefill_kernel_name(n) is None
    ev = (ct.c_void_p * (n + 1))()
    a = _prefill_args()
    args = [a[x] for x in ("q", "k", "v", "g", "beta", "o", "s0", "sf", "B", "T", "HV", "HQK",
                           "DK", "DV", "chunk", "ws", "ws_bytes", "stream")]
    assert lib.deltanet_chunk_prefill_timed(*args, None, n + 1) == INVALID
    assert lib.deltanet_chunk_prefill_timed(*args, ev, n) == INVALID
    assert lib.deltanet_chunk_prefill_timed(*args, ev, n + 1) == INVALID   # null events


def test_single_kernel_rejects_bad_index(lib):
    n = lib.deltanet_prefill_kernel_count()
    a = _prefill_args()
    args = [a[x] for x in ("q", "k", "v", "g", "beta", "o", "s0", "sf", "B", "T", "HV", "HQK",
                           "DK", "DV", "chunk", "ws", "ws_bytes", "stream")]
    assert lib.deltanet_chunk_prefill_kernel(*args, -1) == INVALID
    assert lib.deltanet_chunk_prefill_kernel(*args, n) == INVALID
    bad = _prefill_args(DK=64)
    bargs = [bad[x] for x in ("q", "k", "v", "g", "beta", "o", "s0", "sf", "B", "T", "HV", "HQK",
                              "DK", "DV", "chunk", "ws", "ws_bytes", "stream")]
    assert lib.deltanet_chunk_prefill_kernel(*bargs, 0) == INVALID


def test_varlen_rejects_on_host(lib):
    f = lib.deltanet_chunk_prefill_varlen
    ok = [1, 1, 1, 1, 1, 1, None, 1, 1, 2, 128, 4, 2, 128, 128, 64, 1, 1 << 40, None, 0]
    bad_cu = list(ok)
    bad_cu[8] = None
    assert f(*bad_cu) == INVALID
    bad_n = list(ok)
    bad_n[9] = 0
    assert f(*bad_n) == INVALID
    bad_dk = list(ok)
    bad_dk[13] = 64
    assert f(*bad_dk) == INVALID


def test_decode_and_norm_reject_on_host(lib):
    dec = lib.deltanet_recurrent_step
    assert dec(1, 1, 1, 1, 1, 1, 1, 2, 1, 4, 3, 128, 128, None) == INVALID   # HV % HQK
    assert dec(1, 1, 1, 1, 1, 1, 1, 2, 1, 4, 2, 64, 128, None) == INVALID    # DK
    assert dec(1, 1, 1, 1, 1, 1, None, 2, 1, 4, 2, 128, 128, None) == INVALID
    nrm = lib.gdn_gated_rmsnorm_forward
    assert nrm(1, 1, 1, 1, 10, 96, 1e-6, capi.DTYPE_BF16, capi.DTYPE_BF16, None) == INVALID
    assert nrm(1, 1, 1, 1, 10, 128, 1e-6, capi.DTYPE_FP32, capi.DTYPE_FP32, None) == INVALID
    assert nrm(1, 1, 1, 1, 10, 128, 1e-6, capi.DTYPE_BF16, capi.DTYPE_FP16, None) == INVALID
    assert nrm(None, 1, 1, 1, 10, 128, 1e-6, capi.DTYPE_BF16, capi.DTYPE_BF16, None) == INVALID


def test_fused_prefill_rejects_on_host(lib):
    f = lib.deltanet_chunk_prefill_fused
    # q, k, v, a, b, A_log, dt_bias, o, state, B, T, HV, HQK, io dtype, ws, ws bytes, stream
    ok = [1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 64, 4, 2, capi.DTYPE_FP16, 1, 1 << 40, None]

    def c(**over):
        a = list(ok)
        for i, v in over.items():
            a[int(i[1:])] = v
        return f(*a)

    assert c(a13=capi.DTYPE_FP32) == INVALID                 # fp32 I/O
    assert c(a12=3) == INVALID                               # HV % HQK
    assert c(a8=None) == INVALID                             # no state
    assert c(a3=None) == INVALID and c(a5=None) == INVALID and c(a6=None) == INVALID
    assert c(a14=None) == INVALID
    assert c(a15=16) == INVALID                              # short workspace
    assert c(a9=0) == INVALID


def test_l2norm_prefill_rejects_on_host(lib):
    f = lib.deltanet_chunk_prefill_l2norm
    # q, k, v, g, beta, o, s0, sf, cu, num_seqs, B, T, HV, HQK, ws, ws bytes, stream
    ok = [1, 1, 1, 1, 1, 1, None, 1, None, 0, 1, 64, 4, 2, 1, 1 << 40, None]

    def c(**over):
        a = list(ok)
        for i, v in over.items():
            a[int(i[1:])] = v
        return f(*a)

    assert c(a13=3) == INVALID                               # HV % HQK
    assert c(a8=1, a9=2, a10=2) == INVALID                   # packed needs B = 1
    assert c(a8=1, a9=0) == INVALID                          # packed needs num_seqs > 0
    assert c(a7=None) == INVALID and c(a14=None) == INVALID
    assert c(a0=None) == INVALID and c(a3=None) == INVALID
    assert c(a15=16) == INVALID                              # short workspace


def test_conv_reject_on_host(lib):
    fwd = lib.gdn_causal_conv1d_fwd
    bf, fp32 = capi.DTYPE_BF16, capi.DTYPE_FP32
    # x, w, bias, y, B, T, D, K, strides (x b/t, y b/t), io, w dtype, silu, stream
    ok = [16, 16, None, 16, 1, 8, 64, 4, 0, 64, 0, 64, bf, bf, 1, None]

    def f(**over):
        a = list(ok)
        for i, v in over.items():
            a[int(i[1:])] = v
        return fwd(*a)

    assert f(a7=5) == INVALID and f(a7=1) == INVALID          # K outside 2..4
    assert f(a6=60) == INVALID                                # D % 8
    assert f(a12=fp32, a13=fp32) == INVALID                   # fp32 activations
    assert f(a13=capi.DTYPE_FP16) == INVALID                  # mixed 16-bit dtypes
    assert f(a14=2) == INVALID                                # silu flag
    assert f(a9=68) == INVALID                                # token stride not 8-aligned
    assert f(a0=8) == INVALID                                 # x not 16-byte aligned
    assert f(a0=None) == INVALID and f(a1=None) == INVALID and f(a3=None) == INVALID
    assert f(a4=0) == 0 and f(a5=0) == 0                      # empty: nothing to launch
    upd = lib.gdn_causal_conv1d_update
    # x, state, w, bias, y, B, T, D, K, L, x b/t/d, s b/d, y b/t/d, io, w dtype, silu, stream
    uok = [16, 16, 16, None, 16, 1, 1, 64, 4, 4, 64, 64, 1, 256, 4, 64, 64, 1, bf, fp32, 1, None]

    def u(**over):
        a = list(uok)
        for i, v in over.items():
            a[int(i[1:])] = v
        return upd(*a)

    assert u(a9=2) == INVALID and u(a9=9) == INVALID          # state_len outside K-1..8
    assert u(a8=5) == INVALID
    assert u(a1=None) == INVALID and u(a2=None) == INVALID
    assert u(a18=fp32) == INVALID
    assert u(a6=0) == 0


def test_torch_extension_loads_and_checks_device():
    import torch

    ops = gdn_hip.load()
    for name in ("chunk_prefill", "chunk_prefill_debug", "recurrent_step", "gated_rmsnorm",
                 "chunk_prefill_fused", "causal_conv1d_fwd", "causal_conv1d_update"):
        assert hasattr(ops, name)
    q = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16)
    v = torch.zeros(1, 64, 4, 128, dtype=torch.bfloat16)
    g = torch.zeros(1, 64, 4)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.chunk_prefill(q, q, v, g, g, None)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.gated_rmsnorm(v, v, torch.ones(128, dtype=torch.bfloat16), 1e-6)
    x = torch.zeros(1, 64, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.causal_conv1d_fwd(x, torch.zeros(64, 4, dtype=torch.bfloat16), None, True)


def test_reference_module_names_import():
    """The harness's module names (kernels/harness/parity_cuda.py:56,
    kernels/parity_tco.py:28) import and expose its two ops."""
    import importlib

    for name in ("deltanet_chunk_cuda", "deltanet_chunk_cuda_tco"):
        mod = importlib.import_module(name)
        assert callable(mod.chunk_prefill) and callable(mod.chunk_prefill_debug), name


def test_stream_probe_rejects_on_host(lib):
    """gdn_stream_probe's host checks: unknown kind, size not a multiple of
    16, missing buffers, and more than 4 pieces per lane for the one-pass
    kind 2."""
    p = 16
    assert lib.gdn_stream_probe(3, 0, p, p, p, 1024, 4, None) == INVALID
    assert lib.gdn_stream_probe(0, 0, p, p, p, 1000, 4, None) == INVALID
    assert lib.gdn_stream_probe(0, 0, None, p, p, 1024, 4, None) == INVALID
    assert lib.gdn_stream_probe(2, 1, p, None, p, 1024, 1, None) == INVALID
    assert lib.gdn_stream_probe(2, 1, p, p, p, 1024, 5, None) == INVALID
    assert lib.gdn_stream_probe(1, 0, None, None, None, 1024, 4, None) == INVALID


def test_twolevel_rejects_on_host(lib):
    """The two-level prototype's host checks: malformed host cu_seqlens (not
    starting at 0, decreasing), a bad segment count, a short workspace and a
    wrong event count are rejected before any launch."""
    cu_ok = (ct.c_int32 * 3)(0, 100, 300)
    p = ct.cast(cu_ok, ct.c_void_p)
    size = lib.deltanet_prefill_twolevel_workspace_size(p, 2, 300, 4, 3)
    assert size > 0
    assert lib.deltanet_prefill_twolevel_workspace_size(None, 2, 150, 4, 3) > 0
    for cu in ((5, 100, 300), (0, 200, 100)):
        bad = (ct.c_int32 * 3)(*cu)
        assert lib.deltanet_prefill_twolevel_workspace_size(ct.cast(bad, ct.c_void_p), 2, 300, 4,
                                                            3) == 0
    assert lib.deltanet_prefill_twolevel_workspace_size(p, 2, 300, 4, 0) == 0
    d = 16
    base = [d, d, d, d, d, d, None, d, p, 2, 300, 4, 2]
    assert lib.deltanet_chunk_prefill_twolevel(*base, 3, d, size - 1, None, None, 0) == INVALID
    assert lib.deltanet_chunk_prefill_twolevel(*base, 0, d, size, None, None, 0) == INVALID
    assert lib.deltanet_chunk_prefill_twolevel(*base, 3, d, size, None, d, 5) == INVALID
    assert lib.deltanet_chunk_prefill_twolevel(d, d, d, d, d, d, None, d, p, 2, 300, 4, 3, 3, d,
                                               size, None, None, 0) == INVALID   # HV % HQK


def test_cols_entry_rejects_on_host(lib):
    """deltanet_chunk_prefill_cols: a slice width other than 0, 16 or 32, bad
    head counts, no sequences, a short workspace and missing pointers are
    rejected before any launch."""
    d = 16
    wsb = lib.deltanet_prefill_live_workspace_size(2, 64, 4, 128, 128, 64)
    base = [d, d, d, d, d, d, None, d, None, 2, 64, 4, 2, d, wsb, None]
    for cols in (8, 24, 48, 64, -16, 1):
        assert lib.deltanet_chunk_prefill_cols(*base, cols, 0) == INVALID
    assert lib.deltanet_chunk_prefill_cols(d, d, d, d, d, d, None, d, None, 2, 64, 4, 3, d, wsb,
                                           None, 32, 0) == INVALID          # HV % HQK
    assert lib.deltanet_chunk_prefill_cols(d, d, d, d, d, d, None, d, None, 0, 64, 4, 2, d, wsb,
                                           None, 32, 0) == INVALID          # no sequences
    assert lib.deltanet_chunk_prefill_cols(d, d, d, d, d, d, None, d, None, 2, 64, 4, 2, d, wsb - 1,
                                           None, 32, 0) == INVALID          # short workspace
    assert lib.deltanet_chunk_prefill_cols(d, d, None, d, d, d, None, d, None, 2, 64, 4, 2, d, wsb,
                                           None, 16, 0) == INVALID          # no v
    assert lib.deltanet_chunk_prefill_cols(d, d, d, d, d, d, None, None, None, 2, 64, 4, 2, d, wsb,
                                           None, 0, 0) == INVALID           # no final state
