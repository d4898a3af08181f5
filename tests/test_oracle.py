"""Pins the CPU oracle (oracle/gdn_oracle.py) without trusting it.

Each check is independent of the oracle's own formulas: a brute-force fp64
projector recurrence, closed forms, a library routine, the installed
transformers functions the reference gates against
(kernels/harness/parity_test.py:22-27), or an invariance of the exact
algorithm.  The "mutant" tests plant a plausible mistake in a copy of the
oracle's chunked core (CPU only) and require the pins to catch it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import gdn_cases as gc
from oracle import gdn_oracle as orc

F64 = torch.float64


def _inputs(seed, B=1, T=150, HK=2, HV=4, D=32, s0=True, g_shift=0.0):
    q, k, v, g, beta, st = gc.make_gdn_inputs(seed, B=B, T=T, HK=HK, HV=HV, D=D,
                                              g_shift=g_shift, s0_scale=0.3, with_s0=s0)
    return q.double(), k.double(), v.double(), g.double(), beta.double(), \
        (None if st is None else st.double())


def _err(a, b):
    return (torch.as_tensor(a, dtype=F64) - torch.as_tensor(b, dtype=F64)).abs().max().item()


# ---------------------------------------------------------------- chunked form


@pytest.mark.parametrize("T", [1, 17, 64, 65, 150])
@pytest.mark.parametrize("with_s0", [False, True])
def test_chunked_equals_fp64_recurrence(T, with_s0):
    q, k, v, g, beta, s0 = _inputs(T, T=T, s0=with_s0)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    o_r, S_r = orc.recurrence_fp64(q, k, v, g, beta, s0)
    assert _err(o, o_r) < 1e-10 and _err(S, S_r) < 1e-10


def test_recurrent_equals_fp64_recurrence():
    q, k, v, g, beta, s0 = _inputs(5, B=2, T=40)
    o, S = orc.recurrent_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    o_r, S_r = orc.recurrence_fp64(q, k, v, g, beta, s0)
    assert _err(o, o_r) < 1e-12 and _err(S, S_r) < 1e-12


@pytest.mark.parametrize("C", [16, 32])
def test_chunk_size_invariance(C):
    q, k, v, g, beta, s0 = _inputs(8, T=130)
    o64, S64 = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, chunk_size=64, dtype=F64)
    oc, Sc = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, chunk_size=C, dtype=F64)
    assert _err(o64, oc) < 1e-10 and _err(S64, Sc) < 1e-10


@pytest.mark.parametrize("split", [64, 100])
def test_resume_invariance(split):
    q, k, v, g, beta, s0 = _inputs(9, T=170)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    o1, S1 = orc.chunk_gated_delta_rule(q[:, :split], k[:, :split], v[:, :split],
                                        g[:, :split], beta[:, :split], s0, dtype=F64)
    o2, S2 = orc.chunk_gated_delta_rule(q[:, split:], k[:, split:], v[:, split:],
                                        g[:, split:], beta[:, split:], S1, dtype=F64)
    assert _err(torch.cat([o1, o2], 1), o) < 1e-10 and _err(S2, S) < 1e-10


def test_gqa_equals_repeat_interleave():
    q, k, v, g, beta, s0 = _inputs(10, T=70, HK=2, HV=6)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    # explicit expansion: v-head h reads k-head h // 3 (kernels/chunk_delta_cuda.h:12-14)
    idx = torch.tensor([h // 3 for h in range(6)])
    oe, Se = orc.chunk_gated_delta_rule(q[:, :, idx], k[:, :, idx], v, g, beta, s0, dtype=F64)
    assert torch.equal(o, oe) and torch.equal(S, Se)
    assert torch.equal(orc.expand_kv_heads(q, 6)[:, :, 5], q[:, :, 1])


def test_tail_padding_leaves_state_and_outputs():
    q, k, v, g, beta, s0 = _inputs(11, T=90)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    pad = 23
    z = lambda x: torch.cat([x, torch.zeros_like(x[:, :pad])], 1)  # noqa: E731
    op, Sp = orc.chunk_gated_delta_rule(z(q), z(k), z(v), z(g), z(beta), s0, dtype=F64)
    assert _err(op[:, :90], o) < 1e-12 and _err(Sp, S) < 1e-12
    assert _err(op[:, 90:], 0) < 1e-12                       # padded q = 0 gives o = 0


def test_beta_zero_is_pure_decay():
    q, k, v, g, beta, s0 = _inputs(12, T=100)
    beta = torch.zeros_like(beta)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    c = g.cumsum(1)                                           # [B, T, HV]
    S_exp = s0 * c[:, -1].exp()[..., None, None]
    qe = orc.expand_kv_heads(q, 4) / math.sqrt(q.shape[-1])
    o_exp = torch.einsum("bthk,bhkv->bthv", qe, s0) * c.exp()[..., None]
    assert _err(S, S_exp) < 1e-12 and _err(o, o_exp) < 1e-12


def test_single_token_closed_form():
    q, k, v, g, beta, _ = _inputs(13, T=1, HK=4, HV=4, s0=False)
    g = torch.zeros_like(g)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, None, dtype=F64)
    s = 1 / math.sqrt(q.shape[-1])
    qk = (q[0, 0] * k[0, 0]).sum(-1)                          # [H]
    o_exp = s * beta[0, 0, :, None] * qk[:, None] * v[0, 0]
    S_exp = beta[0, 0, :, None, None] * k[0, 0, :, :, None] * v[0, 0, :, None, :]
    assert _err(o[0, 0], o_exp) < 1e-14 and _err(S[0], S_exp) < 1e-14


def test_output_linear_in_q():
    q, k, v, g, beta, s0 = _inputs(14, T=80)
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    o3, S3 = orc.chunk_gated_delta_rule(3 * q, k, v, g, beta, s0, dtype=F64)
    assert _err(o3, 3 * o) < 1e-12 and torch.equal(S3, S)


def test_unit_lower_inverse_matches_solve_triangular():
    gen = torch.Generator().manual_seed(15)
    A = torch.tril(torch.randn(3, 64, 64, generator=gen, dtype=F64) * 0.2, -1)
    X = orc.unit_lower_inverse(A)
    eye = torch.eye(64, dtype=F64).expand(3, 64, 64)
    ref = torch.linalg.solve_triangular(eye - A, eye, upper=False, unitriangular=True)
    assert _err(X, ref) < 1e-10


def test_chunk_debug_views_pinned():
    """chunk_debug_views: T against solve_triangular(I - A); the chunk-entry
    states against the independent fp64 token recurrence run over each
    prefix; M through the first chunk's closed form o = M T diag(beta) V
    (zero initial state), with o from that same recurrence; c as the per-chunk
    cumulative sum of g."""
    q, k, v, g, beta, s0 = [t.double() for t in gc.make_gdn_inputs(21, B=1, T=150, HK=1, HV=2,
                                                                  D=32)]
    views = orc.chunk_debug_views(q, k, v, g, beta, s0, dtype=torch.float64)
    A, Tm, M, c, S = views["A"], views["T"], views["M"], views["c"], views["S"]
    nc = 3
    assert A.shape == (nc, 2, 64, 64) and S.shape == (nc, 2, 32, 32) and c.shape == (nc, 2, 64)
    eye = torch.eye(64, dtype=torch.float64)
    inv = torch.linalg.solve_triangular(eye - A, eye, upper=False, unitriangular=True)
    assert torch.allclose(Tm, inv, atol=1e-12)
    for n in range(nc):
        if n == 0:
            ref = s0.double()[0]
        else:
            _, sr = orc.recurrence_fp64(q[:, :64 * n], k[:, :64 * n], v[:, :64 * n],
                                        g[:, :64 * n], beta[:, :64 * n], s0)
            ref = torch.from_numpy(sr[0])
        assert torch.allclose(S[n], ref, atol=1e-10), n
    gp = F.pad(g.double(), (0, 0, 0, 42))[0].reshape(nc, 64, 2).permute(0, 2, 1)
    assert torch.allclose(c, gp.cumsum(-1), atol=1e-12)
    o_rec, _ = orc.recurrence_fp64(q[:, :64], k[:, :64], v[:, :64], g[:, :64], beta[:, :64])
    vb = v[0, :64].double().permute(1, 0, 2) * beta[0, :64].double().t().unsqueeze(-1)
    o_m = M[0] @ (Tm[0] @ vb)                      # [H, 64, DV]
    assert torch.allclose(o_m, torch.from_numpy(o_rec[0]).permute(1, 0, 2), atol=1e-10)


def test_varlen_is_independent_per_sequence():
    lens = [0, 1, 63, 70, 5]
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    q, k, v, g, beta, _ = _inputs(16, T=int(cu[-1]), HK=1, HV=2)
    s0 = 0.3 * torch.randn(len(lens), 2, 32, 32, generator=torch.Generator().manual_seed(1),
                           dtype=F64)
    o, sf = orc.chunk_gated_delta_rule_varlen(q, k, v, g, beta, cu, s0, dtype=F64)
    for i, L in enumerate(lens):
        a = int(cu[i])
        if L == 0:
            assert torch.equal(sf[i], s0[i])
            continue
        o_r, S_r = orc.recurrence_fp64(q[:, a:a + L], k[:, a:a + L], v[:, a:a + L],
                                       g[:, a:a + L], beta[:, a:a + L], s0[i:i + 1])
        assert _err(o[:, a:a + L], o_r) < 1e-10 and _err(sf[i], S_r[0]) < 1e-10


def test_fp32_oracle_close_to_fp64():
    q, k, v, g, beta, s0 = _inputs(17, T=200, D=128, HK=1, HV=2)
    o32, S32 = orc.chunk_gated_delta_rule(q.float(), k.float(), v.float(), g.float(),
                                          beta.float(), s0.float(), dtype=torch.float32)
    o64, S64 = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=F64)
    assert _err(o32, o64) < 1e-4 and _err(S32, S64) < 1e-4


# ------------------------------------------------- mutants must fail the pins


def _mutant_chunk(q, k, v, g, beta, s0, mutation):
    """The oracle's chunked formulas with one planted mistake (test only)."""
    B, T, H, D = q.shape
    C = 64
    qh, kh, vh = (x.transpose(1, 2) for x in (q, k, v))
    gh, bh = g.transpose(1, 2), beta.transpose(1, 2)
    n = T // C
    S = s0.clone()
    s = 1 / math.sqrt(D)
    outs = []
    for i in range(n):
        sl = slice(i * C, (i + 1) * C)
        qi, ki, vi = qh[:, :, sl] * s, kh[:, :, sl], vh[:, :, sl]
        c = gh[:, :, sl].cumsum(-1)
        bi = bh[:, :, sl]
        diff = c[..., :, None] - c[..., None, :]
        if mutation == "gamma_sign":
            diff = -diff
        gam = torch.tril(diff.exp())
        A = -torch.tril((ki * bi[..., None]) @ ki.transpose(-1, -2) * gam, -1)
        Tm = orc.unit_lower_inverse(A)
        U = Tm @ (vi * bi[..., None])
        W = Tm @ (ki * (bi * c.exp())[..., None])
        vn = U if mutation == "drop_ws" else U - W @ S
        M = (qi @ ki.transpose(-1, -2)) * gam
        if mutation == "transpose_m":
            M = M.transpose(-1, -2)
        outs.append((qi * c.exp()[..., None]) @ S + M @ vn)
        S = S * c[..., -1:, None].exp() + (ki * (c[..., -1:] - c).exp()[..., None]).transpose(-1, -2) @ vn
    return torch.cat(outs, 2).transpose(1, 2), S


@pytest.mark.parametrize("mutation", [None, "gamma_sign", "drop_ws", "transpose_m"])
def test_pins_detect_planted_mistakes(mutation):
    q, k, v, g, beta, s0 = _inputs(18, T=128, HK=2, HV=2)
    o, S = _mutant_chunk(q, k, v, g, beta, s0, mutation)
    o_r, S_r = orc.recurrence_fp64(q, k, v, g, beta, s0)
    err = max(_err(o, o_r), _err(S, S_r))
    if mutation is None:
        assert err < 1e-10
    else:
        assert err > 1e-3, f"pin missed planted mistake {mutation}"


# ---------------------------------------------------------- rmsnorm, l2, gate


def test_gated_rmsnorm_closed_form():
    # constant rows: rms = |a|, so n = a / sqrt(a^2 + eps) exactly representable
    x = torch.full((4, 128), 2.0, dtype=torch.bfloat16)
    z = torch.full((4, 128), 30.0, dtype=torch.bfloat16)          # silu(30) = 30 (fp32)
    w = torch.full((128,), 0.5, dtype=torch.bfloat16)
    y = orc.gated_rmsnorm(x, z, w, eps=0.0)
    assert torch.equal(y, torch.full((4, 128), 15.0, dtype=torch.bfloat16))
    y0 = orc.gated_rmsnorm(x, torch.zeros_like(z), w, eps=0.0)
    assert torch.equal(y0, torch.zeros_like(y0))                  # silu(0) = 0


@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_gated_rmsnorm_matches_library_composition(wdt):
    x, z, w, eps = gc.rmsnorm_inputs(rows_t=7, heads=3)
    w = w.to(wdt)
    y = orc.gated_rmsnorm(x, z, w, eps)
    n = F.rms_norm(x.float(), (128,), eps=eps).to(torch.bfloat16)
    ref = ((w * n) * F.silu(z.float())).to(torch.bfloat16)
    assert torch.equal(y, ref)


def test_gated_rmsnorm_matches_transformers():
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    x, z, w, eps = gc.rmsnorm_inputs(rows_t=9, heads=4)
    mod = m.Qwen3_5RMSNormGated(128, eps=eps).to(torch.bfloat16)
    with torch.no_grad():
        mod.weight.copy_(w)
        ref = mod(x, z)
    assert torch.equal(orc.gated_rmsnorm(x, z, w, eps), ref)


def test_l2norm_unit_rows():
    x = torch.randn(50, 128, generator=torch.Generator().manual_seed(19), dtype=F64)
    n = orc.l2norm(x)
    assert _err(n.norm(dim=-1), torch.ones(50)) < 1e-6
    assert torch.equal(orc.l2norm(torch.zeros(3, 8)), torch.zeros(3, 8))


def test_gate_closed_form():
    a = torch.zeros(2, 3, 4)
    g, beta = orc.gdn_gate(a, a, torch.zeros(4), torch.zeros(4))
    assert _err(g, -math.log(2)) < 1e-7 and _err(beta, 0.5) < 1e-7
    g2, _ = orc.gdn_gate(a, a, torch.full((4,), math.log(3.0)), torch.full((4,), 50.0))
    assert _err(g2, -150.0) < 1e-3                                # softplus(50) = 50
    gen = torch.Generator().manual_seed(20)
    g3, b3 = orc.gdn_gate(torch.randn(5, 4, generator=gen), torch.randn(5, 4, generator=gen),
                          torch.randn(4, generator=gen), torch.randn(4, generator=gen))
    assert (g3 <= 0).all() and ((b3 > 0) & (b3 < 1)).all()


# ------------------------------------------ installed transformers functions


def test_matches_transformers_chunk_and_recurrent():
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    q, k, v, g, beta, s0 = gc.plumbing_inputs()
    s0 = 0.1 * torch.randn(s0.shape, generator=torch.Generator().manual_seed(2))
    o, S = orc.chunk_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float32)
    o_t, S_t = m.torch_chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0,
                                              output_final_state=True)
    assert _err(o, o_t) < 1e-5 and _err(S, S_t) < 1e-5
    o_r, S_r = orc.recurrent_gated_delta_rule(q, k, v, g, beta, s0, dtype=torch.float32)
    o_rt, S_rt = m.torch_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0,
                                                    output_final_state=True)
    assert _err(o_r, o_rt) < 1e-5 and _err(S_r, S_rt) < 1e-5
    assert _err(orc.l2norm(v), m.l2norm(v, dim=-1, eps=1e-6)) == 0.0


# ------------------------------------------------------- causal conv1d (f3)


def _conv_brute(x, w, bias, silu):
    """Depthwise causal correlation by explicit loops in Python floats
    (fp64), x [B, D, T], w [D, K]; no dtype steps (fp32 inputs)."""
    B, D, T = x.shape
    K = w.shape[1]
    y = torch.zeros(B, D, T, dtype=F64)
    for b in range(B):
        for d in range(D):
            for t in range(T):
                s = 0.0 if bias is None else float(bias[d])
                for j in range(K):
                    tt = t - (K - 1) + j
                    if tt >= 0:
                        s += float(w[d, j]) * float(x[b, d, tt])
                y[b, d, t] = s / (1.0 + math.exp(-s)) if silu else s
    return y


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("silu", [False, True])
def test_conv_matches_brute_force(K, silu):
    gen = torch.Generator().manual_seed(30 + K)
    x = torch.randn(2, 5, 9, generator=gen)
    w = torch.randn(5, K, generator=gen)
    bias = torch.randn(5, generator=gen)
    for bb in (None, bias):
        y = orc.causal_conv1d(x, w, bb, "silu" if silu else None)
        assert _err(y, _conv_brute(x, w, bb, silu)) < 1e-5


def test_conv_closed_forms():
    # a unit impulse at token 3 reproduces the taps in reverse time order
    x = torch.zeros(1, 2, 8)
    x[0, :, 3] = 1.0
    w = torch.tensor([[1.0, 2.0, 3.0, 4.0], [-1.0, 0.5, 0.25, 8.0]])
    y = orc.causal_conv1d(x, w)
    assert torch.equal(y[0, :, 3:7], w.flip(-1))
    assert torch.equal(y[0, :, :3], torch.zeros(2, 3)) and torch.equal(y[0, :, 7], torch.zeros(2))
    # the first output only sees the newest tap (causality, zero history)
    x = torch.randn(1, 3, 5, generator=torch.Generator().manual_seed(3))
    w = torch.randn(3, 4, generator=torch.Generator().manual_seed(4))
    assert _err(orc.causal_conv1d(x, w)[0, :, 0], w[:, 3] * x[0, :, 0]) < 1e-7


def _conv_inputs(seed, io, wd, D=64, T=200, K=4, B=2):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=gen).to(io).transpose(1, 2)
    w = (0.5 * torch.randn(D, K, generator=gen)).to(wd)
    bias = (0.1 * torch.randn(D, generator=gen)).to(wd)
    return x, w, bias


def _tf_conv():
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    # the undecorated torch functions (the decorator may route to a package)
    return (getattr(m.causal_conv1d_fn, "__wrapped__", m.causal_conv1d_fn),
            getattr(m.causal_conv1d_update, "__wrapped__", m.causal_conv1d_update))


@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [2, 3, 4])
def test_conv_matches_transformers_bitwise(io, K):
    fn, _ = _tf_conv()
    x, w, bias = _conv_inputs(40 + K, io, io, K=K)
    for bb in (None, bias):
        for act in (None, "silu"):
            assert torch.equal(orc.causal_conv1d(x, w, bb, act), fn(x, w, bb, act))


def test_conv_fp32_weights_match_transformers_within_an_ulp():
    # fp32 convolution: torch's CPU kernel sums in another order, so the
    # final rounding to bf16 may differ by one unit in rare elements
    fn, _ = _tf_conv()
    x, w, bias = _conv_inputs(50, torch.bfloat16, torch.float32, D=256, T=300)
    a = orc.causal_conv1d(x, w, bias, "silu").float()
    r = fn(x, w, bias, "silu").float()
    ulp = torch.maximum(a.abs(), r.abs()).clamp_min(1e-30) * 2.0 ** -7
    assert ((a - r).abs() <= ulp).all()
    assert (a != r).float().mean().item() < 1e-3


@pytest.mark.parametrize("io", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 3])
def test_conv_update_matches_transformers(io, T):
    _, up = _tf_conv()
    gen = torch.Generator().manual_seed(60 + T)
    x = torch.randn(2, 64, T, generator=gen).to(io)
    st = torch.randn(2, 64, 4, generator=gen).to(io)
    w = (0.5 * torch.randn(64, 4, generator=gen)).to(io)
    bias = (0.1 * torch.randn(64, generator=gen)).to(io)
    st_t = st.clone()
    r = up(x, st_t, w, bias, "silu")
    y, ns = orc.causal_conv1d_update(x, st, w, bias, "silu")
    assert torch.equal(y, r) and torch.equal(ns, st_t)


@pytest.mark.parametrize("L", [3, 4, 6])
def test_conv_prefill_then_updates_equals_one_pass(L):
    # resuming from the carried state reproduces the one-pass outputs exactly
    x, w, bias = _conv_inputs(70, torch.bfloat16, torch.bfloat16, D=32, T=40)
    full = orc.causal_conv1d(x, w, bias, "silu")
    split = 29
    state = F.pad(x[:, :, :split], (L, 0))[:, :, -L:]   # zeros before the first token
    outs = [orc.causal_conv1d(x[:, :, :split], w, bias, "silu")]
    for t0, n in ((29, 1), (30, 3), (33, 1), (34, 6)):
        y, state = orc.causal_conv1d_update(x[:, :, t0:t0 + n], state, w, bias, "silu")
        outs.append(y)
    assert torch.equal(torch.cat(outs, dim=-1), full)
    assert torch.equal(state, x[:, :, -L:])


def _mutant_conv(x, w, bias, act, mutation):
    """The conv oracle's formula with one planted mistake (test only)."""
    K = w.shape[-1]
    T = x.shape[-1]
    xp = F.pad(x.to(w.dtype).float(), (K - 1, 0))
    wf = w.float().flip(-1) if mutation == "reversed_taps" else w.float()
    off = 1 if mutation == "shift" else 0
    xp = F.pad(xp, (off, 0))
    acc = sum(wf[None, :, j:j + 1] * xp[:, :, j:j + T] for j in range(K))
    if bias is not None:
        acc = acc + bias.float()[None, :, None]
    out = acc if mutation == "no_weight_rounding" else acc.to(w.dtype).float()
    if act is not None:
        out = F.silu(out)
    return out.to(x.dtype)


@pytest.mark.parametrize("mutation", ["reversed_taps", "shift", "no_weight_rounding"])
def test_conv_pins_detect_planted_mistakes(mutation):
    # fp32: the brute-force loop pin
    gen = torch.Generator().manual_seed(80)
    x = torch.randn(1, 6, 12, generator=gen)
    w = torch.randn(6, 4, generator=gen)
    brute_err = _err(_mutant_conv(x, w, None, "silu", mutation), _conv_brute(x, w, None, True))
    # bf16: the bitwise transformers pin
    fn, _ = _tf_conv()
    xb, wb, bb = _conv_inputs(81, torch.bfloat16, torch.bfloat16)
    tf_equal = torch.equal(_mutant_conv(xb, wb, bb, "silu", mutation), fn(xb, wb, bb, "silu"))
    assert brute_err > 1e-3 or not tf_equal, f"pins missed planted mistake {mutation}"


# ---------------------------------------------------- fused prefill (f2)


def test_fused_prefill_power_of_two_row_scales_are_invisible():
    # x 2^s changes neither the normalised rows (exact scaling; the sums of
    # squares stay far above the 1e-6 eps) nor anything downstream: pins
    # that q and k are normalised before use
    q, k, v, a, b, A_log, dt_bias, s0 = gc.fused_inputs(90, B=1, T=70, HK=2, HV=4, D=32)
    o1, S1 = orc.fused_prefill(q, k, v, a, b, A_log, dt_bias, s0)
    o2, S2 = orc.fused_prefill(q * 4, k * 0.5, v, a, b, A_log, dt_bias, s0)
    assert torch.equal(o1, o2) and torch.equal(S1, S2)
    o3, _ = orc.fused_prefill(q, k, v * 2, a, b, A_log, dt_bias, s0)
    assert not torch.equal(o1, o3)                       # v is not normalised


def test_fused_prefill_matches_transformers_l2norm_path():
    # transformers' own prefill with use_qk_l2norm_in_kernel=True on the raw
    # rows, gates from the same inputs; differences are the adapter's bf16
    # roundings of q, k, v and o only
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    chunk = getattr(m.torch_chunk_gated_delta_rule, "__wrapped__", m.torch_chunk_gated_delta_rule)
    q, k, v, a, b, A_log, dt_bias, s0 = gc.fused_inputs(91, B=1, T=150, HK=2, HV=2, D=128)
    o, S = orc.fused_prefill(q, k, v, a, b, A_log, dt_bias, s0)
    g, beta = orc.gdn_gate(a, b, A_log, dt_bias)
    o_t, S_t = chunk(q.float(), k.float(), v.float(), g, beta, initial_state=s0,
                     output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert _err(o, o_t) < 2e-2 and _err(S, S_t) < 2e-2
    assert (o.double() - o_t.double()).norm() / o_t.double().norm() < 1e-2


def test_fused_prefill_fp16_and_bf16_inputs_agree_on_shared_values():
    # values representable in both dtypes give the same result; o is the
    # bf16-rounded value, converted to fp16 for fp16 inputs (exact but for
    # fp16 subnormals, |o| < 6.1e-5)
    q, k, v, a, b, A_log, dt_bias, s0 = gc.fused_inputs(92, B=1, T=40, HK=1, HV=2, D=32)
    r = lambda x: (x.float() * 8).round() / 8                  # noqa: E731  dyadic, |x| < 8
    args16 = [r(t).to(torch.float16) for t in (q, k, v, a, b)]
    args_b = [r(t).to(torch.bfloat16) for t in (q, k, v, a, b)]
    o16, S16 = orc.fused_prefill(*args16, A_log, r(dt_bias).to(torch.float16), s0)
    ob, Sb = orc.fused_prefill(*args_b, A_log, r(dt_bias).to(torch.bfloat16), s0)
    assert o16.dtype == torch.float16 and ob.dtype == torch.bfloat16
    assert torch.equal(o16, ob.to(torch.float16)) and torch.equal(S16, Sb)
