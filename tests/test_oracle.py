"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the oracle (dropped term,
wrong sign, transposed operand, off-by-one mask, wrong rounding order) fails:
known answers from the reference's own tests, brute force on tiny inputs,
library routines (torch matmul/tril/autograd, torch bf16 casts), closed forms
in float64 and invariants.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
KA = json.loads((GOLDEN / "known_answers.json").read_text())


def _a(x):
    return np.asarray(x, dtype=np.float32)


def _rng(seed):
    return np.random.default_rng(seed)


# --------------------------------------------------------------------- bf16
def test_bf16_round_matches_torch_cast():
    rng = _rng(0)
    x = rng.standard_normal(100_000).astype(np.float32) * np.float32(3.0)
    # exact ties: bf16 value + half an ulp, both parities of the kept bit
    base = O.bf16_round(rng.standard_normal(1000).astype(np.float32))
    ulp_half = (base.view(np.uint32) & np.uint32(0x7F800000)).view(np.float32) * np.float32(2.0 ** -8)
    ties = (base + ulp_half).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 65504.0], np.float32)
    for arr in (x, ties, special):
        got = O.bf16_round(arr)
        want = torch.from_numpy(arr).to(torch.bfloat16).to(torch.float32).numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    nan = O.bf16_round(np.array([np.nan], np.float32))
    assert np.isnan(nan).all()


# --------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("n", [2, 8, 64, 8192])
def test_get_freqs_closed_form_and_pairs(n):
    f = O.get_freqs(n)
    assert f.dtype == np.float32 and f.shape == (n,)
    i = np.arange(n)
    exact = 1.0 / (65536.0 ** (2 * (i // 2) / n)) / (2 * math.pi)
    np.testing.assert_allclose(f.astype(np.float64), exact, rtol=4e-7, atol=0)
    assert np.array_equal(f[0::2], f[1::2])  # integer floor(i/2): pairs share a frequency
    assert f[0] == np.float32(1.0) / np.float32(2 * math.pi)


def test_rope_phases_positions_and_continuity():
    f = O.get_freqs(64)
    T, S = 37, 11
    ph = O.rope_phases(T, S, f)
    assert ph.shape == (T, 64)
    # column 0 has freq 1/(2 pi): phase = pos / (2 pi) to fp32 rounding
    pos = np.arange(S, S + T, dtype=np.float64)
    np.testing.assert_allclose(ph[:, 0], pos * float(f[0]), rtol=1e-7)
    # continuity (test_attention_mask.py:119-124): bit-exact
    assert np.array_equal(O.rope_phases(T, S, f), O.rope_phases(S + T, 0, f)[S:])


def test_phases_cos_sin_against_float64_trig():
    f = O.get_freqs(128)
    ph = O.rope_phases(300, 5, f)
    c, s = O.phases_cos_sin(ph)
    frac = ph.astype(np.float64) - np.floor(ph.astype(np.float64))
    theta = (frac.astype(np.float32) * np.float32(2 * math.pi)).astype(np.float64)
    np.testing.assert_allclose(c, np.cos(theta), atol=2e-7)
    np.testing.assert_allclose(s, np.sin(theta), atol=2e-7)
    # pair 0: theta == position mod 2*pi (freq = 1/(2 pi)), up to fp32 phase rounding
    pos = np.arange(5, 305, dtype=np.float64)
    assert np.max(np.abs(c[:, 0] - np.cos(pos))) < 2e-4
    assert np.max(np.abs(s[:, 0] - np.sin(pos))) < 2e-4


def test_rope_rotate_is_a_pairwise_rotation():
    rng = _rng(1)
    N, T = 32, 20
    x = rng.standard_normal((2, 3, T, N)).astype(np.float32)
    c, s = O.rope_cos_sin(T, 7, O.get_freqs(N))
    y = O.rope_rotate(x, c, s)
    # float64 dense 2x2 rotation matrix per pair (pairs share c, s)
    x64 = x.astype(np.float64).reshape(2, 3, T, N // 2, 2)
    c64 = c.astype(np.float64).reshape(T, N // 2, 2)[..., 0]
    s64 = s.astype(np.float64).reshape(T, N // 2, 2)[..., 0]
    R = np.stack([np.stack([c64, -s64], -1), np.stack([s64, c64], -1)], -2)  # (T,N/2,2,2)
    want = np.einsum("tpij,bhtpj->bhtpi", R, x64).reshape(2, 3, T, N)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)
    # pair norms preserved
    nx = np.linalg.norm(x64, axis=-1)
    ny = np.linalg.norm(y.astype(np.float64).reshape(2, 3, T, N // 2, 2), axis=-1)
    np.testing.assert_allclose(ny, nx, rtol=1e-5)
    # position 0 is the identity, exactly (cos 0 == 1, sin 0 == 0)
    c0, s0 = O.rope_cos_sin(1, 0, O.get_freqs(N))
    assert np.array_equal(O.rope_rotate(x[:, :, :1], c0, s0), x[:, :, :1])


def test_rope_rotate_bf16_order_matches_torch_bf16_ops():
    """bf16 x with fp32 cis: products rounded to bf16, then a bf16 add (rope.py:120-122)."""
    rng = _rng(2)
    N, T = 64, 16
    x = O.bf16_round(rng.standard_normal((2, 2, T, N)).astype(np.float32))
    c, s = O.rope_cos_sin(T, 3, O.get_freqs(N))
    got = O.rope_rotate(x, c, s, bf16=True)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    ct, st = torch.from_numpy(c), torch.from_numpy(s)
    x0, x1 = xt[..., 0::2], xt[..., 1::2]
    y0 = (x0 * ct[..., 0::2]).to(torch.bfloat16) + ((-x1) * st[..., 0::2]).to(torch.bfloat16)
    y1 = (x1 * ct[..., 1::2]).to(torch.bfloat16) + (x0 * st[..., 1::2]).to(torch.bfloat16)
    want = torch.stack((y0, y1), -1).reshape(xt.shape).float().numpy()
    assert np.array_equal(got, want)
    assert np.array_equal(O.bf16_round(got), got)


def test_rope_backward_is_the_adjoint():
    rng = _rng(3)
    N, T = 16, 9
    x = rng.standard_normal((1, 2, T, N))
    g = rng.standard_normal((1, 2, T, N))
    c, s = O.rope_cos_sin(T, 4, O.get_freqs(N))
    lhs = float(np.sum(O.rope_rotate(x, c, s).astype(np.float64) * g))
    rhs = float(np.sum(x * O.rope_rotate_backward(g, c, s).astype(np.float64)))
    assert abs(lhs - rhs) < 1e-4 * max(1.0, abs(lhs))
    # central finite difference on one coordinate pair
    eps = 1e-2
    for idx in [(0, 1, 3, 4), (0, 0, 8, 7)]:
        xp = x.copy(); xp[idx] += eps
        xm = x.copy(); xm[idx] -= eps
        fd = (np.sum(O.rope_rotate(xp, c, s) * g) - np.sum(O.rope_rotate(xm, c, s) * g)) / (2 * eps)
        an = O.rope_rotate_backward(g, c, s)[idx]
        assert abs(fd - an) < 1e-3


# --------------------------------------------------------- cold forward
def test_known_answer_raw_tril():
    k = KA["raw_tril_fwd_bwd"]
    out = O.tril_score_v_cpu(_a(k["q"]), _a(k["k"]), _a(k["v"]))
    assert np.array_equal(out, _a(k["out"]))


def test_known_answer_self_attn():
    k = KA["self_attn_single_query"]
    q = _a(k["q"])
    assert np.array_equal(O.tril_score_v_cpu(q, q, _a(k["v"])), _a(k["out"]))


def test_known_answer_bench_cold():
    k = KA["bench_cold"]
    assert np.array_equal(O.tril_score_v_cpu(_a(k["q"]), _a(k["k"]), _a(k["v"])), _a(k["out"]))


@pytest.mark.parametrize("shape", [(1, 1, 5, 3, 2, 1), (2, 3, 7, 4, 5, 3), (1, 2, 9, 6, 2, 1)])
def test_cold_matches_bruteforce(shape):
    B, H, T, Dk, Dv, Hv = shape
    rng = _rng(4)
    q = rng.standard_normal((B, H, T, Dk)).astype(np.float32)
    k = rng.standard_normal((B, H, T, Dk)).astype(np.float32)
    v = rng.standard_normal((B, Hv, T, Dv)).astype(np.float32)
    got = O.tril_score_v_cpu(q, k, v)
    np.testing.assert_allclose(got, O.tril_score_v_bruteforce(q, k, v), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T", [1, 2, 63, 255, 256, 300, 700])
def test_cold_eager_and_tiled_match_torch(T):
    rng = _rng(T)
    q = rng.standard_normal((1, 2, T, 8)).astype(np.float32)
    v = rng.standard_normal((1, 1, T, 5)).astype(np.float32)
    got = O.tril_score_v_cpu(q, q, v)
    qt = torch.from_numpy(q).double()
    want = ((qt @ qt.mT).tril(-1) @ torch.from_numpy(v).double()).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    assert np.array_equal(got[:, :, 0], np.zeros_like(got[:, :, 0]))  # row 0 exactly 0


def test_cold_tiled_chunked_past_path():
    """T=2048 makes Bi*i0 exceed the budget, so the past is key-chunked."""
    T = 2048
    assert 128 * 1152 > O.cold_score_budget(T, 128)
    rng = _rng(5)
    q = rng.standard_normal((1, 1, T, 4)).astype(np.float32)
    v = rng.standard_normal((1, 1, T, 3)).astype(np.float32)
    got = O.tril_score_v_tiled(q, q, v)
    want = O.tril_score_v_eager(q.astype(np.float64), q.astype(np.float64), v.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-3)


def test_cold_upper_triangle_never_contributes_and_linear_in_v():
    rng = _rng(6)
    T = 12
    q = rng.standard_normal((1, 1, T, 6)).astype(np.float32)
    v1 = rng.standard_normal((1, 1, T, 4)).astype(np.float32)
    v2 = rng.standard_normal((1, 1, T, 4)).astype(np.float32)
    base = O.tril_score_v_cpu(q, q, v1)
    # poisoning the last key/value changes no output row (nobody attends to row T-1)
    q2 = q.copy(); q2[:, :, -1] = 1e3
    v3 = v1.copy(); v3[:, :, -1] = -1e3
    k2 = q.copy(); k2[:, :, -1] = 1e3
    got = O.tril_score_v_cpu(q, k2, v3)
    np.testing.assert_allclose(got, base, rtol=1e-6, atol=1e-6)
    lin = O.tril_score_v_cpu(q, q, 2 * v1 - 3 * v2)
    np.testing.assert_allclose(lin, 2 * base - 3 * O.tril_score_v_cpu(q, q, v2), rtol=1e-4, atol=1e-4)


def test_cold_contract_errors():
    z = np.zeros((1, 1, 3, 2), np.float32)
    with pytest.raises(ValueError):
        O.tril_score_v_cpu(z, np.zeros((1, 1, 4, 2), np.float32), z[..., :1])
    with pytest.raises(ValueError):
        O.tril_score_v_cpu(z, z, np.zeros((1, 3, 3, 1), np.float32))  # v heads not in {1, H}


# ----------------------------------------------------------------- decode
def test_known_answer_decode():
    k = KA["decode_raw"]
    assert np.array_equal(O.tril_decode_cpu(_a(k["q"]), _a(k["k_past"]), _a(k["v_past"])), _a(k["out"]))
    k = KA["bench_decode"]
    assert np.array_equal(O.tril_decode_cpu(_a(k["q"]), _a(k["k_past"]), _a(k["v_past"])), _a(k["out"]))


@pytest.mark.parametrize("S,Tq", [(1, 1), (17, 1), (40, 3), (600, 128)])
def test_decode_is_last_rows_of_full_tril(S, Tq):
    """Decode of queries at positions >= S against past [0,S) == rows of the full op."""
    rng = _rng(S)
    H, N, D = 2, 8, 4
    past = rng.standard_normal((1, H, S, N)).astype(np.float32)
    vpast = rng.standard_normal((1, 1, S, D)).astype(np.float32)
    q = rng.standard_normal((1, H, 1, N)).astype(np.float32)
    full_k = np.concatenate([past, q], axis=2)
    full_v = np.concatenate([vpast, 1e3 * np.ones((1, 1, 1, D), np.float32)], axis=2)  # poisoned new V
    want = O.tril_score_v_cpu(full_k, full_k, full_v)[:, :, -1:]
    got = O.tril_decode_cpu(q, past, vpast)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    qm = rng.standard_normal((1, H, Tq, N)).astype(np.float32)
    np.testing.assert_allclose(
        O.tril_decode_cpu(qm, past, vpast), O.tril_decode_bruteforce(qm, past, vpast) if S * Tq < 5000 else
        O.tril_decode_eager(qm.astype(np.float64), past.astype(np.float64), vpast.astype(np.float64)),
        rtol=1e-4, atol=1e-4)


def test_decode_empty_past_is_zero():
    q = np.ones((2, 3, 1, 4), np.float32)
    out = O.tril_decode_cpu(q, np.zeros((2, 3, 0, 4), np.float32), np.zeros((2, 1, 0, 5), np.float32))
    assert out.shape == (2, 3, 1, 5) and not out.any()


# --------------------------------------------------------------- backward
def test_known_answer_backward():
    k = KA["raw_tril_fwd_bwd"]
    dq, dk, dv = O.analytic_tril_attn_backward(_a(k["q"]), _a(k["k"]), _a(k["v"]), _a(k["dout"]))
    assert np.array_equal(dq, _a(k["dq"])) and np.array_equal(dk, _a(k["dk"])) and np.array_equal(dv, _a(k["dv"]))
    dq, dk, dv = O.analytic_tril_attn_backward_blocked(_a(k["q"]), _a(k["k"]), _a(k["v"]), _a(k["dout"]))
    assert np.array_equal(dq, _a(k["dq"])) and np.array_equal(dk, _a(k["dk"])) and np.array_equal(dv, _a(k["dv"]))


def test_known_answer_self_backward():
    k = KA["self_attn_single_query"]
    for blocked in (False, True):
        dqm, dv = O.self_attn_backward(_a(k["q"]), _a(k["v"]), _a(k["dout"]), blocked=blocked)
        assert np.array_equal(dqm, _a(k["dq_merged"]))
        assert np.array_equal(dv, _a(k["dv"]))


def test_zero_upstream_gives_zero_grads():
    rng = _rng(2042)
    q = rng.standard_normal((2, 2, 4, 3)); kk = rng.standard_normal((2, 2, 4, 3))
    v = rng.standard_normal((2, 1, 4, 5))
    for g in O.analytic_tril_attn_backward_blocked(q, kk, v, np.zeros((2, 2, 4, 5))):
        assert not np.any(g)


@pytest.mark.parametrize("T,Hv", [(5, 1), (9, 3), (70, 1)])
def test_backward_matches_torch_autograd(T, Hv):
    rng = _rng(T)
    B, H, N, D = 2, 3, 6, 4
    q = rng.standard_normal((B, H, T, N)); k = rng.standard_normal((B, H, T, N))
    v = rng.standard_normal((B, Hv, T, D)); dO = rng.standard_normal((B, H, T, D))
    qt, kt, vt = (torch.tensor(a, requires_grad=True) for a in (q, k, v))
    ((qt @ kt.mT).tril(-1) @ vt).backward(torch.tensor(dO))
    for fn in (O.analytic_tril_attn_backward, O.analytic_tril_attn_backward_blocked):
        dq, dk, dv = fn(q, k, v, dO)
        np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-4, atol=1e-4)
    # self form: Q passed twice accumulates both score paths
    qs = torch.tensor(q, requires_grad=True); vs = torch.tensor(v, requires_grad=True)
    ((qs @ qs.mT).tril(-1) @ vs).backward(torch.tensor(dO))
    dqm, dv = O.self_attn_backward(q, v, dO)
    np.testing.assert_allclose(dqm, qs.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dv, vs.grad.numpy(), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("T,bs", [(64, 16), (130, 64), (300, 64)])
def test_blocked_backward_equals_dense(T, bs):
    rng = _rng(T + bs)
    q = rng.standard_normal((1, 2, T, 5)).astype(np.float32)
    v = rng.standard_normal((1, 1, T, 3)).astype(np.float32)
    dO = rng.standard_normal((1, 2, T, 3)).astype(np.float32)
    a = O.analytic_tril_attn_backward(q, q, v, dO, dtype=np.float64)
    b = O.analytic_tril_attn_backward_blocked(q, q, v, dO, block_size=bs)
    for x, y in zip(a, b):
        np.testing.assert_allclose(y, x, rtol=1e-4, atol=1e-3)


def test_backward_finite_difference():
    rng = _rng(9)
    q = rng.standard_normal((1, 1, 6, 3)); v = rng.standard_normal((1, 1, 6, 2))
    dO = rng.standard_normal((1, 1, 6, 2))
    loss = lambda qq, vv: float(np.sum(O.tril_score_v_eager(qq, qq, vv).astype(np.float64) * dO))  # noqa: E731
    dqm, dv = O.self_attn_backward(q, v, dO, blocked=False)
    eps = 1e-2
    for idx in [(0, 0, 3, 1), (0, 0, 0, 2), (0, 0, 5, 0)]:
        qp = q.copy(); qp[idx] += eps
        qm = q.copy(); qm[idx] -= eps
        assert abs((loss(qp, v) - loss(qm, v)) / (2 * eps) - dqm[idx]) < 2e-2
    for idx in [(0, 0, 1, 1), (0, 0, 4, 0)]:
        vp = v.copy(); vp[idx] += eps
        vm = v.copy(); vm[idx] -= eps
        assert abs((loss(q, vp) - loss(q, vm)) / (2 * eps) - dv[idx]) < 2e-2


# ------------------------------------------------------- fused RoPE + attn
def test_rope_attention_against_torch_autograd():
    rng = _rng(11)
    B, H, T, N, D, start = 1, 2, 10, 8, 3, 4
    x = rng.standard_normal((B, H, T, N)).astype(np.float32)
    v = rng.standard_normal((B, 1, T, D)).astype(np.float32)
    dO = rng.standard_normal((B, H, T, D)).astype(np.float32)
    f = O.get_freqs(N)
    out, qr = O.tril_rope_score_v(x, v, f, start)
    dx, dv = O.tril_rope_score_v_backward(x, v, dO, f, start)
    c, s = (torch.from_numpy(a).double() for a in O.rope_cos_sin(T, start, f))
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    vt = torch.tensor(v, dtype=torch.float64, requires_grad=True)
    x0, x1 = xt[..., 0::2], xt[..., 1::2]
    y = torch.stack((x0 * c[..., 0::2] - x1 * s[..., 0::2], x1 * c[..., 1::2] + x0 * s[..., 1::2]), -1).reshape(xt.shape)
    ot = (y @ y.mT).tril(-1) @ vt
    ot.backward(torch.from_numpy(dO).double())
    np.testing.assert_allclose(out, ot.detach().numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-4, atol=1e-4)
    assert not out[:, :, 0].any()


# ----------------------------------------------------------- queries at an offset
@pytest.mark.parametrize("past,T", [(0, 5), (3, 4), (7, 1), (130, 9)])
def test_past_equals_full_tril_last_rows(past, T):
    """bdh.py:446-461: the reference recomputes past||new and keeps rows past.."""
    rng = np.random.default_rng(past * 31 + T)
    k = rng.standard_normal((2, 2, past + T, 6)).astype(np.float32)
    v = rng.standard_normal((2, 1, past + T, 3)).astype(np.float32)
    got = O.tril_score_v_past(k[:, :, past:], k, v, past)
    want = O.tril_score_v_cpu(k, k, v)[:, :, past:]
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)


def test_past_bruteforce_and_special_cases():
    rng = np.random.default_rng(5)
    past, T = 4, 3
    q = rng.standard_normal((1, 2, T, 5)).astype(np.float32)
    k = rng.standard_normal((1, 2, past + T, 5)).astype(np.float32)
    v = rng.standard_normal((1, 2, past + T, 4)).astype(np.float32)
    # zero-padded query rows in front: row past + i of the full problem is query i
    qf = np.concatenate([np.zeros((1, 2, past, 5), np.float32), q], axis=2)
    want = O.tril_score_v_bruteforce(qf, k, v)[:, :, past:]
    np.testing.assert_allclose(O.tril_score_v_past(q, k, v, past), want, rtol=1e-5, atol=1e-5)
    # past = 0 is the cold op; T = 1 is decode over the past
    np.testing.assert_allclose(O.tril_score_v_past(k, k, v, 0), O.tril_score_v_cpu(k, k, v), rtol=1e-5, atol=1e-5)
    q1 = q[:, :, :1]
    k1 = k[:, :, : past + 1]
    v1 = v[:, :, : past + 1]
    np.testing.assert_allclose(O.tril_score_v_past(q1, k1, v1, past),
                               O.tril_decode_cpu(q1, k1[:, :, :past], v1[:, :, :past]), rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        O.tril_score_v_past(q, k[:, :, :-1], v, past)
