"""numpy restatement of the reference CPU path for BDH strict-tril attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): tests, ``smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` are the only callers.

Conventions
-----------
* Arrays are numpy ``float32`` (the reference's fp32 CPU math) unless a
  function says otherwise.  bf16 tensors are represented by ``float32`` arrays
  whose values are exactly representable in bf16 (see :func:`bf16_round`);
  the reference's ``maybe_acc`` (csrc/tril_attn_cpu.cpp:77-82) widens bf16 to
  fp32 exactly, so fp32 math on those values *is* the reference's math.
* Shapes follow the reference: q, k ``(B, H, T, Dk)``; v ``(B, 1|H, T, Dv)``;
  out ``(B, H, T, Dv)``.
* Matrix products use ``numpy.matmul`` (BLAS sgemm), the counterpart of the
  reference's ``at::matmul`` on CPU.
"""

from __future__ import annotations

import math
from typing import Tuple

import numpy as np

__all__ = [
    "bf16_round",
    "get_freqs",
    "rope_phases",
    "phases_cos_sin",
    "rope_cos_sin",
    "rope_rotate",
    "rope_rotate_backward",
    "pick_cold_tiles_cpu",
    "cold_score_budget",
    "pick_decode_tile_n_cpu",
    "tril_score_v_cpu",
    "tril_score_v_eager",
    "tril_score_v_tiled",
    "tril_decode_cpu",
    "tril_decode_eager",
    "tril_decode_tiled",
    "analytic_tril_attn_backward",
    "analytic_tril_attn_backward_blocked",
    "self_attn_backward",
    "tril_rope_score_v",
    "tril_rope_score_v_backward",
    "tril_score_v_past",
    "tril_score_v_bruteforce",
    "tril_decode_bruteforce",
    "PINNING",
]

# Score-element thresholds of csrc/tril_attn_cpu.cpp:9-17.
TILE_M = 16
TILE_N = 16
TILE_M_CPU_MAX = 128
TILE_N_CPU_MAX = 128
DECODE_TILE_N_CPU_MAX = 512
SCORE_ELEMS_EAGER_OK = 256 * 256
COLD_SCORE_ELEMS_BUDGET = 256 * 256

# Default block of the blocked analytic backward (kernels/attention.py:43-46,
# DEFAULT_BLOCK_COLD) and its score budget (_SCORE_ELEMS_BUDGET).
DEFAULT_BLOCK_COLD = 64
SCORE_ELEMS_BUDGET = 256 * 256


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), as float32.

    Same rounding as ``tensor.to(torch.bfloat16)`` (round-to-nearest-even on
    the upper 16 bits, NaN kept quiet).  Used wherever the reference casts to
    bf16 (rope.py:120-122 products, ``.to(q.scalar_type())`` outputs).
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    rounding = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    r = ((u + rounding) >> np.uint64(16)) << np.uint64(16)
    nan = np.isnan(a)
    r = r.astype(np.uint32)
    if nan.any():
        r[nan] = (a.view(np.uint32)[nan] | np.uint32(0x00400000)) & np.uint32(0xFFFF0000)
    return r.view(np.float32).reshape(a.shape)


# ---------------------------------------------------------------------------
# RoPE (bdh.py / kernels/rope.py)
# ---------------------------------------------------------------------------
def get_freqs(n: int, theta: float = 2.0 ** 16) -> np.ndarray:
    """``freq[i] = 1 / theta**(2*floor(i/2)/n) / (2*pi)`` in fp32 (bdh.py:41-49).

    Adjacent pairs share one frequency because ``quantize`` floors ``i/2``.
    Each step is a separate fp32 operation, as in the torch expression.
    """
    t = np.arange(0, n, 1, dtype=np.float32)
    q = np.floor(t / np.float32(2.0)) * np.float32(2.0)
    expo = q / np.float32(n)
    denom = np.power(np.float32(theta), expo, dtype=np.float32)
    return ((np.float32(1.0) / denom) / np.float32(2 * math.pi)).astype(np.float32)


def rope_phases(T: int, rope_start: int, freqs: np.ndarray) -> np.ndarray:
    """``phase[t, i] = fp32(rope_start + t) * freq[i]`` (bdh.py:142-150).

    Positions are integers made fp32 by ``torch.arange(..., dtype=float32)``
    (exact below 2**24); the product is one fp32 multiply.  Shape ``(T, N)``.
    """
    pos = np.arange(rope_start, rope_start + T, dtype=np.float32).reshape(-1, 1)
    return (pos * np.asarray(freqs, dtype=np.float32).reshape(1, -1)).astype(np.float32)


def phases_cos_sin(phases: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """``theta = (phase mod 1) * 2*pi``; return ``cos(theta), sin(theta)`` (bdh.py:119-122).

    ``phase % 1`` is torch.remainder, ``a - floor(a)`` for the non-negative
    phases of RoPE; the scale by ``2*pi`` is an fp32 multiply by fp32(2*pi).
    """
    ph = np.asarray(phases, dtype=np.float32)
    frac = (ph - np.floor(ph)).astype(np.float32)
    theta = (frac * np.float32(2 * math.pi)).astype(np.float32)
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def rope_cos_sin(T: int, rope_start: int, freqs: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """(cos, sin) tables for positions ``[rope_start, rope_start+T)`` (bdh.py:193-299)."""
    return phases_cos_sin(rope_phases(T, rope_start, freqs))


def rope_rotate(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, *, bf16: bool = False) -> np.ndarray:
    """Adjacent-pair RoPE rotation (kernels/rope.py:108-126, 220-240).

    ``y[2k] = x[2k]*c[2k] - x[2k+1]*s[2k]``;
    ``y[2k+1] = x[2k+1]*c[2k+1] + x[2k]*s[2k+1]``.

    fp32 ``x`` (``bf16=False``): two fp32 products then one fp32 add/sub.
    bf16 ``x`` with fp32 cos/sin (``bf16=True``): each product is computed in
    fp32 and rounded to bf16, and the two bf16 terms are added with one more
    bf16 rounding (rope.py:120-122).  ``cos``/``sin`` broadcast against ``x``.
    """
    x = np.asarray(x, dtype=np.float32)
    c = np.broadcast_to(np.asarray(cos, dtype=np.float32), x.shape)
    s = np.broadcast_to(np.asarray(sin, dtype=np.float32), x.shape)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c0, c1 = c[..., 0::2], c[..., 1::2]
    s0, s1 = s[..., 0::2], s[..., 1::2]
    y = np.empty_like(x)
    if bf16:
        y[..., 0::2] = bf16_round(bf16_round(x0 * c0) + bf16_round((-x1) * s0))
        y[..., 1::2] = bf16_round(bf16_round(x1 * c1) + bf16_round(x0 * s1))
    else:
        y[..., 0::2] = x0 * c0 - x1 * s0
        y[..., 1::2] = x1 * c1 + x0 * s1
    return y


def rope_rotate_backward(g: np.ndarray, cos: np.ndarray, sin: np.ndarray, *, bf16: bool = False) -> np.ndarray:
    """Gradient of :func:`rope_rotate` w.r.t. ``x`` (kernels/rope.py:543-556).

    ``dx[2k] = g[2k]*c[2k] + g[2k+1]*s[2k+1]``;
    ``dx[2k+1] = -g[2k]*s[2k] + g[2k+1]*c[2k+1]``.
    """
    g = np.asarray(g, dtype=np.float32)
    c = np.broadcast_to(np.asarray(cos, dtype=np.float32), g.shape)
    s = np.broadcast_to(np.asarray(sin, dtype=np.float32), g.shape)
    g0, g1 = g[..., 0::2], g[..., 1::2]
    c0, c1 = c[..., 0::2], c[..., 1::2]
    s0, s1 = s[..., 0::2], s[..., 1::2]
    dx = np.empty_like(g)
    if bf16:
        dx[..., 0::2] = bf16_round(bf16_round(g0 * c0) + bf16_round(g1 * s1))
        dx[..., 1::2] = bf16_round(bf16_round((-g0) * s0) + bf16_round(g1 * c1))
    else:
        dx[..., 0::2] = g0 * c0 + g1 * s1
        dx[..., 1::2] = -g0 * s0 + g1 * c1
    return dx


# ---------------------------------------------------------------------------
# Tile pickers / budgets (csrc/tril_attn_cpu.cpp:20-74)
# ---------------------------------------------------------------------------
def pick_cold_tiles_cpu(T: int) -> Tuple[int, int]:
    """Power-of-two query/key tiles (csrc/tril_attn_cpu.cpp:20-44)."""
    if T <= 64:
        want_m, want_n = 16, 16
    elif T <= 256:
        want_m, want_n = 32, 32
    else:
        want_m, want_n = 128, 128
    tm, tn = 16, 16
    tcap = max(T, 1)
    while tm < min(tcap, want_m) and tm < TILE_M_CPU_MAX:
        tm <<= 1
    while tn < min(tcap, want_n) and tn < TILE_N_CPU_MAX:
        tn <<= 1
    return min(tm, TILE_M_CPU_MAX), min(tn, TILE_N_CPU_MAX)


def cold_score_budget(T: int, BS: int) -> int:
    """Past-tile score budget (csrc/tril_attn_cpu.cpp:46-52)."""
    budget = max(BS * BS, COLD_SCORE_ELEMS_BUDGET)
    if T >= 256:
        budget = max(budget, BS * min(T, 1024))
    return budget


def pick_decode_tile_n_cpu(S: int) -> int:
    """Past tile for tiled decode (csrc/tril_attn_cpu.cpp:55-74)."""
    if S <= 64:
        want = 32
    elif S <= 256:
        want = 64
    elif S <= 1024:
        want = 128
    elif S <= 2048:
        want = 256
    else:
        want = 512
    tn = 16
    target = min(max(S, 1), want)
    while tn < target and tn < DECODE_TILE_N_CPU_MAX:
        tn <<= 1
    return min(tn, DECODE_TILE_N_CPU_MAX)


def _check_cold(q, k, v):
    """Input contract of tril_score_v_cpu (csrc/tril_attn_cpu.cpp:161-167)."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q,k,v must be 4D (B,H,T,D)")
    if q.shape != k.shape:
        raise ValueError("q and k must have the same shape")
    if q.shape[0] != v.shape[0] or q.shape[2] != v.shape[2]:
        raise ValueError("batch and seq dims of v must match q")
    if v.shape[1] not in (q.shape[1], 1):
        raise ValueError("v heads must equal q heads or 1 (broadcast)")


# ---------------------------------------------------------------------------
# Cold forward (csrc/tril_attn_cpu.cpp:89-174)
# ---------------------------------------------------------------------------
def tril_score_v_eager(q, k, v) -> np.ndarray:
    """``(q @ k^T).tril(-1) @ v`` with materialised scores (csrc/tril_attn_cpu.cpp:89-99)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    scores = np.matmul(q, np.swapaxes(k, -1, -2))
    scores = np.tril(scores, -1)
    return np.matmul(scores, v).astype(np.float32)


def tril_score_v_tiled(q, k, v) -> np.ndarray:
    """Tiled strict-tril score x V (csrc/tril_attn_cpu.cpp:103-158).

    Query tiles of ``TM`` rows; the whole past ``j < i0`` in one product when
    ``Bi*i0`` fits the budget, else in key chunks; the diagonal ``Bi x Bi``
    tile with ``tril(-1)``.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    B, H, T, _ = q.shape
    Dv = v.shape[3]
    out = np.zeros((B, H, T, Dv), np.float32)
    if T == 0:
        return out
    TM, TN = pick_cold_tiles_cpu(T)
    budget = cold_score_budget(T, TM)
    for i0 in range(0, T, TM):
        i1 = min(i0 + TM, T)
        Bi = i1 - i0
        Qi = q[:, :, i0:i1, :]
        if i0 > 0:
            if Bi * i0 <= budget:
                Kj = k[:, :, :i0, :]
                Vj = v[:, :, :i0, :]
                out[:, :, i0:i1, :] += np.matmul(np.matmul(Qi, np.swapaxes(Kj, -1, -2)), Vj)
            else:
                tile = max(TN, budget // max(Bi, 1))
                for j0 in range(0, i0, tile):
                    j1 = min(j0 + tile, i0)
                    Kj = k[:, :, j0:j1, :]
                    Vj = v[:, :, j0:j1, :]
                    out[:, :, i0:i1, :] += np.matmul(np.matmul(Qi, np.swapaxes(Kj, -1, -2)), Vj)
        if Bi > 1:
            sc = np.matmul(Qi, np.swapaxes(k[:, :, i0:i1, :], -1, -2))
            sc = np.tril(sc, -1)
            out[:, :, i0:i1, :] += np.matmul(sc, v[:, :, i0:i1, :])
    return out


def tril_score_v_cpu(q, k, v) -> np.ndarray:
    """Dispatch eager/tiled on the score footprint (csrc/tril_attn_cpu.cpp:160-174)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    _check_cold(q, k, v)
    T = q.shape[2]
    if T * T > SCORE_ELEMS_EAGER_OK:
        return tril_score_v_tiled(q, k, v)
    return tril_score_v_eager(q, k, v)


# ---------------------------------------------------------------------------
# Decode (csrc/tril_attn_cpu.cpp:178-238)
# ---------------------------------------------------------------------------
def _check_decode(q, k_past, v_past):
    """Input contract of tril_decode_cpu (csrc/tril_attn_cpu.cpp:214-223)."""
    if q.ndim != 4 or k_past.ndim != 4 or v_past.ndim != 4:
        raise ValueError("q,k_past,v_past must be 4D")
    if q.shape[0] != k_past.shape[0] or q.shape[1] != k_past.shape[1]:
        raise ValueError("q and k_past batch/heads must match")
    if q.shape[3] != k_past.shape[3]:
        raise ValueError("q and k_past Dk must match")
    if v_past.shape[0] != q.shape[0] or v_past.shape[2] != k_past.shape[2]:
        raise ValueError("v_past batch/seq must match k_past")
    if v_past.shape[1] not in (q.shape[1], 1):
        raise ValueError("v_past heads must equal q heads or 1 (broadcast)")


def tril_decode_eager(q, k_past, v_past) -> np.ndarray:
    """``(q @ k_past^T) @ v_past`` (csrc/tril_attn_cpu.cpp:178-187)."""
    q = np.asarray(q, np.float32)
    k_past = np.asarray(k_past, np.float32)
    v_past = np.asarray(v_past, np.float32)
    return np.matmul(np.matmul(q, np.swapaxes(k_past, -1, -2)), v_past).astype(np.float32)


def tril_decode_tiled(q, k_past, v_past) -> np.ndarray:
    """Past-chunked decode (csrc/tril_attn_cpu.cpp:189-210)."""
    q = np.asarray(q, np.float32)
    k_past = np.asarray(k_past, np.float32)
    v_past = np.asarray(v_past, np.float32)
    B, H, Tq, _ = q.shape
    S = k_past.shape[2]
    Dv = v_past.shape[3]
    TN = pick_decode_tile_n_cpu(S)
    out = np.zeros((B, H, Tq, Dv), np.float32)
    for j0 in range(0, S, TN):
        j1 = min(j0 + TN, S)
        Kj = k_past[:, :, j0:j1, :]
        Vj = v_past[:, :, j0:j1, :]
        out += np.matmul(np.matmul(q, np.swapaxes(Kj, -1, -2)), Vj)
    return out


def tril_decode_cpu(q, k_past, v_past) -> np.ndarray:
    """Decode against the packed past (csrc/tril_attn_cpu.cpp:212-238).

    Every past key is strictly earlier than the query, so no mask applies;
    ``S == 0`` gives zeros.
    """
    q = np.asarray(q, np.float32)
    k_past = np.asarray(k_past, np.float32)
    v_past = np.asarray(v_past, np.float32)
    _check_decode(q, k_past, v_past)
    B, H, Tq, _ = q.shape
    S = k_past.shape[2]
    Dv = v_past.shape[3]
    if S == 0:
        return np.zeros((B, H, Tq, Dv), np.float32)
    if Tq * S > SCORE_ELEMS_EAGER_OK:
        return tril_decode_tiled(q, k_past, v_past)
    return tril_decode_eager(q, k_past, v_past)


# ---------------------------------------------------------------------------
# Backward (kernels/attention_bwd.py)
# ---------------------------------------------------------------------------
def analytic_tril_attn_backward(q, k, v, dO, dtype=np.float32):
    """Dense analytic gradients of ``tril(q k^T, -1) v`` (kernels/attention_bwd.py:45-83).

    ``M = tril(q k^T, -1)``, ``dS = tril(dO v^T, -1)``, ``dq = dS k``,
    ``dk = dS^T q``, ``dv = M^T dO`` summed over heads when v broadcasts.
    """
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    dO = np.asarray(dO, dtype)
    B, H, T, _ = q.shape
    D = v.shape[3]
    bcast = v.shape[1] == 1 and H != 1
    vh = np.broadcast_to(v, (B, H, T, D)) if bcast else v
    M = np.tril(np.matmul(q, np.swapaxes(k, -1, -2)), -1)
    dS = np.tril(np.matmul(dO, np.swapaxes(vh, -1, -2)), -1)
    dq = np.matmul(dS, k)
    dk = np.matmul(np.swapaxes(dS, -1, -2), q)
    dvh = np.matmul(np.swapaxes(M, -1, -2), dO)
    dv = dvh.sum(axis=1, keepdims=True) if bcast else dvh
    return dq.astype(dtype), dk.astype(dtype), dv.astype(dtype)


def analytic_tril_attn_backward_blocked(q, k, v, dO, block_size: int = DEFAULT_BLOCK_COLD):
    """Tiled analytic backward without a T x T buffer (kernels/attention_bwd.py:86-181).

    Past tiles use the whole past when ``Bi*i0`` fits the budget, else key
    chunks; diagonal tiles mask with ``tril(-1)``.  fp32 accumulation.
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    dO = np.asarray(dO, np.float32)
    B, H, T, _ = q.shape
    D = v.shape[3]
    bcast = v.shape[1] == 1 and H != 1
    vh = np.broadcast_to(v, (B, H, T, D)) if bcast else v
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dvh = np.zeros((B, H, T, D), np.float32)
    BS = max(1, int(block_size))
    budget = max(BS * BS, SCORE_ELEMS_BUDGET)
    mT = lambda a: np.swapaxes(a, -1, -2)  # noqa: E731
    for i0 in range(0, T, BS):
        i1 = min(i0 + BS, T)
        Qi = q[:, :, i0:i1]
        dOi = dO[:, :, i0:i1]
        Bi = i1 - i0
        if i0 > 0:
            tile = i0 if Bi * i0 <= budget else max(BS, budget // max(Bi, 1))
            for j0 in range(0, i0, tile):
                j1 = min(j0 + tile, i0)
                Kj = k[:, :, j0:j1]
                Vj = vh[:, :, j0:j1]
                dS = np.matmul(dOi, mT(Vj))
                dq[:, :, i0:i1] += np.matmul(dS, Kj)
                dk[:, :, j0:j1] += np.matmul(mT(dS), Qi)
                M = np.matmul(Qi, mT(Kj))
                dvh[:, :, j0:j1] += np.matmul(mT(M), dOi)
        if Bi > 1:
            Ki = k[:, :, i0:i1]
            Vi = vh[:, :, i0:i1]
            dS = np.tril(np.matmul(dOi, mT(Vi)), -1)
            dq[:, :, i0:i1] += np.matmul(dS, Ki)
            dk[:, :, i0:i1] += np.matmul(mT(dS), Qi)
            M = np.tril(np.matmul(Qi, mT(Ki)), -1)
            dvh[:, :, i0:i1] += np.matmul(mT(M), dOi)
    dv = dvh.sum(axis=1, keepdims=True) if bcast else dvh
    return dq, dk, dv


def self_attn_backward(q, v, dO, *, blocked: bool = True):
    """Self-attention form (K is Q): returns ``(dQ + dK, dV)`` (kernels/attention_bwd.py:259-291)."""
    if blocked:
        dq, dk, dv = analytic_tril_attn_backward_blocked(q, q, v, dO)
    else:
        dq, dk, dv = analytic_tril_attn_backward(q, q, v, dO)
    return (dq + dk).astype(np.float32), dv


# ---------------------------------------------------------------------------
# Fused RoPE + attention (bdh.py:348-413 cold path)
# ---------------------------------------------------------------------------
def tril_rope_score_v(x, v, freqs, rope_start: int = 0, *, bf16: bool = False):
    """Cold BDH attention: ``QR = RoPE(x)`` then ``tril(QR QR^T, -1) V``.

    Follows ``Attention.forward`` (bdh.py:396-413): cos/sin from
    ``rope_cos_sin(T, rope_start)`` (bdh.py:193-299), rotation by
    ``bdh_rope_rotate`` (rope.py:220-240), then ``bdh_attn(QR, QR, V)``
    evaluated by the CPU path (csrc/tril_attn_cpu.cpp:160-174).  With
    ``bf16=True`` the rotation follows the bf16 rounding order and QR is bf16.
    Returns ``(out_fp32, QR)``.
    """
    x = np.asarray(x, np.float32)
    T = x.shape[2]
    cos, sin = rope_cos_sin(T, rope_start, freqs)
    qr = rope_rotate(x, cos, sin, bf16=bf16)
    return tril_score_v_cpu(qr, qr, v), qr


def tril_rope_score_v_backward(x, v, dO, freqs, rope_start: int = 0):
    """Gradients of :func:`tril_rope_score_v` in fp32: ``(dx, dV)``.

    ``dQR = dQ + dK`` of the self-attention backward (attention_bwd.py:259-291)
    pulled back through the rotation (rope.py:543-556).
    """
    x = np.asarray(x, np.float32)
    T = x.shape[2]
    cos, sin = rope_cos_sin(T, rope_start, freqs)
    qr = rope_rotate(x, cos, sin)
    dqr, dv = self_attn_backward(qr, v, dO)
    return rope_rotate_backward(dqr, cos, sin), dv


# ---------------------------------------------------------------------------
# Queries at an offset (chunked prefill)
# ---------------------------------------------------------------------------
def tril_score_v_past(q, k, v, past: int) -> np.ndarray:
    """``out[b,h,i] = sum_{j < past + i} <q_i, k_j> v_j`` for q ``(B,H,T,Dk)``
    over k ``(B,H,past+T,Dk)``, v ``(B,1|H,past+T,Dv)``.

    The op the reference computes for a multi-token step with a cache by
    running the full strict-tril attention over past||new and keeping the
    last T rows (bdh.py:446-461: ``bdh_attn(QR_all, QR_all, V_all)``, then
    ``[..., S:, :]``).
    """
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    B, H, T, Dk = q.shape
    Tk = k.shape[2]
    if k.shape != (B, H, past + T, Dk) or v.shape[2] != Tk or v.shape[1] not in (1, H):
        raise ValueError("tril_score_v_past: q (B,H,T,Dk), k (B,H,past+T,Dk), v (B,1|H,past+T,Dv)")
    s = np.matmul(q, np.swapaxes(k, -1, -2))  # (B,H,T,Tk)
    keep = np.arange(Tk)[None, :] < (past + np.arange(T))[:, None]
    s = np.where(keep, s, np.float32(0))
    return np.matmul(s, v).astype(np.float32)


# ---------------------------------------------------------------------------
# Brute force (tiny shapes only; pins the BLAS-based paths)
# ---------------------------------------------------------------------------
def tril_score_v_bruteforce(q, k, v):
    """Triple loop in Python floats: ``out[b,h,i] = sum_{j<i} <q_i,k_j> v_j``."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, T, Dk = q.shape
    Dv = v.shape[3]
    out = np.zeros((B, H, T, Dv), np.float64)
    for b in range(B):
        for h in range(H):
            hv = h if v.shape[1] == H else 0
            for i in range(T):
                for j in range(i):
                    s = 0.0
                    for e in range(Dk):
                        s += float(q[b, h, i, e]) * float(k[b, h, j, e])
                    for d in range(Dv):
                        out[b, h, i, d] += s * float(v[b, hv, j, d])
    return out


def tril_decode_bruteforce(q, k_past, v_past):
    """Triple loop in Python floats: ``out[b,h,t] = sum_{s<S} <q_t,k_s> v_s``."""
    q = np.asarray(q, np.float64)
    k_past = np.asarray(k_past, np.float64)
    v_past = np.asarray(v_past, np.float64)
    B, H, Tq, Dk = q.shape
    S = k_past.shape[2]
    Dv = v_past.shape[3]
    out = np.zeros((B, H, Tq, Dv), np.float64)
    for b in range(B):
        for h in range(H):
            hv = h if v_past.shape[1] == H else 0
            for t in range(Tq):
                for j in range(S):
                    s = 0.0
                    for e in range(Dk):
                        s += float(q[b, h, t, e]) * float(k_past[b, h, j, e])
                    for d in range(Dv):
                        out[b, h, t, d] += s * float(v_past[b, hv, j, d])
    return out


# How each oracle function is pinned (checked in tests/test_oracle.py).
PINNING = {
    "bf16_round": "torch .to(torch.bfloat16) (library rounding) on random, tie and special values",
    "get_freqs": "float64 closed form 1/theta^(2*floor(i/2)/n)/(2*pi) within fp32 rounding; pair equality exact",
    "rope_phases": "exact integer positions; phase continuity _rope_phases(T,S) == _rope_phases(S+T,0)[S:] (test_attention_mask.py:119-124)",
    "phases_cos_sin": "math.cos/math.sin in float64 of the same reduced angle; pair 0 angle == position mod 2*pi",
    "rope_rotate": "dense 2x2 rotation-matrix product in float64; pair-norm preservation; position 0 is identity; bf16 order vs torch ops",
    "rope_rotate_backward": "adjoint identity <R x, g> == <x, R^T g> in float64; central finite differences",
    "tril_score_v_cpu": "known answers out [0,14,124] (test_attn_bwd_v4_contract.py:15-27), [0,22,151] (:241-246); brute-force triple loop; torch matmul+tril; row 0 == 0; linearity in v",
    "tril_decode_cpu": "known answer 31 (test_decode_contract_v12.py:21-28); decode == last row of full tril over past||new (test_cuda_decode.py:119-141); S=0 -> zeros; brute force",
    "analytic_tril_attn_backward": "known answers dQ/dK/dV (test_attn_bwd_v4_contract.py:29-36); zero upstream -> zero grads (:39-59); torch autograd of the eager formula in float64; finite differences",
    "analytic_tril_attn_backward_blocked": "equal to the dense form (test_attn_bwd.py:314-323) at several T and block sizes",
    "self_attn_backward": "known answers merged dQ/dV (test_attn_bwd_v4_contract.py:247-253); torch autograd with Q passed twice",
    "tril_rope_score_v": "composition of pinned parts; T=1 -> zeros; rope_start continuity",
    "tril_rope_score_v_backward": "torch autograd (float64) through RoPE + eager tril attention; finite differences",
    "tril_score_v_past": "the reference's own path: tril_score_v_cpu over past||new, last T rows (bdh.py:446-461); brute force on a zero-padded query; past = 0 is the cold op; T = 1 is decode over the past",
}
