"""Autograd for strict-tril BDH attention: tril(Q @ K.T, -1) @ V.

Mirrors the reference surface kernels/attention_bwd.py:
``analytic_tril_attn_backward`` (dense, :45-83), ``StrictTrilAttnFn``
(:218-256), ``StrictTrilSelfAttnFn`` (:259-291; Q is K -> returns dQ + dK),
``strict_tril_attn`` (:294-320) and ``_env_autograd_enabled`` (:323-325).

For ``impl="hip"`` the forward is the HIP kernel and the backward is the HIP
analytic backward (one library call: the score tiles the forward kept, or
recomputed ones, G = dS + dS^T, merged dQ, head-summed dV).  ``eager`` keeps
the reference's dense PyTorch math.

:class:`TrilRopeSelfAttnFn` covers the fused RoPE entry (Q = K = RoPE(x)):
its backward returns dx directly (RoPE and its transpose fused in-kernel),
from the forward's kept score tiles when the shapes allow it.
"""

from __future__ import annotations

import os
from typing import Optional

import torch

from .attention import eager_tril_attn
from . import hip_attn

_VALID_IMPLS = ("eager", "hip")


def analytic_tril_attn_backward(Q, K, V, dO):
    """Dense analytic gradients of ``tril(Q K^T, -1) V`` (reference attention_bwd.py:45-83)."""
    B, H, T, _ = Q.shape
    D = V.shape[-1]
    bcast = V.size(1) == 1 and H != 1
    Vh = V.expand(B, H, T, D) if bcast else V
    # transposed operands are materialised (bf16 batched products on transposed
    # views have faulted ROCm GPUs); the values are the same
    def t(x):
        return x.transpose(-2, -1).contiguous()

    M = (Q @ t(K)).tril(diagonal=-1)
    dS = (dO @ t(Vh)).tril(diagonal=-1)
    dQ = dS @ K
    dK = t(dS) @ Q
    dVh = t(M) @ dO
    dV = dVh.sum(dim=1, keepdim=True) if bcast else dVh
    return dQ, dK, dV


# The reference's tiled variant (attention_bwd.py:86-181) exists to bound the
# score memory of its PyTorch backends; the same gradients come from the dense
# form here, and ``hip`` tiles inside the kernel.
analytic_tril_attn_backward_blocked = analytic_tril_attn_backward


def _normalize_impl(impl: Optional[str]) -> str:
    name = (impl or "eager").strip().lower()
    if name not in _VALID_IMPLS:
        raise ValueError(f"unknown attn impl={impl!r} (expected one of {_VALID_IMPLS})")
    return name


def _use_blocked_analytic_bwd(impl: str) -> bool:
    """True when the backward runs tiled (no T x T tensor): the HIP kernels."""
    return _normalize_impl(impl) == "hip"


def _forward_impl(Q, K, V, impl: str):
    name = _normalize_impl(impl)
    if name == "eager":
        return eager_tril_attn(Q, K, V)
    return hip_attn.tril_score_v(Q, K, V)


class StrictTrilAttnFn(torch.autograd.Function):
    """Forward via eager / hip; analytic backward for distinct Q, K, V."""

    @staticmethod
    def forward(ctx, Q, K, V, impl: str):  # type: ignore[override]
        ctx.impl = impl
        ctx.save_for_backward(Q, K, V)
        with torch.no_grad():
            return _forward_impl(Q, K, V, impl)

    @staticmethod
    def backward(ctx, dO):  # type: ignore[override]
        Q, K, V = ctx.saved_tensors
        if _use_blocked_analytic_bwd(ctx.impl):
            dQ, dK, dV = hip_attn.tril_score_v_bwd(Q, K, V, dO.to(Q.dtype))
            dV = dV.to(V.dtype)
        else:
            dQ, dK, dV = analytic_tril_attn_backward(Q, K, V, dO)
        return dQ, dK, dV, None


def _save_scores() -> bool:
    """``BDH_ATTN_SAVE_SCORES`` (default on): the hip forward keeps its score
    tiles for the backward instead of the backward recomputing them."""
    return os.environ.get("BDH_ATTN_SAVE_SCORES", "1").strip().lower() not in ("0", "false", "no", "off")


class StrictTrilSelfAttnFn(torch.autograd.Function):
    """Self-attention form (K is Q): returns dQ + dK for Q (reference :259-291).

    With ``impl="hip"`` the forward's bf16 score tiles are kept for the
    backward when the shapes allow it (the reference's default autograd path
    keeps S too); otherwise the backward recomputes them.
    """

    @staticmethod
    def forward(ctx, Q, V, impl: str):  # type: ignore[override]
        ctx.impl = impl
        scores = None
        with torch.no_grad():
            if _use_blocked_analytic_bwd(impl) and _save_scores():
                out, scores = hip_attn.tril_score_v_save(Q, V)
            else:
                out = _forward_impl(Q, Q, V, impl)
        ctx.has_scores = scores is not None
        if scores is not None:
            ctx.save_for_backward(Q, V, scores)
        else:
            ctx.save_for_backward(Q, V)
        return out

    @staticmethod
    def backward(ctx, dO):  # type: ignore[override]
        if ctx.has_scores:
            Q, V, scores = ctx.saved_tensors
            dQm, dV = hip_attn.tril_score_v_bwd_saved(Q, V, dO.to(Q.dtype), scores)
            return dQm, dV.to(V.dtype), None
        Q, V = ctx.saved_tensors
        if _use_blocked_analytic_bwd(ctx.impl):
            dQm, _, dV = hip_attn.tril_score_v_bwd(Q, None, V, dO.to(Q.dtype))
            return dQm, dV.to(V.dtype), None
        dQ, dK, dV = analytic_tril_attn_backward(Q, Q, V, dO)
        return dQ + dK, dV, None


class TrilRopeSelfAttnFn(torch.autograd.Function):
    """``tril(R(x) R(x)^T, -1) V`` with R = BDH RoPE fused into the HIP kernels.

    The backward returns dx (RoPE^T of the merged dQR) and dV; ``freqs`` is a
    constant buffer (no gradient), like the reference's detached cos/sin.
    Without ``qr_out`` the forward's bf16 score tiles are kept for the
    backward when the shapes allow it (``BDH_ATTN_SAVE_SCORES=0`` turns this
    off), so the backward recomputes none of them.
    """

    @staticmethod
    def forward(ctx, x, V, freqs, rope_start: int, qr_out=None):  # type: ignore[override]
        ctx.rope_start = int(rope_start)
        scores = None
        with torch.no_grad():
            if qr_out is None and x.dtype == torch.bfloat16 and _save_scores():
                out, scores = hip_attn.tril_rope_score_v_save(x, V, freqs, rope_start)
            else:
                out = hip_attn.tril_rope_score_v(x, V, freqs, rope_start, qr_out=qr_out)
        ctx.has_scores = scores is not None
        if scores is not None:
            ctx.save_for_backward(x, V, freqs, scores)
        else:
            ctx.save_for_backward(x, V, freqs)
        return out

    @staticmethod
    def backward(ctx, dO):  # type: ignore[override]
        if ctx.has_scores:
            x, V, freqs, scores = ctx.saved_tensors
        else:
            x, V, freqs = ctx.saved_tensors
        # bf16 x: V enters the products as bf16, as in the forward (and as the
        # reference's autocast matmul casts it), which lets the backward run on
        # the MFMA kernels; dV comes back in V's own dtype
        Vc = V.to(x.dtype) if x.dtype == torch.bfloat16 else V
        dV = torch.empty_like(V, memory_format=torch.contiguous_format)
        if ctx.has_scores:
            # contiguous dO rows keep its span inside the limits the forward
            # checked before keeping the tiles
            dx, dV = hip_attn.tril_rope_score_v_bwd_saved(x, Vc, dO.to(x.dtype).contiguous(), freqs,
                                                          ctx.rope_start, scores, dv=dV)
        else:
            dx, dV = hip_attn.tril_rope_score_v_bwd(x, Vc, dO.to(x.dtype), freqs, ctx.rope_start, dv=dV)
        return dx, dV, None, None, None


def strict_tril_attn(Q, K, V, *, impl: Optional[str] = None, use_fn: Optional[bool] = None):
    """Strict-tril score @ V with optional analytic autograd.Function (reference :294-320)."""
    if use_fn is None:
        use_fn = _env_autograd_enabled()
    name = _normalize_impl(impl if impl is not None else os.environ.get("BDH_ATTN_IMPL", "eager"))
    if use_fn:
        if Q is K:
            return StrictTrilSelfAttnFn.apply(Q, V, name)
        return StrictTrilAttnFn.apply(Q, K, V, name)
    return _forward_impl(Q, K, V, name)


def _env_autograd_enabled() -> bool:
    raw = os.environ.get("BDH_ATTN_AUTOGRAD", "").strip().lower()
    return raw in ("1", "true", "yes", "on")


__all__ = [
    "analytic_tril_attn_backward",
    "analytic_tril_attn_backward_blocked",
    "StrictTrilAttnFn",
    "StrictTrilSelfAttnFn",
    "TrilRopeSelfAttnFn",
    "strict_tril_attn",
    "_env_autograd_enabled",
]
