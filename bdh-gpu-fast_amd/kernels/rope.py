"""BDH RoPE apply: ``eager`` (PyTorch pair math) and ``hip`` (gfx950 kernel).

BDH RoPE is not the classic half-dim rotation: each adjacent pair (2m, 2m+1)
rotates by its own phase, ``frac(pos * freq[i])`` (pairs share a frequency)::

    y0 = x0 * c0 - x1 * s0
    y1 = x1 * c1 + x0 * s1

Validation helpers keep the reference's ``ValueError`` contract
(kernels/rope.py:30-100).  The ``eager`` functions restate the reference's
pair path (kernels/rope.py:108-240) with plain torch ops; the ``hip``
functions call the library kernel, which reproduces the same rounding (fp32
products then add; for bf16 inputs each product rounded to bf16 before the
bf16 add) and supports autograd through :class:`HipRopeFn`.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import hip_attn


# ----------------------------------------------------------------- validation
def _validate_rope_out(v: torch.Tensor, out: Optional[torch.Tensor], *cis: torch.Tensor) -> None:
    """``out=`` must match v's shape/device and must not alias v or cis (rope.py:30-50)."""
    if out is None:
        return
    if out.shape != v.shape or out.device != v.device:
        raise ValueError(
            f"rope out= must match v shape/device, got out={tuple(out.shape)}/"
            f"{out.device} vs v={tuple(v.shape)}/{v.device}"
        )
    for t in (v, *cis):
        if out is t or (out.device == t.device and torch._C._overlaps(out, t)):
            raise ValueError("rope out= must not alias v or cis")


def _validate_rope_inputs(v, cos, sin, out) -> None:
    """Flat cis checks (rope.py:53-74)."""
    if v.shape[-1] % 2 != 0:
        raise ValueError(f"RoPE last dim must be even, got {v.shape[-1]}")
    if cos.shape != sin.shape:
        raise ValueError(f"cos/sin shape mismatch: {cos.shape} vs {sin.shape}")
    if cos.shape[-1] != v.shape[-1]:
        raise ValueError(f"cos/sin last dim {cos.shape[-1]} != v last dim {v.shape[-1]}")
    try:
        torch.broadcast_shapes(v.shape[:-1], cos.shape[:-1])
    except RuntimeError as exc:
        raise ValueError(
            f"cos/sin leading dims {cos.shape[:-1]} are not broadcastable with v leading dims {v.shape[:-1]}"
        ) from exc
    _validate_rope_out(v, out, cos, sin)


def _validate_paired_cis(v, cos_p, sin_p, out) -> None:
    """Paired cis ``(..., N/2, 2)`` checks (rope.py:77-100)."""
    if v.shape[-1] % 2 != 0:
        raise ValueError(f"RoPE last dim must be even, got {v.shape[-1]}")
    n_pairs = v.shape[-1] // 2
    if cos_p.shape != sin_p.shape:
        raise ValueError(f"paired cos/sin shape mismatch: {cos_p.shape} vs {sin_p.shape}")
    if cos_p.shape[-2:] != (n_pairs, 2):
        raise ValueError(f"paired cis trailing dims must be ({n_pairs}, 2), got {cos_p.shape[-2:]}")
    try:
        torch.broadcast_shapes(v.shape[:-1], cos_p.shape[:-2])
    except RuntimeError as exc:
        raise ValueError(
            f"paired cis leading dims {cos_p.shape[:-2]} are not broadcastable with v leading dims {v.shape[:-1]}"
        ) from exc
    _validate_rope_out(v, out, cos_p, sin_p)


# ------------------------------------------------------------ cos/sin tables
def get_freqs(n: int, theta: float = 2 ** 16, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``1 / theta**(2*floor(i/2)/n) / (2*pi)`` (reference bdh.py:41-49)."""
    t = torch.arange(0, n, 1, dtype=dtype)
    q = (t / 2).floor() * 2
    return 1.0 / (theta ** (q / n)) / (2 * math.pi)


def rope_cos_sin(T: int, rope_start: int, freqs: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) of ``2*pi*frac((rope_start + t) * freq)`` (bdh.py:119-122, 142-150)."""
    f = freqs.reshape(1, 1, 1, -1)
    pos = torch.arange(rope_start, rope_start + T, device=f.device, dtype=f.dtype).view(1, 1, -1, 1)
    ph = (pos * f % 1) * (2 * math.pi)
    return torch.cos(ph), torch.sin(ph)


# ------------------------------------------------------------------- eager
def _rotate_pair_views(vp, cp, sp, *, v_dtype, cis_dtype):
    """(y0, y1) from pair views (rope.py:108-126)."""
    x0, x1 = vp[..., 0], vp[..., 1]
    c0, c1 = cp[..., 0], cp[..., 1]
    s0, s1 = sp[..., 0], sp[..., 1]
    if v_dtype != cis_dtype:
        y0 = (x0 * c0).to(v_dtype) + ((-x1) * s0).to(v_dtype)
        y1 = (x1 * c1).to(v_dtype) + (x0 * s1).to(v_dtype)
    else:
        y0 = x0 * c0 - x1 * s0
        y1 = x1 * c1 + x0 * s1
    return y0, y1


def _store_pairs(y0, y1, v, out):
    """Interleave pairs into ``out`` or a fresh contiguous buffer (rope.py:129-171)."""
    if out is None:
        out = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    op = out.reshape(*v.shape[:-1], -1, 2) if out.is_contiguous() else out.unflatten(-1, (-1, 2))
    op[..., 0] = y0
    op[..., 1] = y1
    return out


def eager_rope_rotate(v, cos, sin, out=None):
    """Reference-semantics rotation with torch ops (rope.py:220-240)."""
    _validate_rope_inputs(v, cos, sin, out)
    vp = v.reshape(*v.shape[:-1], -1, 2)
    cp = cos.reshape(*cos.shape[:-1], -1, 2)
    sp = sin.reshape(*sin.shape[:-1], -1, 2)
    y0, y1 = _rotate_pair_views(vp, cp, sp, v_dtype=v.dtype, cis_dtype=cos.dtype)
    return _store_pairs(y0, y1, v, out)


def rope_rotate_t1(v, cos, sin, out=None):
    """T=1 decode rotation (rope.py:193-217); same math as :func:`eager_rope_rotate`."""
    if not (v.dim() >= 2 and v.shape[-2] == 1):
        raise ValueError(f"rope_rotate_t1 expects sequence length 1, got shape {tuple(v.shape)}")
    return eager_rope_rotate(v, cos, sin, out=out)


def rope_rotate_paired(v, cos_p, sin_p, out=None):
    """Rotation from paired cis ``(..., N/2, 2)`` (rope.py:174-190)."""
    _validate_paired_cis(v, cos_p, sin_p, out)
    vp = v.reshape(*v.shape[:-1], -1, 2)
    y0, y1 = _rotate_pair_views(vp, cos_p, sin_p, v_dtype=v.dtype, cis_dtype=cos_p.dtype)
    return _store_pairs(y0, y1, v, out)


# --------------------------------------------------------------------- hip
class HipRopeFn(torch.autograd.Function):
    """HIP rotation forward; HIP transpose rotation backward (cis are constants)."""

    @staticmethod
    def forward(ctx, v, cos, sin):  # type: ignore[override]
        ctx.save_for_backward(cos.detach(), sin.detach())
        ext = hip_attn._require(v, cos, sin)
        return ext.rope_rotate(v, cos.detach(), sin.detach())

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        cos, sin = ctx.saved_tensors
        ext = hip_attn._require(g)
        gg = g if g.stride(-1) == 1 else g.contiguous()
        return ext.rope_rotate(gg, cos, sin, backward=True), None, None


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    return t if (t.size(-1) <= 1 or t.stride(-1) == 1) else t.contiguous()


def hip_rope_rotate(v, cos, sin, out=None):
    """gfx950 rotation; ``out=`` (e.g. a KR cache slot) is written in place, cast to its dtype."""
    _validate_rope_inputs(v, cos, sin, out)
    ext = hip_attn._require(v, cos, sin, out)
    v = _unit_last(v)
    cos, sin = _unit_last(cos), _unit_last(sin)
    if torch.is_grad_enabled() and v.requires_grad:
        y = HipRopeFn.apply(v, cos, sin)
        if out is not None:
            out.copy_(y)
            return out
        return y
    return ext.rope_rotate(v, cos, sin, out)


def hip_rope_rotate_paired(v, cos_p, sin_p, out=None):
    """gfx950 rotation from paired cis (flattened to ``(..., N)`` views)."""
    _validate_paired_cis(v, cos_p, sin_p, out)
    return hip_rope_rotate(v, cos_p.flatten(-2), sin_p.flatten(-2), out=out)


__all__ = [
    "get_freqs",
    "rope_cos_sin",
    "eager_rope_rotate",
    "rope_rotate_t1",
    "rope_rotate_paired",
    "hip_rope_rotate",
    "hip_rope_rotate_paired",
    "HipRopeFn",
    "_validate_rope_out",
    "_validate_rope_inputs",
    "_validate_paired_cis",
    "_store_pairs",
]
