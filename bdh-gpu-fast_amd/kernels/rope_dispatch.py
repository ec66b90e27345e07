"""Env-gated dispatch for BDH RoPE apply (reference kernels/rope_dispatch.py).

Backends (``BDH_ROPE_IMPL``)::

    export BDH_ROPE_IMPL=eager   # default: PyTorch pair math (reference semantics)
    export BDH_ROPE_IMPL=hip     # gfx950 kernel (same rounding order, out= in place)

``rope_cos_sin`` caching stays in the caller (bdh.Attention); this module
only picks how (cos, sin) are applied to ``v``.  Unknown names raise
``ValueError`` like the reference (rope_dispatch.py:41-61).
"""

from __future__ import annotations

import os
from typing import Literal, Optional

import torch

from . import hip_attn
from .rope import (
    eager_rope_rotate,
    hip_rope_rotate,
    hip_rope_rotate_paired,
    rope_rotate_paired,
    rope_rotate_t1,
)

ImplName = Literal["eager", "hip"]
_VALID = ("eager", "hip")


def _parse_rope_impl(raw: str | None) -> ImplName:
    name = (raw or "eager").strip().lower()
    if name not in _VALID:
        raise ValueError(f"BDH_ROPE_IMPL must be {'|'.join(_VALID)}, got {name!r}")
    return name  # type: ignore[return-value]


class _EnvChoice:
    """``BDH_ROPE_IMPL`` parsed once per distinct raw value of the variable."""

    def __init__(self) -> None:
        self.raw: str | None = None
        self.value: ImplName | None = None

    def get(self) -> ImplName:
        raw = os.environ.get("BDH_ROPE_IMPL", "eager")
        if self.value is None or raw != self.raw:
            self.value = _parse_rope_impl(raw)  # raises before the cache is touched
            self.raw = raw
        return self.value


_rope_env = _EnvChoice()


def resolve_rope_impl(requested: str | None = None) -> ImplName:
    """Backend for RoPE apply: ``requested`` if given, else ``BDH_ROPE_IMPL``
    (default ``eager``).  Unknown names raise ``ValueError``."""
    if requested is not None:
        return _parse_rope_impl(requested)
    return _rope_env.get()


def bdh_rope_rotate(
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    *,
    impl: str | None = None,
) -> torch.Tensor:
    """Apply RoPE (cos, sin) to ``v``; returns ``out`` itself when given."""
    name = resolve_rope_impl(impl)
    if name == "eager":
        if v.dim() >= 2 and v.shape[-2] == 1:
            return rope_rotate_t1(v, cos, sin, out=out)
        return eager_rope_rotate(v, cos, sin, out=out)
    return hip_rope_rotate(v, cos, sin, out=out)


def bdh_rope_rotate_paired(
    v: torch.Tensor,
    cos_p: torch.Tensor,
    sin_p: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    *,
    impl: str | None = None,
) -> torch.Tensor:
    """Apply already-paired cis ``(..., N/2, 2)`` with the selected backend."""
    name = resolve_rope_impl(impl)
    if name == "eager":
        return rope_rotate_paired(v, cos_p, sin_p, out=out)
    return hip_rope_rotate_paired(v, cos_p, sin_p, out=out)


def backend_info(device: torch.device | None = None) -> dict:
    """Small diagnostic (reference rope_dispatch.py:102-124)."""
    return {
        "BDH_ROPE_IMPL": resolve_rope_impl(),
        "has_hip_ext": hip_attn.has_hip_ext(),
        "hip_usable": hip_attn.has_hip_kernel(),
        "device": str(device) if device is not None else ("cuda" if torch.cuda.is_available() else "cpu"),
    }


__all__ = [
    "resolve_rope_impl",
    "bdh_rope_rotate",
    "bdh_rope_rotate_paired",
    "backend_info",
    "eager_rope_rotate",
    "hip_rope_rotate",
    "hip_rope_rotate_paired",
    "rope_rotate_paired",
    "rope_rotate_t1",
]
