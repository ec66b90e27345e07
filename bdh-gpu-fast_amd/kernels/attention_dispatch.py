"""Env-gated dispatch for BDH strict-tril attention (reference kernels/attention_dispatch.py).

Backends (``BDH_ATTN_IMPL``)::

    export BDH_ATTN_IMPL=eager   # default: full T x T scores then tril_(-1) (reference eager)
    export BDH_ATTN_IMPL=hip     # gfx950 kernels (no T x T tensor; RoPE fusion available)
    export BDH_ATTN_AUTOGRAD=1   # analytic autograd.Function (hip: HIP backward kernels)

Opt-in long-sequence switch, same knobs as the reference::

    export BDH_ATTN_AUTO=1                    # off unless set
    export BDH_ATTN_AUTO_THRESHOLD=512        # decode past_len > thr -> hip
    export BDH_ATTN_AUTO_COLD_THRESHOLD=...   # cold T > thr -> hip (mirrors AUTO_THRESHOLD)

With AUTO on and base ``eager``, lengths above the threshold switch to
``hip`` when the library is loaded, a ROCm device is visible and the operands
are ROCm tensors in fp32/bf16; otherwise they stay ``eager`` (the reference
switched to triton|blocked, attention_dispatch.py:203-260, and never to a
backend that raises).  An explicit ``hip`` is never silently
replaced: a missing library or CPU tensors raise ``RuntimeError``.

``hip`` with gradients: when autograd needs gradients of Q or V, ``bdh_attn``
routes through the analytic Function (:mod:`kernels.attention_bwd`) so the
default (``BDH_ATTN_AUTOGRAD`` unset) training path still trains.
"""

from __future__ import annotations

import os
from typing import Literal, Optional

import torch

from . import hip_attn
from .attention import DEFAULT_BLOCK_DECODE, eager_decode_attn, eager_past_attn, eager_tril_attn
from .attention_bwd import TrilRopeSelfAttnFn, _env_autograd_enabled, strict_tril_attn
from .rope import eager_rope_rotate, rope_cos_sin

ImplName = Literal["eager", "hip"]
_VALID = ("eager", "hip")
_ALIASES: dict = {}

DEFAULT_ATTN_AUTO_THRESHOLD = 512
_TRUTHY = ("1", "true", "yes", "on")

_ATTN_IMPL_ENV: object | None = object()
_ATTN_IMPL_RESOLVED: ImplName = "eager"
_ATTN_AUTO_ENV: object | None = object()
_ATTN_AUTO_ENABLED: bool = False
_ATTN_AUTO_THR_ENV: object | None = object()
_ATTN_AUTO_THR: int = DEFAULT_ATTN_AUTO_THRESHOLD
_ATTN_AUTO_COLD_THR_ENV: object | None = object()
_ATTN_AUTO_COLD_THR: int | None = None


def resolve_attn_impl(requested: str | None = None) -> ImplName:
    """Resolve ``BDH_ATTN_IMPL`` (or an explicit override); env string cached (reference :99-125)."""
    global _ATTN_IMPL_ENV, _ATTN_IMPL_RESOLVED

    def _normalize(raw: str) -> ImplName:
        raw = (raw or "eager").strip().lower()
        raw = _ALIASES.get(raw, raw)
        if raw not in _VALID:
            raise ValueError(f"BDH_ATTN_IMPL must be {'|'.join(_VALID)}, got {raw!r}")
        return raw  # type: ignore[return-value]

    if requested is not None:
        return _normalize(requested)
    env = os.environ.get("BDH_ATTN_IMPL", "eager")
    if env is _ATTN_IMPL_ENV or env == _ATTN_IMPL_ENV:
        return _ATTN_IMPL_RESOLVED
    resolved = _normalize(env or "eager")
    _ATTN_IMPL_ENV = env
    _ATTN_IMPL_RESOLVED = resolved
    return _ATTN_IMPL_RESOLVED


def attn_auto_enabled() -> bool:
    """True when ``BDH_ATTN_AUTO`` is truthy (``1|true|yes|on``)."""
    global _ATTN_AUTO_ENV, _ATTN_AUTO_ENABLED
    env = os.environ.get("BDH_ATTN_AUTO", "")
    if env is _ATTN_AUTO_ENV or env == _ATTN_AUTO_ENV:
        return _ATTN_AUTO_ENABLED
    _ATTN_AUTO_ENABLED = (env or "").strip().lower() in _TRUTHY
    _ATTN_AUTO_ENV = env
    return _ATTN_AUTO_ENABLED


def _parse_thr(name: str, raw: str) -> int:
    try:
        thr = int(raw)
    except ValueError as exc:
        raise ValueError(f"{name} must be an int, got {raw!r}") from exc
    if thr < 0:
        raise ValueError(f"{name} must be >= 0, got {thr}")
    return thr


def attn_auto_threshold() -> int:
    """Decode past-length threshold (default 512; reference :128-160)."""
    global _ATTN_AUTO_THR_ENV, _ATTN_AUTO_THR
    env = os.environ.get("BDH_ATTN_AUTO_THRESHOLD", "")
    if env is _ATTN_AUTO_THR_ENV or env == _ATTN_AUTO_THR_ENV:
        return _ATTN_AUTO_THR
    raw = (env or "").strip()
    thr = DEFAULT_ATTN_AUTO_THRESHOLD if not raw else _parse_thr("BDH_ATTN_AUTO_THRESHOLD", raw)
    _ATTN_AUTO_THR_ENV = env
    _ATTN_AUTO_THR = thr
    return _ATTN_AUTO_THR


def attn_auto_cold_threshold() -> int:
    """Cold/prefill threshold; mirrors :func:`attn_auto_threshold` when unset (reference :163-200)."""
    global _ATTN_AUTO_COLD_THR_ENV, _ATTN_AUTO_COLD_THR
    env = os.environ.get("BDH_ATTN_AUTO_COLD_THRESHOLD", "")
    if env is _ATTN_AUTO_COLD_THR_ENV or env == _ATTN_AUTO_COLD_THR_ENV:
        return attn_auto_threshold() if _ATTN_AUTO_COLD_THR is None else _ATTN_AUTO_COLD_THR
    raw = (env or "").strip()
    _ATTN_AUTO_COLD_THR = None if not raw else _parse_thr("BDH_ATTN_AUTO_COLD_THRESHOLD", raw)
    _ATTN_AUTO_COLD_THR_ENV = env
    return attn_auto_threshold() if _ATTN_AUTO_COLD_THR is None else _ATTN_AUTO_COLD_THR


_HIP_DTYPES = (torch.float32, torch.bfloat16)


def _hip_can_take(tensors) -> bool:
    """Whether the HIP library accepts these operands: ROCm device tensors in
    fp32 or bf16 (``None`` entries are ignored)."""
    return all(t is None or (t.is_cuda and t.dtype in _HIP_DTYPES) for t in tensors)


def _resolve_auto_impl(length: int, threshold: int, tensors=None) -> ImplName:
    """One strict AUTO gate: above the threshold prefer ``hip`` when it can run.

    Like the reference's switch (attention_dispatch.py:203-260), AUTO never
    picks a backend that would raise: with operands given, ``hip`` is chosen
    only when they are ROCm tensors in fp32/bf16; CPU tensors, other dtypes,
    a missing library or no device keep ``eager``.
    """
    if int(length) <= int(threshold):
        return "eager"
    if not hip_attn.hip_available():
        return "eager"
    if tensors is not None and not _hip_can_take(tensors):
        return "eager"
    return "hip"


def resolve_decode_impl(past_len: int, requested: str | None = None, *, tensors=None) -> ImplName:
    """T=1 decode backend with the optional AUTO switch (reference :210-231).

    ``tensors`` (the operands) lets AUTO keep ``eager`` for inputs the HIP
    library does not take; an explicit ``hip`` is returned as requested.
    """
    name = resolve_attn_impl(requested)
    if name != "eager" or not attn_auto_enabled():
        return name
    return _resolve_auto_impl(past_len, attn_auto_threshold(), tensors)


def resolve_cold_impl(seq_len: int, requested: str | None = None, *, tensors=None) -> ImplName:
    """Cold/prefill backend with the optional AUTO switch (reference :234-260)."""
    name = resolve_attn_impl(requested)
    if name != "eager" or not attn_auto_enabled():
        return name
    return _resolve_auto_impl(seq_len, attn_auto_cold_threshold(), tensors)


def _needs_grad(*ts: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def bdh_attn(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    *,
    impl: str | None = None,
    use_autograd_fn: Optional[bool] = None,
) -> torch.Tensor:
    """``tril(Q @ K.T, -1) @ V`` with the selected backend (reference :263-308)."""
    name = resolve_cold_impl(int(Q.size(2)), requested=impl, tensors=(Q, K, V))
    if use_autograd_fn is None:
        use_autograd_fn = _env_autograd_enabled()
    if name == "hip" and not use_autograd_fn and _needs_grad(Q, K, V):
        use_autograd_fn = True
    if use_autograd_fn:
        return strict_tril_attn(Q, K, V, impl=name, use_fn=True)
    if name == "eager":
        return eager_tril_attn(Q, K, V)
    return hip_attn.tril_score_v(Q, K, V)


def bdh_attn_rope(
    x: torch.Tensor,
    V: torch.Tensor,
    freqs: torch.Tensor,
    rope_start: int = 0,
    *,
    out_kr: Optional[torch.Tensor] = None,
    impl: str | None = None,
) -> torch.Tensor:
    """Cold BDH attention from the un-rotated latent: ``tril(R(x) R(x)^T, -1) @ V``.

    New surface entry of this build: the reference applies RoPE and then calls
    ``bdh_attn(QR, QR, V)`` (bdh.py:405-412).  ``hip`` fuses the rotation into
    the kernel's operand loads (and can write ``R(x)`` into ``out_kr``, the KR
    cache slot); ``eager`` does the same two steps with torch ops.
    """
    name = resolve_cold_impl(int(x.size(2)), requested=impl, tensors=(x, V, freqs))
    if name == "hip":
        if _needs_grad(x, V):
            if out_kr is not None:
                raise ValueError("out_kr is for inference (generate) calls; it cannot be used under autograd")
            return TrilRopeSelfAttnFn.apply(x, V, freqs, int(rope_start), None)
        return hip_attn.tril_rope_score_v(x, V, freqs, rope_start, qr_out=out_kr)
    cos, sin = rope_cos_sin(int(x.size(2)), int(rope_start), freqs)
    qr = eager_rope_rotate(x, cos, sin, out=out_kr)
    return bdh_attn(qr, qr, V, impl="eager")


def bdh_attn_past(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    past: int,
    *,
    impl: str | None = None,
) -> torch.Tensor:
    """T new queries after ``past`` cached rows: ``bdh_attn(K, K, V)[..., past:, :]``
    when ``Q`` is ``K[..., past:, :]`` (the reference's multi-token cached step,
    bdh.py:446-461, recomputes that whole attention and slices it).

    New surface entry of this build.  ``hip`` computes only the score tiles that
    reach a new row; ``eager`` recomputes past||new with torch ops as the
    reference does.  Inference only under ``hip`` (no autograd).
    """
    name = resolve_cold_impl(int(K.size(2)), requested=impl, tensors=(Q, K, V))
    if name == "eager":
        return eager_past_attn(Q, K, V, int(past))
    if _needs_grad(Q, K, V):
        raise ValueError("bdh_attn_past with impl='hip' is an inference entry; it has no backward")
    return hip_attn.tril_score_v_past(Q, K, V, int(past))


def bdh_attn_decode(
    Q: torch.Tensor,
    K_past: torch.Tensor,
    V_past: torch.Tensor,
    *,
    impl: str | None = None,
    block_size: int = DEFAULT_BLOCK_DECODE,
) -> torch.Tensor:
    """Queries against the packed past only (reference :311-347); never T x T."""
    del block_size  # tiling is internal to the HIP kernel
    name = resolve_decode_impl(int(K_past.size(2)), requested=impl, tensors=(Q, K_past, V_past))
    if name == "eager":
        return eager_decode_attn(Q, K_past, V_past)
    return hip_attn.tril_decode(Q, K_past, V_past)


def backend_info() -> dict:
    """Diagnostics for benchmarks and logs (reference :350-389)."""
    impl = resolve_attn_impl()
    return {
        "BDH_ATTN_IMPL": impl,
        "BDH_ATTN_AUTOGRAD": _env_autograd_enabled(),
        "BDH_ATTN_AUTO": attn_auto_enabled(),
        "BDH_ATTN_AUTO_THRESHOLD": attn_auto_threshold(),
        "BDH_ATTN_AUTO_COLD_THRESHOLD": attn_auto_cold_threshold(),
        "has_hip_ext": hip_attn.has_hip_ext(),
        "has_hip_kernel": hip_attn.has_hip_kernel(),
        "auto_prefers": "hip" if hip_attn.hip_available() else "eager",
        "cuda": torch.cuda.is_available(),
        "effective": impl,
        "ext_status": hip_attn.ext_status(),
    }


__all__ = [
    "DEFAULT_ATTN_AUTO_THRESHOLD",
    "resolve_attn_impl",
    "resolve_cold_impl",
    "resolve_decode_impl",
    "attn_auto_enabled",
    "attn_auto_threshold",
    "attn_auto_cold_threshold",
    "bdh_attn",
    "bdh_attn_rope",
    "bdh_attn_past",
    "bdh_attn_decode",
    "backend_info",
]
