"""MI355X (gfx950) native backend behind ``BDH_ATTN_IMPL=hip``.

Counterpart of the reference's kernels/cuda_attn.py: shape validation with the
same ``ValueError`` contract (cuda_attn.py:103-131), then the HIP library via
:mod:`bdh_hip_ext`.  Unlike the reference wrapper there is **no silent
fallback**: when ``hip`` is requested and the library is missing, or the
tensors are not on a ROCm device, a ``RuntimeError`` is raised, so a
measurement can never time a substitute path.

Semantics::

    tril_score_v(q, k, v)      = (q @ k.T).tril(-1) @ v          (no softmax, no scale)
    tril_decode(q, k_past, v)  = (q @ k_past.T) @ v_past          (all past keys valid)
    tril_rope_score_v(x, v, freqs, rope_start)
                               = tril_score_v(R(x), R(x), v),  R = BDH RoPE fused in-kernel
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

_ext = None
_ext_load_error: Optional[BaseException] = None
try:
    import bdh_hip_ext as _ext  # type: ignore
except Exception as exc:  # ImportError or missing symbols: reported, never hidden
    _ext = None
    _ext_load_error = exc


def has_hip_ext() -> bool:
    """True if the native HIP library loaded."""
    return _ext is not None


def has_hip_kernel() -> bool:
    """True if the library loaded and a ROCm device is visible."""
    return _ext is not None and torch.cuda.is_available()


def hip_available() -> bool:
    return has_hip_kernel()


def _require(*ts: Optional[torch.Tensor]):
    if _ext is None:
        raise RuntimeError(
            "BDH_ATTN_IMPL=hip requested but the HIP library is not loaded "
            f"({type(_ext_load_error).__name__}: {_ext_load_error}); build it with "
            "`python bdh-gpu-fast_amd/build.py`"
        )
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"BDH_ATTN_IMPL=hip needs ROCm device tensors, got a tensor on {t.device}"
            )
    return _ext


def _check_cold_shapes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Input contract of the cold op (reference kernels/cuda_attn.py:103-111)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4D (B, H, T, D)")
    if q.shape != k.shape:
        raise ValueError(f"q and k shapes must match, got {tuple(q.shape)} vs {tuple(k.shape)}")
    if v.size(0) != q.size(0) or v.size(2) != q.size(2):
        raise ValueError("v batch/seq must match q")
    if v.size(1) not in (1, q.size(1)):
        raise ValueError("v heads must equal q heads or 1")


def _check_decode_shapes(
    q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor
) -> Tuple[int, int, int, int, int]:
    """Input contract of decode (reference kernels/cuda_attn.py:114-131)."""
    if q.dim() != 4 or k_past.dim() != 4 or v_past.dim() != 4:
        raise ValueError("q, k_past, v_past must be 4D")
    B, H, Tq, Dk = q.shape
    S = k_past.size(2)
    if k_past.shape[:2] != (B, H) or k_past.size(-1) != Dk:
        raise ValueError(f"k_past shape {tuple(k_past.shape)} incompatible with q {tuple(q.shape)}")
    if v_past.size(0) != B or v_past.size(2) != S:
        raise ValueError(f"v_past shape {tuple(v_past.shape)} incompatible with k_past S={S}")
    if v_past.size(1) not in (1, H):
        raise ValueError("v_past heads must equal q heads or 1")
    return B, H, Tq, S, v_past.size(-1)


def _last_dim_unit(t: torch.Tensor) -> torch.Tensor:
    """The library needs a unit-stride last dim; other strides are passed through."""
    if t.size(-1) > 1 and t.stride(-1) != 1:
        return t.contiguous()
    return t


def tril_score_v(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """``tril(q @ k^T, -1) @ v`` on the GPU (out in q's dtype, fp32 accumulation)."""
    _check_cold_shapes(q, k, v)
    ext = _require(q, k, v)
    same = q is k
    q = _last_dim_unit(q)
    k = q if same else _last_dim_unit(k)
    return ext.tril_score_v(q, k, _last_dim_unit(v))


def _check_past_shapes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, past: int) -> None:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 4D (B, H, T, D)")
    if past < 0:
        raise ValueError(f"past must be >= 0, got {past}")
    B, H, T, N = q.shape
    if tuple(k.shape) != (B, H, past + T, N):
        raise ValueError(f"k must be (B, H, past+T, N) = {(B, H, past + T, N)}, got {tuple(k.shape)}")
    if v.size(0) != B or v.size(2) != past + T or v.size(1) not in (1, H):
        raise ValueError(f"v must be (B, 1|H, past+T, D), got {tuple(v.shape)}")


def tril_score_v_past(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, past: int) -> torch.Tensor:
    """Queries at an offset (chunked prefill): rows ``past..past+T-1`` of the
    strict-tril attention over k, v of length ``past+T``; out (B, H, T, D)."""
    past = int(past)
    _check_past_shapes(q, k, v, past)
    ext = _require(q, k, v)
    if q.dtype != k.dtype:
        raise TypeError(f"q and k dtypes differ: {q.dtype} vs {k.dtype}")
    return ext.tril_score_v_past(_last_dim_unit(q), _last_dim_unit(k), _last_dim_unit(v), past)


def relu_mul(x: torch.Tensor, y: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x * relu(y)`` on the GPU (the BDH layer's gated product, bdh.py:914-945)."""
    ext = _require(x, y, out)
    return ext.relu_mul(_last_dim_unit(x), _last_dim_unit(y), out)


def gated_gemm(y: torch.Tensor, wt: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """``x * relu(y @ wt^T)`` per head on the GPU (encoder_v GEMM + gated product, bdh.py:914-945)."""
    ext = _require(y, wt, x)
    return ext.gated_gemm(y, wt, x)


def relu_gemm(y: torch.Tensor, wt: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``relu(y @ wt^T)`` per head on the GPU, (B, T, nh, N) bf16 (the encoder and its
    ReLU, bdh.py:861-912); y (B, nh, T, K) may share one row set over the heads
    (head stride 0); ``out`` may be a strided (B, T, nh, N) view (padded rows)."""
    ext = _require(y, wt, out)
    return ext.relu_gemm(y, wt, out)


def gated_decoder(y: torch.Tensor, wt: torch.Tensor, x: torch.Tensor, dec: torch.Tensor,
                  out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``(x * relu(y @ wt^T)) @ decoder`` in one pass on the GPU (bdh.py:914-945), the
    product never stored; fp32 output unless ``out_dtype`` says otherwise."""
    ext = _require(y, wt, x, dec)
    return ext.gated_decoder(y, wt, x, dec, out_dtype)


def layer_norm_rows(y: torch.Tensor, x: Optional[torch.Tensor] = None,
                    out_dtype: Optional[torch.dtype] = None, out_bf16: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``LN(y)`` or ``LN(x + LN(y))`` over the last dim on the GPU (bdh.py:565-574, 731-750);
    ``out_bf16`` (bf16, y's shape) also receives the result rounded once to bf16."""
    ext = _require(y, x, out_bf16)
    return ext.layer_norm_rows(_last_dim_unit(y), _last_dim_unit(x) if x is not None else None, out_dtype,
                               out_bf16=out_bf16)


def small_gemm(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``a @ b`` for few rows of a on the GPU, split over K (the decoder product of a decode step)."""
    ext = _require(a, b)
    return ext.small_gemm(a, b, out_dtype)


def tril_rope_score_v(
    x: torch.Tensor,
    v: torch.Tensor,
    freqs: torch.Tensor,
    rope_start: int = 0,
    *,
    qr_out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Cold BDH attention with RoPE fused into the kernel loads."""
    _check_cold_shapes(x, x, v)
    if x.size(-1) % 2 != 0:
        raise ValueError(f"RoPE last dim must be even, got {x.size(-1)}")
    ext = _require(x, v, qr_out)
    check_pair_freqs(freqs)
    if qr_out is not None and (qr_out.shape != x.shape or qr_out.device != x.device):
        raise ValueError("qr_out must match x shape/device")
    return ext.tril_rope_score_v(_last_dim_unit(x), _last_dim_unit(v), freqs, int(rope_start), qr_out=qr_out)


def tril_decode(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """``(q @ k_past^T) @ v_past``; capacity-strided cache views are read in place."""
    _check_decode_shapes(q, k_past, v_past)
    ext = _require(q, k_past, v_past)
    return ext.tril_decode(_last_dim_unit(q), _last_dim_unit(k_past), _last_dim_unit(v_past))


def tril_score_v_bwd(q, k, v, dout):
    """Analytic gradients; ``k is None`` -> self attention (merged dq+dk)."""
    ext = _require(q, k, v, dout)
    return ext.tril_score_v_bwd(
        _last_dim_unit(q), None if k is None else _last_dim_unit(k), _last_dim_unit(v), _last_dim_unit(dout)
    )


def tril_score_v_save(x: torch.Tensor, v: torch.Tensor):
    """Self-attention forward that also returns its score tiles for the backward
    (``(out, scores)``; ``scores`` is None when the shapes take another path)."""
    _check_cold_shapes(x, x, v)
    ext = _require(x, v)
    return ext.tril_score_v_save(_last_dim_unit(x), _last_dim_unit(v))


def tril_score_v_bwd_saved(x, v, dout, scores):
    """Merged dx and dv from the score tiles saved by :func:`tril_score_v_save`."""
    ext = _require(x, v, dout, scores)
    return ext.tril_score_v_bwd_saved(_last_dim_unit(x), _last_dim_unit(v), _last_dim_unit(dout), scores)


def tril_rope_score_v_save(x: torch.Tensor, v: torch.Tensor, freqs: torch.Tensor, rope_start: int = 0):
    """Fused RoPE forward that also returns its score tiles for the backward
    (``(out, scores)``; ``scores`` is None when the shapes take another path)."""
    _check_cold_shapes(x, x, v)
    if x.size(-1) % 2 != 0:
        raise ValueError(f"RoPE last dim must be even, got {x.size(-1)}")
    ext = _require(x, v)
    check_pair_freqs(freqs)
    return ext.tril_rope_score_v_save(_last_dim_unit(x), _last_dim_unit(v), freqs, int(rope_start))


def tril_rope_score_v_bwd_saved(x, v, dout, freqs, rope_start: int, scores, *, dv=None):
    """dx and dv of the fused RoPE op from the score tiles saved by
    :func:`tril_rope_score_v_save`."""
    ext = _require(x, v, dout, scores)
    return ext.tril_rope_score_v_bwd_saved(
        _last_dim_unit(x), _last_dim_unit(v), _last_dim_unit(dout), freqs, int(rope_start), scores, dv=dv
    )


def tril_rope_score_v_bwd(x, v, dout, freqs, rope_start: int = 0, *, dv=None):
    ext = _require(x, v, dout)
    return ext.tril_rope_score_v_bwd(
        _last_dim_unit(x), _last_dim_unit(v), _last_dim_unit(dout), freqs, int(rope_start), dv=dv
    )


_PAIR_CHECKED: dict = {}


def check_pair_freqs(freqs: torch.Tensor) -> None:
    """The fused kernel assumes pair-shared frequencies (bdh.py:41-49 layout).

    Checked once per (storage, version) of the buffer, then cached.
    """
    key = (freqs.data_ptr(), freqs._version, freqs.numel(), str(freqs.device))
    if _PAIR_CHECKED.get(key):
        return
    f = freqs.reshape(-1)
    if f.dtype != torch.float32:
        raise ValueError(f"freqs must be float32, got {f.dtype}")
    if f.numel() % 2 != 0 or not torch.equal(f[0::2], f[1::2]):
        raise ValueError("fused RoPE needs pair-shared frequencies (freq[2m] == freq[2m+1])")
    _PAIR_CHECKED[key] = True


def ext_status() -> str:
    """Human-readable status (reference kernels/cuda_attn.py:505-513)."""
    if _ext is None:
        err = _ext_load_error
        detail = f"{type(err).__name__}: {err}" if err is not None else "not attempted"
        return f"native=unavailable ({detail})"
    gpu = "yes" if torch.cuda.is_available() else "no"
    return f"native=loaded ({_ext.version()}, {_ext.lib_path}) gpu={gpu} has_decode=yes has_bwd=yes"


__all__ = [
    "has_hip_ext",
    "has_hip_kernel",
    "hip_available",
    "tril_score_v",
    "tril_score_v_past",
    "relu_mul",
    "gated_gemm",
    "gated_decoder",
    "relu_gemm",
    "small_gemm",
    "tril_rope_score_v",
    "tril_decode",
    "tril_score_v_bwd",
    "tril_rope_score_v_bwd",
    "check_pair_freqs",
    "ext_status",
    "_check_cold_shapes",
    "_check_decode_shapes",
]
