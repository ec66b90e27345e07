"""``bdh_hip_ext``: Python binding of the gfx950 C-ABI library ``libbdh_hip.so``.

Counterpart of the reference's native module ``bdh_cuda_ext`` (pybind module of
csrc/tril_attn_bind.cpp:25-40): same entry names (``tril_score_v``,
``tril_decode`` and their ``*_hip`` device-specific spellings) plus the
entries this build adds (fused RoPE forward/backward, analytic backward, RoPE
apply).  Only ROCm device tensors are accepted; there is no CPU path in this
module (``has_hip`` is the analogue of the reference's ``has_cuda``).

The C ABI (``include/bdh_hip.h``) takes plain pointers, sizes and strides;
PyTorch is used here only for device memory (outputs and workspaces come from
its caching allocator) and for the current stream.

Importing this module loads the library and fails loudly (ImportError) when it
is missing or does not export the expected symbols.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional, Sequence, Tuple

import torch

__all__ = [
    "has_hip",
    "has_cuda",
    "lib_path",
    "version",
    "tril_score_v",
    "tril_score_v_hip",
    "tril_score_v_cpu",
    "tril_score_v_past",
    "tril_rope_score_v",
    "tril_decode",
    "tril_decode_hip",
    "tril_decode_cpu",
    "tril_decode_noalloc",
    "tril_score_v_bwd",
    "keeps_scores",
    "tril_score_v_save",
    "tril_score_v_bwd_saved",
    "tril_rope_score_v_bwd",
    "rope_keeps_scores",
    "tril_rope_score_v_save",
    "tril_rope_score_v_bwd_saved",
    "rope_rotate",
    "relu_mul",
    "gated_gemm",
    "relu_gemm",
    "gated_decoder",
    "small_gemm",
    "layer_norm_rows",
    "profile_enable",
    "profile_collect",
    "launch_count",
    "EXPORTED_SYMBOLS",
]

BDH_F32 = 0
BDH_BF16 = 1

EXPORTED_SYMBOLS = (
    "bdh_version",
    "bdh_error_string",
    "bdh_tril_score_v_workspace",
    "bdh_tril_score_v",
    "bdh_tril_score_v_past_workspace",
    "bdh_tril_score_v_past",
    "bdh_tril_rope_score_v",
    "bdh_tril_decode_workspace",
    "bdh_tril_decode",
    "bdh_tril_decode_noalloc",
    "bdh_rope_rotate",
    "bdh_tril_score_v_bwd_workspace",
    "bdh_tril_score_v_bwd",
    "bdh_tril_score_v_keeps_scores",
    "bdh_tril_score_v_bwd_saved_workspace",
    "bdh_tril_score_v_bwd_saved",
    "bdh_tril_rope_score_v_bwd_workspace",
    "bdh_tril_rope_score_v_bwd",
    "bdh_tril_rope_score_v_keeps_scores",
    "bdh_tril_rope_score_v_bwd_saved_workspace",
    "bdh_tril_rope_score_v_bwd_saved",
    "bdh_relu_mul",
    "bdh_gated_gemm",
    "bdh_relu_gemm",
    "bdh_gated_decoder_workspace",
    "bdh_gated_decoder",
    "bdh_small_gemm_workspace",
    "bdh_small_gemm",
    "bdh_layer_norm_rows",
    "bdh_layer_norm_rows2",
    "bdh_profile_enable",
    "bdh_profile_collect",
)


class Tensor4(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("size", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


def _find_lib() -> Path:
    env = os.environ.get("BDH_HIP_LIB")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "libbdh_hip.so"


def _load():
    path = _find_lib()
    if not path.exists():
        raise ImportError(
            f"bdh_hip_ext: {path} not found; build it with "
            "`python bdh-gpu-fast_amd/build.py` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(str(path))
    missing = [s for s in EXPORTED_SYMBOLS if not hasattr(lib, s)]
    if missing:
        raise ImportError(f"bdh_hip_ext: {path} lacks symbols {missing}")
    P = ctypes.POINTER(Tensor4)
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    fp = ctypes.POINTER(ctypes.c_float)
    sig = {
        "bdh_version": (ctypes.c_char_p, []),
        "bdh_error_string": (ctypes.c_char_p, [ctypes.c_int]),
        "bdh_tril_score_v_workspace": (sz, [i64, i64, i64, i64, i64, i32]),
        "bdh_tril_score_v": (ctypes.c_int, [P, P, P, P, vp, sz, vp]),
        "bdh_tril_score_v_past_workspace": (sz, [i64, i64, i64, i64, i64, i64, i32]),
        "bdh_tril_score_v_past": (ctypes.c_int, [P, P, P, P, i64, vp, sz, vp]),
        "bdh_tril_rope_score_v": (ctypes.c_int, [P, P, P, fp, i64, P, vp, sz, vp]),
        "bdh_tril_decode_workspace": (sz, [i64, i64, i64, i64, i64, i64]),
        "bdh_tril_decode": (ctypes.c_int, [P, P, P, P, vp, sz, vp]),
        "bdh_tril_decode_noalloc": (ctypes.c_int, [P, P, P, P, vp]),
        "bdh_rope_rotate": (ctypes.c_int, [P, P, P, P, i32, vp]),
        "bdh_tril_score_v_bwd_workspace": (sz, [i64, i64, i64, i64, i64, i64, i32]),
        "bdh_tril_score_v_bwd": (ctypes.c_int, [P, P, P, P, P, P, P, vp, sz, vp]),
        "bdh_tril_score_v_keeps_scores": (ctypes.c_int, [P, P, ctypes.POINTER(sz)]),
        "bdh_tril_score_v_bwd_saved_workspace": (sz, [i64, i64, i64, i64, i64, i64, i32]),
        "bdh_tril_score_v_bwd_saved": (ctypes.c_int, [P, P, P, P, P, vp, sz, vp, sz, vp]),
        "bdh_tril_rope_score_v_bwd_workspace": (sz, [i64, i64, i64, i64, i64, i64, i32]),
        "bdh_tril_rope_score_v_bwd": (ctypes.c_int, [P, P, P, fp, i64, P, P, vp, sz, vp]),
        "bdh_tril_rope_score_v_keeps_scores": (ctypes.c_int, [P, P, ctypes.POINTER(sz)]),
        "bdh_tril_rope_score_v_bwd_saved_workspace": (sz, [i64, i64, i64, i64, i64, i64, i32]),
        "bdh_tril_rope_score_v_bwd_saved": (ctypes.c_int, [P, P, P, fp, i64, P, P, vp, sz, vp, sz, vp]),
        "bdh_relu_mul": (ctypes.c_int, [P, P, P, vp]),
        "bdh_layer_norm_rows": (ctypes.c_int, [P, P, P, vp]),
        "bdh_layer_norm_rows2": (ctypes.c_int, [P, P, P, P, vp]),
        "bdh_gated_gemm": (ctypes.c_int, [P, P, P, P, vp]),
        "bdh_relu_gemm": (ctypes.c_int, [P, P, P, vp]),
        "bdh_gated_decoder_workspace": (sz, [i64, i64]),
        "bdh_gated_decoder": (ctypes.c_int, [P, P, P, P, P, vp, sz, vp]),
        "bdh_small_gemm_workspace": (sz, [i64, i64, i64]),
        "bdh_small_gemm": (ctypes.c_int, [P, P, P, vp, sz, vp]),
        "bdh_profile_enable": (None, [i32]),
        "bdh_profile_collect": (ctypes.c_int, [ctypes.c_char_p, i32, fp, i32]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib, path


_lib, _path = _load()
has_hip = True
# The reference's pybind module reports has_cuda (tril_attn_bind.cpp:34-39); this
# library has no CUDA path, so a caller probing that attribute sees False.
has_cuda = False
lib_path = str(_path)
_launches = 0


def version() -> str:
    return _lib.bdh_version().decode()


def launch_count() -> int:
    """Number of successful library entry-point calls made through this module."""
    return _launches


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return BDH_F32
    if t.dtype == torch.bfloat16:
        return BDH_BF16
    raise TypeError(f"bdh_hip_ext supports float32 and bfloat16 tensors, got {t.dtype}")


def _t4(t: torch.Tensor) -> Tensor4:
    if t.dim() != 4:
        raise ValueError(f"bdh_hip_ext expects 4-D tensors, got shape {tuple(t.shape)}")
    s = Tensor4()
    s.data = t.data_ptr() if t.numel() > 0 else None
    for i in range(4):
        s.size[i] = t.size(i)
        s.stride[i] = t.stride(i)
    s.dtype = _dtype_code(t)
    return s


def _require_device(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "bdh_hip_ext: tensors must live on a ROCm GPU (the HIP library has no CPU path); "
                f"got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"bdh_hip_ext: tensors on different devices ({dev} vs {t.device})")
    assert dev is not None
    return dev


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _check(rc: int, what: str) -> None:
    global _launches
    if rc != 0:
        raise RuntimeError(f"bdh_hip_ext.{what} failed: {_lib.bdh_error_string(rc).decode()} (code {rc})")
    _launches += 1


def _workspace(nbytes: int, dev: torch.device) -> Tuple[Optional[torch.Tensor], int]:
    if nbytes == 0:
        return None, 0
    return torch.empty(int(nbytes), dtype=torch.uint8, device=dev), int(nbytes)


def _freqs_ptr(freqs: torch.Tensor, n: int, dev: torch.device):
    if freqs.dtype != torch.float32:
        raise TypeError(f"freqs must be float32, got {freqs.dtype}")
    f = freqs.reshape(-1)
    if f.numel() != n:
        raise ValueError(f"freqs must hold {n} values (one per latent dim), got {f.numel()}")
    if f.device != dev:
        raise RuntimeError(f"freqs on {f.device}, tensors on {dev}")
    f = f.contiguous()
    return f, ctypes.cast(ctypes.c_void_p(f.data_ptr()), ctypes.POINTER(ctypes.c_float))


# ------------------------------------------------------------------- forward
def tril_score_v(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """``tril(q @ k^T, -1) @ v`` (no softmax, no scale) on the GPU; out in q's dtype."""
    dev = _require_device(q, k, v)
    B, H, T, Dk = q.shape
    out = torch.empty(B, H, T, v.size(-1), dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_workspace(B, H, T, Dk, v.size(-1), _dtype_code(q))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_score_v(
            ctypes.byref(_t4(q)), ctypes.byref(_t4(k)), ctypes.byref(_t4(v)), ctypes.byref(_t4(out)),
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_score_v")
    return out


tril_score_v_hip = tril_score_v


def tril_score_v_past(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, past: int) -> torch.Tensor:
    """Queries at an offset: ``out[..., i, :] = sum_{j < past+i} <q_i, k_j> v_j``.

    q ``(B,H,T,Dk)`` are rows ``past..past+T-1`` of the sequence k ``(B,H,past+T,Dk)``
    and v ``(B,1|H,past+T,Dv)`` cover; out ``(B,H,T,Dv)`` in q's dtype.
    """
    dev = _require_device(q, k, v)
    B, H, T, Dk = q.shape
    past = int(past)
    out = torch.empty(B, H, T, v.size(-1), dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_past_workspace(B, H, T, past, Dk, v.size(-1), _dtype_code(q))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_score_v_past(
            ctypes.byref(_t4(q)), ctypes.byref(_t4(k)), ctypes.byref(_t4(v)), ctypes.byref(_t4(out)),
            past, ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_score_v_past")
    return out


def keeps_scores(x: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether ``tril_score_v(x, x, v)`` leaves reusable score tiles in its workspace."""
    if not (x.is_cuda and v.is_cuda) or x.dim() != 4 or v.dim() != 4:
        return False
    return bool(_lib.bdh_tril_score_v_keeps_scores(ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), None))


def tril_score_v_save(x: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Self attention ``tril(x x^T, -1) v`` that also returns its workspace when
    it holds the score tiles (:func:`keeps_scores`), for
    :func:`tril_score_v_bwd_saved`; else ``(out, None)``."""
    dev = _require_device(x, v)
    B, H, T, N = x.shape
    out = torch.empty(B, H, T, v.size(-1), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_workspace(B, H, T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_score_v(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(out)),
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_score_v")
    return out, (ws if keeps_scores(x, v) else None)


def tril_rope_score_v(
    x: torch.Tensor,
    v: torch.Tensor,
    freqs: torch.Tensor,
    rope_start: int = 0,
    qr_out: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Cold BDH attention with RoPE fused into the loads: ``tril(R(x) R(x)^T, -1) v``.

    ``freqs`` is the (N,) or (1,1,1,N) fp32 frequency buffer (pairs share a
    value); positions are ``rope_start + t``.  ``qr_out`` optionally receives
    ``R(x)`` (e.g. the KR cache slot).
    """
    dev = _require_device(x, v, qr_out, out)
    B, H, T, N = x.shape
    f, fptr = _freqs_ptr(freqs, N, dev)
    if out is None:
        out = torch.empty(B, H, T, v.size(-1), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_workspace(B, H, T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_rope_score_v(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(out)), fptr, int(rope_start),
            ctypes.byref(_t4(qr_out)) if qr_out is not None else None,
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_rope_score_v")
    return out


def rope_keeps_scores(x: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether ``tril_rope_score_v(x, v, ...)`` (no ``qr_out``) leaves reusable
    score tiles in its workspace."""
    if not (x.is_cuda and v.is_cuda) or x.dim() != 4 or v.dim() != 4:
        return False
    return bool(_lib.bdh_tril_rope_score_v_keeps_scores(ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), None))


def tril_rope_score_v_save(
    x: torch.Tensor, v: torch.Tensor, freqs: torch.Tensor, rope_start: int = 0
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """:func:`tril_rope_score_v` that also returns its workspace when it holds
    the score tiles (:func:`rope_keeps_scores`), for
    :func:`tril_rope_score_v_bwd_saved`; else ``(out, None)``."""
    dev = _require_device(x, v)
    B, H, T, N = x.shape
    f, fptr = _freqs_ptr(freqs, N, dev)
    out = torch.empty(B, H, T, v.size(-1), dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_workspace(B, H, T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_rope_score_v(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(out)), fptr, int(rope_start), None,
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_rope_score_v")
    return out, (ws if rope_keeps_scores(x, v) else None)


def tril_rope_score_v_bwd_saved(
    x: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    freqs: torch.Tensor,
    rope_start: int,
    scores: torch.Tensor,
    *,
    dv: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(dx, dv)`` of :func:`tril_rope_score_v` from the score tiles kept by
    :func:`tril_rope_score_v_save` on the same ``x``, ``v``, ``freqs`` and
    ``rope_start`` (no recompute of the tiles)."""
    dev = _require_device(x, v, dout, scores, dv)
    B, H, T, N = x.shape
    f, fptr = _freqs_ptr(freqs, N, dev)
    dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    if dv is None:
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_rope_score_v_bwd_saved_workspace(B, H, v.size(1), T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_rope_score_v_bwd_saved(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(dout)), fptr, int(rope_start),
            ctypes.byref(_t4(dx)), ctypes.byref(_t4(dv)), scores.data_ptr(), scores.numel() * scores.element_size(),
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_rope_score_v_bwd_saved")
    return dx, dv


# ------------------------------------------------------------ CPU entries
def _acc_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.float32 if t.dtype in (torch.float16, torch.bfloat16) else t.dtype


def _require_cpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.device.type != "cpu":
            raise RuntimeError(f"bdh_hip_ext CPU entry: tensors must be on the CPU, got {t.device}")


def tril_score_v_cpu(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """CPU cold op, ``tril(q @ k^T, -1) @ v`` in torch, fp32 accumulation for 16-bit
    inputs and the result in q's dtype: the entry the reference module exports
    beside its device kernel (csrc/tril_attn_bind.cpp:29 -> tril_attn_cpu.cpp:160-174).
    The device path never comes here."""
    _require_cpu(q, k, v)
    acc = _acc_dtype(q)
    s = torch.matmul(q.to(acc), k.to(acc).transpose(-2, -1).contiguous())
    s.tril_(-1)
    return torch.matmul(s, v.to(acc)).to(q.dtype)


def tril_decode_cpu(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """CPU decode, ``(q @ k_past^T) @ v_past`` in torch (fp32 accumulation for 16-bit
    inputs, result in q's dtype); reference csrc/tril_attn_bind.cpp:32 ->
    tril_attn_cpu.cpp:212-238."""
    _require_cpu(q, k_past, v_past)
    acc = _acc_dtype(q)
    s = torch.matmul(q.to(acc), k_past.to(acc).transpose(-2, -1).contiguous())
    return torch.matmul(s, v_past.to(acc)).to(q.dtype)


# -------------------------------------------------------------------- decode
def tril_decode(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """``(q @ k_past^T) @ v_past`` against the packed past (strided cache views OK)."""
    dev = _require_device(q, k_past, v_past)
    B, H, Tq, Dk = q.shape
    S = k_past.size(2)
    Dv = v_past.size(-1)
    out = torch.empty(B, H, Tq, Dv, dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_decode_workspace(B, H, Tq, S, Dk, Dv)
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_decode(
            ctypes.byref(_t4(q)), ctypes.byref(_t4(k_past)), ctypes.byref(_t4(v_past)), ctypes.byref(_t4(out)),
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_decode")
    return out


tril_decode_hip = tril_decode


def tril_decode_noalloc(
    q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor, out: Optional[torch.Tensor] = None
) -> torch.Tensor:
    """Decode through ``bdh_tril_decode_noalloc``: no workspace; the partial sums
    go to the library's per-GPU scratch array, so calls that overlap in time on
    one GPU race.  ``out`` (B, H, Tq, Dv) defaults to a fresh tensor in q's dtype
    (the entry point itself allocates nothing)."""
    dev = _require_device(q, k_past, v_past, out)
    B, H, Tq, _ = q.shape
    if out is None:
        out = torch.empty(B, H, Tq, v_past.size(-1), dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.bdh_tril_decode_noalloc(
            ctypes.byref(_t4(q)), ctypes.byref(_t4(k_past)), ctypes.byref(_t4(v_past)), ctypes.byref(_t4(out)),
            _stream(dev),
        )
    _check(rc, "tril_decode_noalloc")
    return out


# ------------------------------------------------------------------ backward
def tril_score_v_bwd(
    q: torch.Tensor,
    k: Optional[torch.Tensor],
    v: torch.Tensor,
    dout: torch.Tensor,
    *,
    dq: Optional[torch.Tensor] = None,
    dk: Optional[torch.Tensor] = None,
    dv: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], torch.Tensor]:
    """Analytic gradients of ``tril(q k^T, -1) v``.

    ``k is None`` means self attention (k is q): returns ``(dq + dk, None, dv)``.
    Otherwise ``(dq, dk, dv)``.  Gradients take their input's dtype unless
    output tensors (any float dtype, same shapes) are passed.
    """
    dev = _require_device(q, k, v, dout, dq, dk, dv)
    B, H, T, N = q.shape
    if dq is None:
        dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    if dk is None and k is not None:
        dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    if k is None:
        dk = None
    if dv is None:
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_bwd_workspace(B, H, v.size(1), T, N, v.size(-1), _dtype_code(q))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_score_v_bwd(
            ctypes.byref(_t4(q)), ctypes.byref(_t4(k)) if k is not None else None, ctypes.byref(_t4(v)),
            ctypes.byref(_t4(dout)), ctypes.byref(_t4(dq)), ctypes.byref(_t4(dk)) if dk is not None else None,
            ctypes.byref(_t4(dv)), ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_score_v_bwd")
    return dq, dk, dv


def tril_score_v_bwd_saved(
    x: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    scores: torch.Tensor,
    *,
    dx: Optional[torch.Tensor] = None,
    dv: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(dx, dv)`` of self attention from the score tiles saved by
    :func:`tril_score_v_save` on the same ``x`` (no recompute)."""
    dev = _require_device(x, v, dout, scores, dx, dv)
    B, H, T, N = x.shape
    if dx is None:
        dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    if dv is None:
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_score_v_bwd_saved_workspace(B, H, v.size(1), T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_score_v_bwd_saved(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(dout)), ctypes.byref(_t4(dx)),
            ctypes.byref(_t4(dv)), scores.data_ptr(), scores.numel() * scores.element_size(),
            ws.data_ptr() if ws is not None else None, nb, _stream(dev),
        )
    _check(rc, "tril_score_v_bwd_saved")
    return dx, dv


def tril_rope_score_v_bwd(
    x: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    freqs: torch.Tensor,
    rope_start: int = 0,
    *,
    dv: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gradients ``(dx, dv)`` of :func:`tril_rope_score_v` (``dv`` may be passed
    in any float dtype; it defaults to ``v``'s)."""
    dev = _require_device(x, v, dout, dv)
    B, H, T, N = x.shape
    f, fptr = _freqs_ptr(freqs, N, dev)
    dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    if dv is None:
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    with torch.cuda.device(dev):
        need = _lib.bdh_tril_rope_score_v_bwd_workspace(B, H, v.size(1), T, N, v.size(-1), _dtype_code(x))
        ws, nb = _workspace(need, dev)
        rc = _lib.bdh_tril_rope_score_v_bwd(
            ctypes.byref(_t4(x)), ctypes.byref(_t4(v)), ctypes.byref(_t4(dout)), fptr, int(rope_start),
            ctypes.byref(_t4(dx)), ctypes.byref(_t4(dv)), ws.data_ptr() if ws is not None else None, nb,
            _stream(dev),
        )
    _check(rc, "tril_rope_score_v_bwd")
    return dx, dv


# ---------------------------------------------------------------------- RoPE
def rope_rotate(
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    *,
    backward: bool = False,
) -> torch.Tensor:
    """Adjacent-pair RoPE with caller tables; ``cos``/``sin`` broadcast to ``v``.

    ``v`` may have 1 to 4 dims (leading dims are padded to 4); ``out`` defaults
    to a fresh contiguous tensor of ``v``'s dtype.
    """
    dev = _require_device(v, cos, sin, out)
    shape = tuple(v.shape)
    pad = (1,) * (4 - v.dim())
    if v.dim() > 4:
        raise ValueError(f"rope_rotate supports up to 4 dims, got {v.dim()}")
    v4 = v.reshape(pad + shape) if pad else v
    c4 = cos.expand(shape).reshape(pad + shape) if pad else cos.expand(shape)
    s4 = sin.expand(shape).reshape(pad + shape) if pad else sin.expand(shape)
    if out is None:
        out = torch.empty(shape, dtype=v.dtype, device=dev)
    o4 = out.view(pad + shape) if pad else out
    with torch.cuda.device(dev):
        rc = _lib.bdh_rope_rotate(
            ctypes.byref(_t4(v4)), ctypes.byref(_t4(c4)), ctypes.byref(_t4(s4)), ctypes.byref(_t4(o4)),
            1 if backward else 0, _stream(dev),
        )
    _check(rc, "rope_rotate")
    return out


# ---------------------------------------------------------------- profiling
def relu_mul(x: torch.Tensor, y: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x * relu(y)`` elementwise for 4-D views of one shape; ``out`` defaults to a
    contiguous tensor in x's dtype."""
    dev = _require_device(x, y, out)
    if x.dim() != 4 or y.shape != x.shape:
        raise ValueError(f"relu_mul: x and y must be 4-D of one shape, got {tuple(x.shape)} and {tuple(y.shape)}")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.bdh_relu_mul(ctypes.byref(_t4(x)), ctypes.byref(_t4(y)), ctypes.byref(_t4(out)), _stream(dev))
    _check(rc, "relu_mul")
    return out


def layer_norm_rows(y: torch.Tensor, x: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
                    out: Optional[torch.Tensor] = None, out_bf16: Optional[torch.Tensor] = None) -> torch.Tensor:
    """LayerNorm over the last dim (no affine, eps 1e-5): ``LN(y)``, or ``LN(x + LN(y))``
    with ``x``; 1- to 4-D tensors of one shape, fp32 or bf16; ``out`` defaults to a
    contiguous tensor in ``out_dtype`` (y's dtype).  ``out_bf16`` (bf16, y's shape, any
    strides) also receives the result rounded once to bf16."""
    dev = _require_device(y, x, out, out_bf16)
    if x is not None and x.shape != y.shape:
        raise ValueError(f"layer_norm_rows: x {tuple(x.shape)} and y {tuple(y.shape)} differ")
    if out is None:
        out = torch.empty(y.shape, dtype=out_dtype or y.dtype, device=dev)

    def v4(t: torch.Tensor) -> torch.Tensor:
        return t.reshape((1,) * (4 - t.dim()) + tuple(t.shape)) if t.dim() < 4 else t

    with torch.cuda.device(dev):
        if out_bf16 is None:
            rc = _lib.bdh_layer_norm_rows(ctypes.byref(_t4(v4(x))) if x is not None else None,
                                          ctypes.byref(_t4(v4(y))), ctypes.byref(_t4(v4(out))), _stream(dev))
        else:
            if out_bf16.shape != y.shape:
                raise ValueError(f"layer_norm_rows: out_bf16 {tuple(out_bf16.shape)} and y {tuple(y.shape)} differ")
            rc = _lib.bdh_layer_norm_rows2(ctypes.byref(_t4(v4(x))) if x is not None else None,
                                           ctypes.byref(_t4(v4(y))), ctypes.byref(_t4(v4(out))),
                                           ctypes.byref(_t4(v4(out_bf16))), _stream(dev))
    _check(rc, "layer_norm_rows")
    return out


def gated_gemm(y: torch.Tensor, wt: torch.Tensor, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x * relu(y @ wt^T)`` per head, bf16: y (B, nh, T, K), wt (nh, N, K), x (B, T, nh, N)."""
    dev = _require_device(y, wt, x, out)
    if wt.dim() != 3:
        raise ValueError(f"gated_gemm: wt must be (nh, N, K), got {tuple(wt.shape)}")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.bdh_gated_gemm(ctypes.byref(_t4(y)), ctypes.byref(_t4(wt.unsqueeze(0))), ctypes.byref(_t4(x)),
                                 ctypes.byref(_t4(out)), _stream(dev))
    _check(rc, "gated_gemm")
    return out


def relu_gemm(y: torch.Tensor, wt: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``relu(y @ wt^T)`` per head, bf16: y (B, nh, T, K) (head stride 0 when the
    heads share it), wt (nh, N, K) -> (B, T, nh, N)."""
    dev = _require_device(y, wt, out)
    if wt.dim() != 3 or y.dim() != 4:
        raise ValueError(f"relu_gemm: y (B, nh, T, K) and wt (nh, N, K), got {tuple(y.shape)}, {tuple(wt.shape)}")
    B, nh, T, _ = y.shape
    if out is None:
        out = torch.empty(B, T, nh, wt.size(1), dtype=y.dtype, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.bdh_relu_gemm(ctypes.byref(_t4(y)), ctypes.byref(_t4(wt.unsqueeze(0))), ctypes.byref(_t4(out)),
                                _stream(dev))
    _check(rc, "relu_gemm")
    return out


def gated_decoder(y: torch.Tensor, wt: torch.Tensor, x: torch.Tensor, dec: torch.Tensor,
                  out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``(x * relu(y @ wt^T)).view(B, T, nh*N) @ dec`` in one pass, bf16 operands:
    y (B, nh, T, K), wt (nh, N, K), x (B, T, nh, N), dec (nh*N, D) -> (B, T, D) in
    ``out_dtype`` (default fp32).  K = D = 256, N a multiple of 32."""
    dev = _require_device(y, wt, x, dec)
    if wt.dim() != 3 or dec.dim() != 2 or x.dim() != 4:
        raise ValueError(f"gated_decoder: wt (nh, N, K), dec (nh*N, D), x (B, T, nh, N); got "
                         f"{tuple(wt.shape)}, {tuple(dec.shape)}, {tuple(x.shape)}")
    B, T, nh, N = x.shape
    out = torch.empty(B, T, dec.size(1), dtype=out_dtype or torch.float32, device=dev)
    with torch.cuda.device(dev):
        ws, nb = _workspace(_lib.bdh_gated_decoder_workspace(nh, B * T), dev)
        rc = _lib.bdh_gated_decoder(ctypes.byref(_t4(y)), ctypes.byref(_t4(wt.unsqueeze(0))), ctypes.byref(_t4(x)),
                                    ctypes.byref(_t4(dec.view(1, 1, *dec.shape))),
                                    ctypes.byref(_t4(out.view(B, T, 1, -1))),
                                    ws.data_ptr() if ws is not None else None, nb, _stream(dev))
    _check(rc, "gated_decoder")
    return out


def small_gemm(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``a @ b`` for few rows of a: a (M, K), b (K, D) bf16 -> (M, D) in ``out_dtype`` (default a's)."""
    dev = _require_device(a, b)
    if a.dim() != 2 or b.dim() != 2 or a.size(1) != b.size(0):
        raise ValueError(f"small_gemm: a (M, K) and b (K, D), got {tuple(a.shape)} and {tuple(b.shape)}")
    M, K = a.shape
    D = b.size(1)
    out = torch.empty(M, D, dtype=out_dtype or a.dtype, device=dev)
    with torch.cuda.device(dev):
        ws, nb = _workspace(_lib.bdh_small_gemm_workspace(M, K, D), dev)
        rc = _lib.bdh_small_gemm(ctypes.byref(_t4(a.view(1, 1, M, K))), ctypes.byref(_t4(b.view(1, 1, K, D))),
                                 ctypes.byref(_t4(out.view(1, 1, M, D))),
                                 ws.data_ptr() if ws is not None else None, nb, _stream(dev))
    _check(rc, "small_gemm")
    return out


def profile_enable(on: bool = True) -> None:
    """Bracket every library kernel launch with HIP events (on its stream)."""
    _lib.bdh_profile_enable(1 if on else 0)


def profile_collect(max_records: int = 65536) -> Sequence[Tuple[str, float]]:
    """Wait for and return ``(kernel_name, ms)`` for launches since the last collect."""
    name_len = 64
    names = ctypes.create_string_buffer(name_len * max_records)
    ms = (ctypes.c_float * max_records)()
    n = _lib.bdh_profile_collect(names, name_len, ms, max_records)
    raw = names.raw
    return [
        (raw[i * name_len:(i + 1) * name_len].split(b"\0", 1)[0].decode(), float(ms[i])) for i in range(n)
    ]
