"""The reference's ``kernels.cuda_attn`` names, served by the gfx950 library.

Counterpart of reference kernels/cuda_attn.py:1-513.  Code written against
that module (tests, benches, ``from kernels import tril_score_v_ref, ...``)
imports the same names from here:

- the tile constants and pickers (cuda_attn.py:52-71, 134-301) — pure integer
  functions, kept value-for-value because callers assert on them; the gfx950
  kernels do not use them (their tiles are fixed 256x256 score tiles, 64-row
  S.V blocks and 64-key decode chunks);
- the golden torch references ``tril_score_v_ref`` / ``tril_decode_ref`` and
  their tiled CPU mirrors (cuda_attn.py:305-383, 434-487);
- the native dispatchers ``tril_score_v`` / ``tril_decode`` (cuda_attn.py:391-414,
  490-502) and the probes ``has_cuda_ext`` / ``has_cuda_kernel`` / ``ext_status``.

One behaviour differs on purpose.  The reference's dispatchers swallow any
native error and fall back to the torch reference (cuda_attn.py:407-409).  Here
ROCm tensors go to the HIP library and its errors are raised: a silent
substitute would let a measurement time the wrong path.  CPU tensors run the
library module's CPU entries, as the reference's pybind module routes them
(tril_attn_bind.cpp:3-23); without the library they run the torch references,
as the reference does when its extension is absent.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import hip_attn
from .attention import _two_gemm_decode

# Tile constants of the reference surface (cuda_attn.py:52-71).
CUDA_TILE_M = 16
CUDA_TILE_N = 16
CUDA_TILE_D = 32
CUDA_TILE_M_MAX = 32
CUDA_TILE_N_MAX = 64
CUDA_TILE_M_CPU_MAX = 128
CUDA_TILE_N_CPU_MAX = 128
CUDA_DECODE_TILE_N = 32
CUDA_DECODE_TILE_N_MAX = 128
CUDA_DECODE_TILE_N_CPU_MAX = 512
_SMEM_CAP = 48 * 1024
_SCORE_ELEMS_EAGER_OK = 256 * 256
_COLD_SCORE_ELEMS_BUDGET = 256 * 256

_check_cold_shapes = hip_attn._check_cold_shapes
_check_decode_shapes = hip_attn._check_decode_shapes


def has_cuda_ext() -> bool:
    """True when the native library loaded (the reference's "extension imported")."""
    return hip_attn.has_hip_ext()


def has_cuda_kernel() -> bool:
    """True when the library loaded and a device is visible.  On PyTorch-ROCm the
    ``cuda`` device type is the HIP device, so this is the reference's
    "built with a device kernel" probe (cuda_attn.py:93-97)."""
    return hip_attn.has_hip_kernel()


def ext_status() -> str:
    """One-line status in the reference's format (cuda_attn.py:505-513)."""
    if not hip_attn.has_hip_ext():
        err = hip_attn._ext_load_error
        detail = f"{type(err).__name__}: {err}" if err is not None else "not attempted"
        return f"native=unavailable ({detail})"
    dev = "yes" if has_cuda_kernel() else "no"
    return f"native=loaded has_cuda_kernel={dev} has_decode=yes backend=hip-gfx950"


def _pow2_ceil(x: int, lo: int, hi: int) -> int:
    """Smallest ``lo * 2^k`` >= clamp(x, lo, hi), never above ``hi``."""
    x = max(lo, min(int(x), hi))
    p = lo
    while p < x and p * 2 <= hi:
        p *= 2
    return p


def _want_cold(T: int, for_smem: bool, wide_head: bool) -> int:
    if T <= 64:
        return 16
    if T <= 256:
        return 32
    want = 64 if for_smem else 128
    if wide_head:
        want = min(want, 32 if for_smem else 64)
    return want


def pick_cuda_cold_tiles(
    T: int,
    Dk: int = 64,
    *,
    Dv: int | None = None,
    for_smem: bool = False,
    tile_m: int | None = None,
    tile_n: int | None = None,
) -> tuple[int, int]:
    """Query/key tile widths of the reference's cold kernel (cuda_attn.py:134-223).

    Powers of two from 16: 16 up to T=64, 32 up to T=256, then 128 for the CPU
    mirrors (64 with ``for_smem``), halved for wide heads (Dk > 64 or Dv > 128);
    ``for_smem`` then shrinks the pair until a float tile set fits 48 KiB.
    Explicit widths are rounded up to the same power-of-two ladder.
    """
    hi_m = CUDA_TILE_M_MAX if for_smem else CUDA_TILE_M_CPU_MAX
    hi_n = CUDA_TILE_N_MAX if for_smem else CUDA_TILE_N_CPU_MAX
    T = max(int(T), 1)
    wide = int(Dk) > 64 or (Dv is not None and int(Dv) > 128)
    want = _want_cold(T, for_smem, wide)
    tm = _pow2_ceil(tile_m if tile_m is not None else min(T, want), 16, hi_m)
    tn = _pow2_ceil(tile_n if tile_n is not None else min(T, want), 16, hi_n)
    if for_smem:
        dk = max(int(Dk), 1)

        def smem(a: int, b: int) -> int:
            return 4 * (a * dk + b * dk + b * CUDA_TILE_D)

        while (tm > CUDA_TILE_M or tn > CUDA_TILE_N) and smem(tm, tn) > _SMEM_CAP:
            if tn > tm and tn > CUDA_TILE_N:
                tn //= 2
            elif tm > CUDA_TILE_M:
                tm //= 2
            elif tn > CUDA_TILE_N:
                tn //= 2
            else:
                break
        tm, tn = min(tm, CUDA_TILE_M_MAX), min(tn, CUDA_TILE_N_MAX)
    return max(16, tm), max(16, tn)


def pick_cuda_decode_tile_n(
    S: int,
    Dk: int = 64,
    *,
    for_smem: bool = False,
    tile_n: int | None = None,
) -> int:
    """Past-key tile width of the reference's decode kernel (cuda_attn.py:239-300):
    32 / 64 / 128 / 256 / 512 for S up to 64 / 256 / 1024 / 2048 / beyond, capped
    at 512 for the CPU mirrors and 128 (and a 48 KiB float tile set) with ``for_smem``."""
    hi = CUDA_DECODE_TILE_N_MAX if for_smem else CUDA_DECODE_TILE_N_CPU_MAX
    if tile_n is not None:
        tn = _pow2_ceil(tile_n, 16, hi)
    else:
        S = max(int(S), 1)
        want = 32 if S <= 64 else 64 if S <= 256 else 128 if S <= 1024 else 256 if S <= 2048 else 512
        tn = _pow2_ceil(min(S, want), 16, hi)
    if for_smem:
        dk = max(int(Dk), 1)

        def smem(n: int) -> int:
            return 4 * (dk + n * dk + n * CUDA_TILE_D)

        while tn > CUDA_DECODE_TILE_N and smem(tn) > _SMEM_CAP:
            tn //= 2
        if smem(CUDA_DECODE_TILE_N) <= _SMEM_CAP:
            tn = max(tn, CUDA_DECODE_TILE_N)
        tn = min(tn, CUDA_DECODE_TILE_N_MAX)
    return max(16, tn)


def _cold_score_budget(T: int, tm: int) -> int:
    """Score elements one past product may hold (cuda_attn.py:226-236)."""
    budget = max(tm * tm, _COLD_SCORE_ELEMS_BUDGET)
    if int(T) >= 256:
        budget = max(budget, tm * min(int(T), 1024))
    return budget


def _acc(t: torch.Tensor) -> torch.dtype:
    return torch.float32 if t.dtype in (torch.float16, torch.bfloat16) else t.dtype


def tril_score_v_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Golden reference ``(q @ k^T).tril(-1) @ v`` (cuda_attn.py:305-323); V broadcasts over heads."""
    _check_cold_shapes(q, k, v)
    s = q @ k.transpose(-2, -1).contiguous()
    return s.tril(diagonal=-1) @ v


def tril_score_v_tiled_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tile_m: int | None = None,
    tile_n: int | None = None,
) -> torch.Tensor:
    """The reference's tiled cold mirror (cuda_attn.py:326-388): per query tile, the
    keys before it in one product when (rows x past) fits the budget, else in key
    chunks, then the tile's own strictly-lower block; fp32 sums for 16-bit inputs."""
    _check_cold_shapes(q, k, v)
    B, H, T, _ = q.shape
    D = v.size(-1)
    if T == 0:
        return q.new_zeros(B, H, 0, D)
    tm, tn = pick_cuda_cold_tiles(T, q.size(-1), Dv=D, tile_m=tile_m, tile_n=tile_n)
    budget = _cold_score_budget(T, tm)
    acc = _acc(q)
    qf, kf, vf = q.to(acc), k.to(acc), v.to(acc)
    out = torch.zeros(B, H, T, D, device=q.device, dtype=acc)
    for r0 in range(0, T, tm):
        r1 = min(r0 + tm, T)
        rows = r1 - r0
        qi = qf[:, :, r0:r1]
        dst = out[:, :, r0:r1]
        if r0 > 0:
            chunk = r0 if rows * r0 <= budget else max(tn, budget // max(rows, 1))
            for c0 in range(0, r0, chunk):
                c1 = min(c0 + chunk, r0)
                dst.add_((qi @ kf[:, :, c0:c1].transpose(-2, -1).contiguous()) @ vf[:, :, c0:c1])
        if rows > 1:
            s = (qi @ kf[:, :, r0:r1].transpose(-2, -1).contiguous()).tril(diagonal=-1)
            dst.add_(s @ vf[:, :, r0:r1])
    return out if out.dtype == q.dtype else out.to(q.dtype)


def tril_decode_ref(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """Decode reference ``(q @ k_past^T) @ v_past`` (cuda_attn.py:417-448): one two-GEMM
    product while Tq x S <= 65536, else the tiled mirror."""
    B, H, Tq, S, D = _check_decode_shapes(q, k_past, v_past)
    if S == 0:
        return q.new_zeros(B, H, Tq, D)
    if Tq * S <= _SCORE_ELEMS_EAGER_OK:
        return _two_gemm_decode(q, k_past, v_past)
    return tril_decode_tiled_ref(q, k_past, v_past)


def tril_decode_tiled_ref(
    q: torch.Tensor,
    k_past: torch.Tensor,
    v_past: torch.Tensor,
    *,
    tile_n: int | None = None,
) -> torch.Tensor:
    """The reference's tiled decode mirror (cuda_attn.py:451-487): the past in key
    chunks of ``pick_cuda_decode_tile_n`` width, fp32 sums for 16-bit inputs."""
    B, H, Tq, S, D = _check_decode_shapes(q, k_past, v_past)
    if S == 0:
        return q.new_zeros(B, H, Tq, D)
    tn = pick_cuda_decode_tile_n(S, q.size(-1), tile_n=tile_n)
    acc = _acc(q)
    qf, kf, vf = q.to(acc), k_past.to(acc), v_past.to(acc)
    out = torch.zeros(B, H, Tq, D, device=q.device, dtype=acc)
    for c0 in range(0, S, tn):
        c1 = min(c0 + tn, S)
        out.add_(_two_gemm_decode(qf, kf[:, :, c0:c1], vf[:, :, c0:c1]))
    return out.to(q.dtype)


def _native_module():
    return hip_attn._ext


def tril_score_v(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Cold op dispatch (cuda_attn.py:391-414): ROCm tensors run the HIP kernels
    (errors raised, never replaced), CPU tensors the library's CPU entry, or the
    torch references when the library is absent."""
    _check_cold_shapes(q, k, v)
    if q.is_cuda:
        return hip_attn.tril_score_v(q, k, v)
    ext = _native_module()
    if ext is not None:
        return ext.tril_score_v_cpu(q, k, v)
    T = q.size(2)
    return tril_score_v_tiled_ref(q, k, v) if T * T > _SCORE_ELEMS_EAGER_OK else tril_score_v_ref(q, k, v)


def tril_decode(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """Decode dispatch (cuda_attn.py:490-502), with the same routing as :func:`tril_score_v`."""
    _check_decode_shapes(q, k_past, v_past)
    if q.is_cuda:
        return hip_attn.tril_decode(q, k_past, v_past)
    ext = _native_module()
    if ext is not None:
        return ext.tril_decode_cpu(q, k_past, v_past)
    return tril_decode_ref(q, k_past, v_past)


__all__ = [
    "CUDA_TILE_M",
    "CUDA_TILE_N",
    "CUDA_TILE_D",
    "CUDA_TILE_M_MAX",
    "CUDA_TILE_N_MAX",
    "CUDA_TILE_M_CPU_MAX",
    "CUDA_TILE_N_CPU_MAX",
    "CUDA_DECODE_TILE_N",
    "CUDA_DECODE_TILE_N_MAX",
    "CUDA_DECODE_TILE_N_CPU_MAX",
    "ext_status",
    "has_cuda_ext",
    "has_cuda_kernel",
    "pick_cuda_cold_tiles",
    "pick_cuda_decode_tile_n",
    "tril_decode",
    "tril_decode_ref",
    "tril_decode_tiled_ref",
    "tril_score_v",
    "tril_score_v_ref",
    "tril_score_v_tiled_ref",
]
