"""Strict lower-triangular BDH attention: tril(Q @ K.T, diagonal=-1) @ V.

No softmax, no 1/sqrt(d).  Position i attends only to j < i.

This module keeps the reference's ``eager`` backend (plain PyTorch ops, the
default of ``BDH_ATTN_IMPL``; reference kernels/attention.py:27-40 and
:193-219, :1356-1366) so callers that never select ``hip`` behave exactly as
before.  The MI355X kernels live behind ``BDH_ATTN_IMPL=hip``
(:mod:`kernels.hip_attn`).
"""

from __future__ import annotations

import torch

# Default tile widths of the reference surface (kernels/attention.py:43-46).
DEFAULT_BLOCK_COLD = 64
DEFAULT_BLOCK_DECODE = 256


def eager_tril_attn(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """Materialise full T x T scores, ``tril_(-1)``, then ``@ V`` (kernels/attention.py:27-40).

    Q, K: (B, H, T, N); V: (B, 1, T, D) or (B, H, T, D) -> (B, H, T, D).
    Kᵀ is materialised before the batched product: bf16 batched products with
    a transposed-view operand have faulted ROCm GPUs.  Same values.
    """
    scores = Q @ K.transpose(-2, -1).contiguous()
    scores.tril_(diagonal=-1)
    return scores @ V


def eager_past_attn(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, past: int) -> torch.Tensor:
    """Queries at offset ``past`` the way the reference's multi-token cached step
    gets them: strict-tril attention over the whole past||new sequence, last T rows
    kept (bdh.py:446-461).  Q: (B, H, T, N) are rows past.. of K: (B, H, past+T, N).
    The rows before ``past`` are zero queries here, so they add nothing.
    """
    if past == 0:
        return eager_tril_attn(Q, K, V)
    B, H, _, N = Q.shape
    q_all = torch.cat([Q.new_zeros(B, H, past, N), Q], dim=2)
    return eager_tril_attn(q_all, K, V)[..., past:, :]


def _two_gemm_decode(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """``(Q @ K.mT) @ V`` for decode against the packed past (kernels/attention.py:193-219)."""
    B, H, Tq, N = Q.shape
    S = K.size(2)
    D = V.size(-1)
    if S == 0:
        return Q.new_zeros(B, H, Tq, D)
    if Tq == 1 and V.size(1) == H:
        scores = torch.bmm(Q.reshape(B * H, 1, N), K.reshape(B * H, S, N).transpose(1, 2).contiguous())
        return torch.bmm(scores, V.reshape(B * H, S, D)).view(B, H, 1, D)
    return (Q @ K.transpose(-2, -1).contiguous()) @ V


def eager_decode_attn(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor) -> torch.Tensor:
    """Reference decode ``(Q @ K.mT) @ V`` (past only; kernels/attention.py:1356-1366)."""
    return _two_gemm_decode(Q, K, V)


# The reference's Triton backend is not part of this package (the gfx950 path
# is hand-written HIP).  Its probes keep their names and answer "unavailable",
# so callers that ask before choosing a backend take another one.

def pick_cold_block_size(T: int, block_size: int | None = None) -> int:
    """Cold query-tile width (kernels/attention.py:542-553): 64, or 128 from T = 256."""
    if block_size is not None:
        return max(1, int(block_size))
    return min(128, 2 * DEFAULT_BLOCK_COLD) if int(T) >= 256 else DEFAULT_BLOCK_COLD


def pick_triton_cold_tiles(
    T: int,
    N: int = 64,
    D: int = 128,
    *,
    block_m: int | None = None,
    block_n: int | None = None,
) -> tuple[int, int, int, int]:
    """``(BLOCK_M, BLOCK_N, BLOCK_D, BLOCK_K)`` of the reference's cold Triton tiles
    (kernels/attention.py:98-164): query/key widths from :func:`pick_cold_block_size`,
    at most 64 for wide heads (N > 64 or D > 128), and D / N widths, each rounded up
    to a power of two within [16, 128] (D and N within [16, 64])."""

    def ceil_pow2(x: int, lo: int, hi: int) -> int:
        x = max(lo, min(int(x), hi))
        p = 1
        while p < x:
            p *= 2
        return min(p, hi)

    wide = N > 64 or D > 128
    want = pick_cold_block_size(T)
    if wide:
        want = min(want, DEFAULT_BLOCK_COLD)
    bm = ceil_pow2(block_m, 16, 128) if block_m is not None else ceil_pow2(min(T, want) if T > 0 else want, 16, 128)
    bn = ceil_pow2(block_n, 16, 128) if block_n is not None else ceil_pow2(min(max(T, 1), want), 16, 128)
    return bm, bn, ceil_pow2(D if D > 0 else 1, 16, 64), ceil_pow2(N if N > 0 else 1, 16, 64)


def triton_decode_available() -> bool:
    """Always False: this package ships no Triton decode (kernels/attention.py:800-807)."""
    return False


def triton_cold_skip_reason() -> str | None:
    """Why the Triton cold kernel is not used (kernels/attention.py:810-827): it is not
    part of this package; ``BDH_ATTN_IMPL=hip`` runs the gfx950 kernels."""
    return "Triton backend not built into this package; BDH_ATTN_IMPL=hip selects the gfx950 kernels (CPU-safe skip)"


__all__ = [
    "DEFAULT_BLOCK_COLD",
    "DEFAULT_BLOCK_DECODE",
    "eager_tril_attn",
    "eager_decode_attn",
    "eager_past_attn",
    "_two_gemm_decode",
    "pick_cold_block_size",
    "pick_triton_cold_tiles",
    "triton_decode_available",
    "triton_cold_skip_reason",
]
