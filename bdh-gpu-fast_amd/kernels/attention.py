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


__all__ = [
    "DEFAULT_BLOCK_COLD",
    "DEFAULT_BLOCK_DECODE",
    "eager_tril_attn",
    "eager_decode_attn",
    "eager_past_attn",
    "_two_gemm_decode",
]
