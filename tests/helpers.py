"""Shared test helpers: seeded inputs (BASELINE seeds), error metrics, devices."""

from __future__ import annotations

import numpy as np
import torch

import oracle as O


def rel_fro(got, want) -> float:
    """Relative Frobenius error ||got - want|| / ||want|| (0 when both are 0)."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    den = np.linalg.norm(w.ravel())
    num = np.linalg.norm((g - w).ravel())
    if den == 0.0:
        return float(num)
    return float(num / den)


def gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def latent(shape, seed: int = 0) -> np.ndarray:
    """Q = K = relu(0.32 * N(0,1)): the sparse BDH latent (about half zeros)."""
    g = torch.randn(shape, generator=gen(seed), dtype=torch.float32)
    return torch.relu(0.32 * g).numpy()


def normal(shape, seed: int) -> np.ndarray:
    return torch.randn(shape, generator=gen(seed), dtype=torch.float32).numpy()


def to_dev(a: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)


def as_dtype_values(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """The float32 values a tensor of ``dtype`` holds (bf16 rounding applied)."""
    return O.bf16_round(a) if dtype == torch.bfloat16 else np.asarray(a, np.float32)


def np_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
