"""Write ``fixtures.npz``: seeded inputs and CPU-oracle outputs at small shapes.

The fixtures pin the oracle against regressions
(tests/test_surface.py::test_golden_fixtures_reproduce recomputes them) and
give the GPU tests reference outputs that do not depend on running the oracle.  Inputs follow the BASELINE seeds: latent
Q = relu(0.32 * N(0,1)) (seed 0), V ~ N(0,1) (seed 1), dY ~ N(0,1) (seed 2).

Run from the repo root:  ``python tests/golden/make_fixtures.py``
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle as O  # noqa: E402


def _randn(shape, seed):
    return torch.randn(shape, generator=torch.Generator("cpu").manual_seed(seed), dtype=torch.float32).numpy()


def build() -> dict:
    B, H, T, N, D = 2, 2, 40, 16, 8
    x = np.maximum(0.32 * _randn((B, H, T, N), 0), 0).astype(np.float32)
    k = np.maximum(0.32 * _randn((B, H, T, N), 3), 0).astype(np.float32)
    v = _randn((B, 1, T, D), 1)
    dy = _randn((B, H, T, D), 2)
    freqs = O.get_freqs(N)
    start = 3
    cold = O.tril_score_v_cpu(x, k, v)
    rope_out, qr = O.tril_rope_score_v(x, v, freqs, start)
    dx, dv_rope = O.tril_rope_score_v_backward(x, v, dy, freqs, start)
    dq, dk, dv = O.analytic_tril_attn_backward_blocked(x, k, v, dy)
    S = 25
    q1 = np.maximum(0.32 * _randn((B, H, 1, N), 4), 0).astype(np.float32)
    dec = O.tril_decode_cpu(q1, qr[:, :, :S], v[:, :, :S])
    cos, sin = O.rope_cos_sin(T, start, freqs)
    xb = O.bf16_round(x)
    rope_bf16 = O.rope_rotate(xb, cos, sin, bf16=True)
    return {
        "x": x, "k": k, "v": v, "dy": dy, "freqs": freqs, "rope_start": np.array(start),
        "cold_out": cold, "rope_out": rope_out, "qr": qr, "rope_dx": dx, "rope_dv": dv_rope,
        "bwd_dq": dq, "bwd_dk": dk, "bwd_dv": dv,
        "dec_q": q1, "dec_S": np.array(S), "dec_out": dec,
        "cos": cos, "sin": sin, "x_bf16": xb, "rope_bf16": rope_bf16,
    }


def main() -> None:
    path = HERE / "fixtures.npz"
    np.savez_compressed(path, **build())
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
