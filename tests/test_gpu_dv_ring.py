"""GPU parity of the dV kernel that moves its operands through an LDS ring
(``k_dv_dma``: score tiles of one split, taken by the backward from kept or
recomputed tiles), against the CPU oracle.

dV[b, hv] = sum over heads h and rows i > j of M_h[i, j] dO_h[i, :], M the
forward's score tiles rounded once to bf16 (kernels/attention_bwd.py:259-291
through the oracle's ``self_attn_backward`` / ``tril_rope_score_v_backward``).
Shapes have B * nh * (tiles per slab) >= 129, so the plan keeps one split and
the ring kernel runs (checked in the launch log): ragged T (1000, 700, 33,
520), D below 256 (192, 64, 128), per-head V, a single 64-row block, fp32
and bf16 dV, the relative-RoPE tile order.  Tolerance: bf16 2e-2 relative
Frobenius on the batch elements the oracle covers; doubling dO doubles dV
exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, latent, normal, np_of, rel_fro, to_dev

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402
import kernels  # noqa: E402

BF = torch.bfloat16

SHAPES = [
    # B, H, T, N, D, Hv
    (16, 4, 1024, 256, 256, 1),
    (8, 4, 1000, 256, 192, 1),
    (8, 4, 700, 256, 64, 4),
    (130, 1, 33, 256, 128, 1),
]


def _kernels_of(fn):
    ext.profile_enable(True)
    try:
        out = fn()
        torch.cuda.synchronize()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    return out, names


def _slabs(B):
    return [0, B - 1] if B > 1 else [0]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("fp32_dv", [False, True])
def test_ring_dv_matches_oracle(shape, fp32_dv):
    B, H, T, N, D, Hv = shape
    print(f"ring dV {shape} fp32_dv={fp32_dv}", flush=True)
    q = to_dev(O.bf16_round(latent((B, H, T, N), 21)), BF)
    v = to_dev(O.bf16_round(normal((B, Hv, T, D), 22)), BF)
    d = to_dev(O.bf16_round(normal((B, H, T, D), 23)), BF)
    _, scores = ext.tril_score_v_save(q, v)
    assert scores is not None
    dv0 = torch.empty(B, Hv, T, D, dtype=torch.float32 if fp32_dv else BF, device=q.device)
    (_, dv), names = _kernels_of(lambda: ext.tril_score_v_bwd_saved(q, v, d, scores, dv=dv0))
    assert "k_dv_dma" in names and "k_dv_sy" not in names, names
    _, dv2 = ext.tril_score_v_bwd_saved(q, v, d * 2, scores, dv=torch.empty_like(dv0))
    assert torch.equal(dv2, dv * 2)
    for b in _slabs(B):
        _, wv = O.self_attn_backward(np_of(q[b:b + 1]), np_of(v[b:b + 1]), np_of(d[b:b + 1]))
        e = rel_fro(np_of(dv[b:b + 1]), wv)
        print(f"  batch {b}: dv rel {e:.3e}", flush=True)
        assert e <= TOL[BF]


def test_ring_dv_recompute_route_equals_kept_tiles():
    """The backward that recomputes the tiles runs the same dV kernel on the same
    tiles: its dV equals the kept-tiles dV bit for bit."""
    B, H, T, N, D, Hv = SHAPES[1]
    q = to_dev(O.bf16_round(latent((B, H, T, N), 31)), BF)
    v = to_dev(O.bf16_round(normal((B, Hv, T, D), 32)), BF)
    d = to_dev(O.bf16_round(normal((B, H, T, D), 33)), BF)
    _, scores = ext.tril_score_v_save(q, v)
    _, dv_s = ext.tril_score_v_bwd_saved(q, v, d, scores)
    (_, _, dv_r), names = _kernels_of(lambda: ext.tril_score_v_bwd(q, None, v, d))
    assert "k_dv_dma" in names, names
    assert torch.equal(dv_s, dv_r)


def test_ring_dv_relative_rope_tiles():
    """Tiles kept by the relative-RoPE forward (fragment slot order of that
    kernel): dV against the oracle's RoPE backward on two batch elements."""
    B, H, T, N, D = 8, 4, 520, 512, 256
    print(f"ring dV, relative RoPE tiles {(B, H, T, N, D)}", flush=True)
    x = to_dev(O.bf16_round(latent((B, H, T, N), 41)), BF)
    v = to_dev(O.bf16_round(normal((B, 1, T, D), 42)), BF)
    d = to_dev(O.bf16_round(normal((B, H, T, D), 43)), BF)
    f = kernels.get_freqs(N).to(x.device)
    _, scores = ext.tril_rope_score_v_save(x, v, f, 0)
    assert scores is not None
    (_, dv), names = _kernels_of(lambda: ext.tril_rope_score_v_bwd_saved(x, v, d, f, 0, scores))
    assert "k_dv_dma" in names, names
    for b in _slabs(B):
        _, wv = O.tril_rope_score_v_backward(np_of(x[b:b + 1]), np_of(v[b:b + 1]), np_of(d[b:b + 1]), np_of(f), 0)
        e = rel_fro(np_of(dv[b:b + 1]), wv)
        print(f"  batch {b}: dv rel {e:.3e}", flush=True)
        assert e <= TOL[BF]
