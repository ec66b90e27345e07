"""GPU parity of the score x V kernel that moves its operands through an LDS
ring (``k_sv_dma``: score tiles of one split, bf16 V), against the CPU oracle.

out[b, h, i] = sum over j < i of M_h[i, j] V[b, hv, j] with M the score tiles
rounded once to bf16 (csrc/tril_attn_cpu.cpp:160-174 through the oracle's
``tril_score_v_cpu``; with RoPE ``tril_rope_score_v``, bdh.py:396-413).  The
A operand is read out of the score kernel's accumulator order by transposing
LDS reads.  Shapes have B * nh * (tiles per slab) >= 129, so the plan keeps
one split and the ring kernel runs (checked in the launch log): ragged T
(1000, 700, 33, 520), D below 256 (192, 64, 128) and above (512: two
256-column launches), per-head V, the relative-RoPE tile order, queries at an
offset.  Tolerance: bf16 2e-2 relative Frobenius on the batch elements the
oracle covers; repeated calls give the same bits.
"""

from __future__ import annotations

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
    (8, 4, 520, 256, 512, 1),
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
def test_ring_sv_matches_oracle(shape):
    B, H, T, N, D, Hv = shape
    print(f"ring S.V {shape}", flush=True)
    q = to_dev(O.bf16_round(latent((B, H, T, N), 51)), BF)
    v = to_dev(O.bf16_round(normal((B, Hv, T, D), 52)), BF)
    out, names = _kernels_of(lambda: ext.tril_score_v(q, q, v))
    assert "k_sv_dma" in names and "k_sy_sv" not in names, names
    assert torch.equal(out, ext.tril_score_v(q, q, v))
    for b in _slabs(B):
        want = O.tril_score_v_cpu(np_of(q[b:b + 1]), np_of(q[b:b + 1]), np_of(v[b:b + 1]))
        e = rel_fro(np_of(out[b:b + 1]), want)
        print(f"  batch {b}: rel {e:.3e}", flush=True)
        assert e <= TOL[BF]


def test_ring_sv_relative_rope_tiles():
    """The fused RoPE op (relative-RoPE score tiles) at one split: two batch
    elements against the oracle's RoPE attention."""
    B, H, T, N, D = 8, 4, 520, 512, 256
    x = to_dev(O.bf16_round(latent((B, H, T, N), 61)), BF)
    v = to_dev(O.bf16_round(normal((B, 1, T, D), 62)), BF)
    f = kernels.get_freqs(N).to(x.device)
    out, names = _kernels_of(lambda: ext.tril_rope_score_v(x, v, f, 0))
    assert "k_sv_dma" in names, names
    for b in _slabs(B):
        want, _ = O.tril_rope_score_v(np_of(x[b:b + 1]), np_of(v[b:b + 1]), np_of(f), 0)
        e = rel_fro(np_of(out[b:b + 1]), want)
        print(f"  batch {b}: rel {e:.3e}", flush=True)
        assert e <= TOL[BF]


@pytest.mark.parametrize("past,T", [(100, 300), (256, 256)])
def test_ring_sv_queries_at_an_offset(past, T):
    """Queries at an offset (rows below past not stored, row i at i - past) over
    enough slabs for one split: against the oracle."""
    B, H, N, D = 64, 4, 256, 128
    k = to_dev(O.bf16_round(latent((B, H, past + T, N), 71)), BF)
    v = to_dev(O.bf16_round(normal((B, 1, past + T, D), 72)), BF)
    got, names = _kernels_of(lambda: ext.tril_score_v_past(k[:, :, past:], k, v, past))
    assert "k_sv_dma" in names, names
    for b in _slabs(B):
        kk = np_of(k[b:b + 1])
        want = O.tril_score_v_past(kk[:, :, past:], kk, np_of(v[b:b + 1]), past)
        assert rel_fro(np_of(got[b:b + 1]), want) <= TOL[BF]
