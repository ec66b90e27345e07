"""GPU parity of the fused-RoPE backward on the MFMA route.

bf16 self attention with RoPE (``tril_rope_score_v_bwd``, the backward of
``TrilRopeSelfAttnFn`` that ``bdh_attn_rope`` uses under autograd): one
absolute-position score kernel recomputes M's tiles and writes R(x), dV comes
from the tiles, G from dO and V, and the dQ kernel forms dx = R^T(G R(x)),
applying R^T to its fp32 sums in the epilogue.  Checked against the oracle's gradients
(oracle/tril_attn_oracle.py ``tril_rope_score_v_backward``, the reference's
attention_bwd.py:45-83 composed with rope.py:543-556) at the bf16 tolerance
(2e-2, relative Frobenius), against the generic kernels on the same inputs,
and through autograd with an fp32 V (the AMP case: V is the LayerNorm output).
Each case checks that the route ran (its dQ kernel in the launch log).  The
route from the score tiles the forward kept (no recompute) is checked against
the recompute route and the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import latent, normal, np_of, rel_fro, to_dev

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)
import kernels  # noqa: E402

DEV = "cuda"
BF = torch.bfloat16
TOL = 2e-2


def _names(fn):
    torch.cuda.synchronize()
    ext.profile_enable(True)
    try:
        out = fn()
        torch.cuda.synchronize()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    return out, names


# (B, H, T, N, D, Hv, rope_start)
SHAPES = [
    (2, 2, 260, 256, 64, 1, 3),
    (1, 3, 517, 512, 128, 3, 0),
    (2, 4, 1, 256, 256, 1, 5),
    (1, 2, 700, 768, 256, 1, 1000),
    (3, 1, 256, 256, 64, 1, 0),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_rope_backward_mfma_route_matches_oracle(shape):
    B, H, T, N, D, Hv, start = shape
    print(f"rope bwd route {shape}", flush=True)
    x = O.bf16_round(latent((B, H, T, N), 0))
    v = O.bf16_round(normal((B, Hv, T, D), 1))
    dO = O.bf16_round(normal((B, H, T, D), 2))
    f = O.get_freqs(N)
    xd, vd, dd = to_dev(x, BF), to_dev(v, BF), to_dev(dO, BF)
    fd = torch.from_numpy(f).to(DEV)
    (dx, dv), names = _names(lambda: ext.tril_rope_score_v_bwd(xd, vd, dd, fd, start))
    assert "k_dq_sy" in names and names & {"k_dv_sy", "k_dv_dma"}, names
    wx, wv = O.tril_rope_score_v_backward(x, v, dO, f, start)
    ex, ev = rel_fro(np_of(dx), wx), rel_fro(np_of(dv), wv)
    print(f"  dx rel {ex:.3e}, dv rel {ev:.3e}", flush=True)
    assert dx.dtype == BF and ex <= TOL
    assert ev <= TOL
    # the generic kernels on the same values (fp32 V takes them): same gradients within bf16
    (gx, gv), gnames = _names(lambda: ext.tril_rope_score_v_bwd(xd, vd.float(), dd, fd, start))
    assert "k_dq_sy" not in gnames
    assert rel_fro(np_of(dx), np_of(gx)) <= TOL
    assert rel_fro(np_of(dv), np_of(gv)) <= TOL


def test_rope_backward_mfma_route_fp32_dv_output():
    """dV can be written in fp32 (the autograd function keeps V's dtype)."""
    B, H, T, N, D = 2, 2, 300, 256, 64
    x = O.bf16_round(latent((B, H, T, N), 3))
    v = O.bf16_round(normal((B, 1, T, D), 4))
    dO = O.bf16_round(normal((B, H, T, D), 5))
    f = O.get_freqs(N)
    dv32 = torch.empty(B, 1, T, D, device=DEV, dtype=torch.float32)
    dx, dv = ext.tril_rope_score_v_bwd(to_dev(x, BF), to_dev(v, BF), to_dev(dO, BF), torch.from_numpy(f).to(DEV),
                                       7, dv=dv32)
    assert dv is dv32
    wx, wv = O.tril_rope_score_v_backward(x, v, dO, f, 7)
    assert rel_fro(np_of(dx), wx) <= TOL and rel_fro(np_of(dv), wv) <= TOL


def test_rope_autograd_with_fp32_v_takes_the_mfma_route():
    """bdh_attn_rope under autograd with bf16 x and fp32 V (V is the LayerNorm
    output under autocast): gradients in each input's dtype, V entering the
    products as bf16 (as the forward and the reference's autocast matmul use
    it), against the oracle at 2e-2."""
    B, H, T, N, D, start = 2, 4, 333, 512, 256, 2
    x = O.bf16_round(latent((B, H, T, N), 6))
    v = normal((B, 1, T, D), 7)
    dO = O.bf16_round(normal((B, H, T, D), 8))
    f = O.get_freqs(N)
    xd = to_dev(x, BF).requires_grad_(True)
    vd = to_dev(v, torch.float32).requires_grad_(True)

    def run():
        out = kernels.bdh_attn_rope(xd, vd, torch.from_numpy(f).to(DEV), start, impl="hip")
        out.backward(to_dev(dO, BF))
        return out

    out, names = _names(run)
    assert "k_dq_sy" in names, names
    assert xd.grad.dtype == BF and vd.grad.dtype == torch.float32
    wx, wv = O.tril_rope_score_v_backward(x, O.bf16_round(v), dO, f, start)
    assert rel_fro(np_of(xd.grad), wx) <= TOL
    assert rel_fro(np_of(vd.grad), wv) <= TOL


def test_rope_backward_c2_width_batch0():
    """C2 attention width (nh=4, T=512, N=8192, D=256) on two sequences:
    sequence 0 against the oracle; doubling dO doubles both gradients exactly."""
    B, H, T, N, D = 2, 4, 512, 8192, 256
    g = torch.Generator(device=DEV).manual_seed(9)
    xd = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    vd = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    dd = torch.randn(B, H, T, D, generator=g, device=DEV).to(BF)
    fd = kernels.get_freqs(N).to(DEV)
    dx, dv = ext.tril_rope_score_v_bwd(xd, vd, dd, fd, 0)
    dx2, dv2 = ext.tril_rope_score_v_bwd(xd, vd, dd * 2, fd, 0)
    assert torch.equal(dx2, dx * 2) and torch.equal(dv2, dv * 2)
    wx, wv = O.tril_rope_score_v_backward(np_of(xd[:1]), np_of(vd[:1]), np_of(dd[:1]), np_of(fd), 0)
    ex, ev = rel_fro(np_of(dx[:1]), wx), rel_fro(np_of(dv[:1]), wv)
    print(f"C2 width batch 0: dx rel {ex:.3e}, dv rel {ev:.3e}", flush=True)
    assert ex <= TOL and ev <= TOL


@pytest.mark.parametrize("shape", SHAPES)
def test_rope_backward_from_saved_tiles(shape):
    """The forward keeps its score tiles (relative layout) and the backward
    recomputes none: dV from the kept tiles, dx with x rotated as the dQ
    kernel stages it.  dx equals the recompute route's bit for bit (the same
    R(x) bits and G); dV is within the bf16 tolerance of it and of the oracle
    (the kept tiles rotate about the tile centres, the recomputed ones by
    absolute positions)."""
    B, H, T, N, D, Hv, start = shape
    print(f"rope bwd saved tiles {shape}", flush=True)
    x = O.bf16_round(latent((B, H, T, N), 10))
    v = O.bf16_round(normal((B, Hv, T, D), 11))
    dO = O.bf16_round(normal((B, H, T, D), 12))
    f = O.get_freqs(N)
    xd, vd, dd = to_dev(x, BF), to_dev(v, BF), to_dev(dO, BF)
    fd = torch.from_numpy(f).to(DEV)
    out, scores = ext.tril_rope_score_v_save(xd, vd, fd, start)
    assert scores is not None
    assert torch.equal(out, ext.tril_rope_score_v(xd, vd, fd, start))
    (sx, sv), names = _names(lambda: ext.tril_rope_score_v_bwd_saved(xd, vd, dd, fd, start, scores))
    assert "k_dq_sy" in names and names & {"k_dv_sy", "k_dv_dma"}, names
    assert "k_rope_table" not in names, names
    assert not any(n.startswith("k_sy_scores") and n != "k_sy_scores_g" for n in names), names
    rx, rv = ext.tril_rope_score_v_bwd(xd, vd, dd, fd, start)
    assert torch.equal(sx, rx)
    assert rel_fro(np_of(sv), np_of(rv)) <= TOL
    wx, wv = O.tril_rope_score_v_backward(x, v, dO, f, start)
    ex, ev = rel_fro(np_of(sx), wx), rel_fro(np_of(sv), wv)
    print(f"  dx rel {ex:.3e}, dv rel {ev:.3e}", flush=True)
    assert ex <= TOL and ev <= TOL


def test_rope_autograd_saved_tiles_switch(monkeypatch):
    """bdh_attn_rope under autograd keeps the forward's tiles by default and
    recomputes them with BDH_ATTN_SAVE_SCORES=0: same dx bits, dV within the
    bf16 tolerance."""
    B, H, T, N, D, start = 2, 4, 300, 512, 128, 4
    x = O.bf16_round(latent((B, H, T, N), 13))
    v = normal((B, 1, T, D), 14)
    dO = O.bf16_round(normal((B, H, T, D), 15))
    fd = torch.from_numpy(O.get_freqs(N)).to(DEV)
    grads = {}
    for save in ("1", "0"):
        monkeypatch.setenv("BDH_ATTN_SAVE_SCORES", save)
        xd = to_dev(x, BF).requires_grad_(True)
        vd = to_dev(v, torch.float32).requires_grad_(True)

        def run():
            out = kernels.bdh_attn_rope(xd, vd, fd, start, impl="hip")
            out.backward(to_dev(dO, BF))
            return out

        _, names = _names(run)
        assert ("k_rope_table" in names) == (save == "0"), names
        grads[save] = (xd.grad.clone(), vd.grad.clone())
    assert torch.equal(grads["1"][0], grads["0"][0])
    assert rel_fro(np_of(grads["1"][1]), np_of(grads["0"][1])) <= TOL


def test_rope_backward_from_saved_tiles_absolute_layout():
    """More than 512 k stages per workgroup (N = 16640, one split because 129 slabs
    of one 256-row tile fill the chip) keeps the forward's tiles in the absolute
    layout, with the (cos, sin) table ahead of them.  dx equals the recompute
    route's bit for bit; batch element 0 matches the oracle at 2e-2."""
    B, H, T, N, D, start = 43, 3, 256, 16640, 64, 9
    print(f"rope bwd saved tiles, absolute layout {(B, H, T, N, D)}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    xd = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    vd = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    dd = torch.randn(B, H, T, D, generator=g, device=DEV).to(BF)
    fd = kernels.get_freqs(N).to(DEV)
    assert ext.rope_keeps_scores(xd, vd)
    out, scores = ext.tril_rope_score_v_save(xd, vd, fd, start)
    assert scores is not None
    assert torch.equal(out, ext.tril_rope_score_v(xd, vd, fd, start))
    (sx, sv), names = _names(lambda: ext.tril_rope_score_v_bwd_saved(xd, vd, dd, fd, start, scores))
    assert "k_dq_sy" in names and names & {"k_dv_sy", "k_dv_dma"}, names
    rx, rv = ext.tril_rope_score_v_bwd(xd, vd, dd, fd, start)
    assert torch.equal(sx, rx)
    assert rel_fro(np_of(sv), np_of(rv)) <= TOL
    wx, wv = O.tril_rope_score_v_backward(np_of(xd[:1]), np_of(vd[:1]), np_of(dd[:1]), np_of(fd), start)
    ex, ev = rel_fro(np_of(sx[:1]), wx), rel_fro(np_of(sv[:1]), wv)
    print(f"  dx rel {ex:.3e}, dv rel {ev:.3e}", flush=True)
    assert ex <= TOL and ev <= TOL
