"""GPU parity of the bf16 self-attention backward on the MFMA dQ path
(dQ = G X with transposing LDS reads of X) against the CPU oracle.

Shapes qualify for that path (bf16, N a multiple of 256, no RoPE): ragged T
(1, 31, 130, 257, 520, 600), several N tiles, per-head V, the permuted x_sparse
view and an fp32 output; with D a multiple of 64, G = dS + dS^T comes from the
MFMA score kernel as well.  Tolerance: bf16 2e-2 relative Frobenius.  At the C4 shape
(B=16 nh=4 T=1024 N=8192 D=256): exact homogeneity in dO and one slab against
the oracle.
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

DEV = "cuda"
BF = torch.bfloat16

SHAPES = [
    # B, H, T, N, D, Hv
    (1, 1, 1, 256, 16, 1),
    (2, 2, 31, 512, 24, 1),
    (1, 2, 257, 256, 64, 2),
    (1, 1, 520, 768, 32, 1),
    # D a multiple of 64: G on the MFMA score kernel too (one 256-tile past tpad
    # at T = 600, a single row at T = 1, D below 256)
    (1, 2, 600, 256, 128, 2),
    (2, 1, 1, 256, 64, 1),
    (1, 1, 130, 512, 192, 1),
]


@pytest.mark.parametrize("shape", SHAPES)
def test_self_backward_bf16_matches_oracle(shape):
    B, H, T, N, D, Hv = shape
    q = O.bf16_round(latent((B, H, T, N), 0))
    v = O.bf16_round(normal((B, Hv, T, D), 1))
    dO = O.bf16_round(normal((B, H, T, D), 2))
    dq, _, dv = ext.tril_score_v_bwd(to_dev(q, BF), None, to_dev(v, BF), to_dev(dO, BF))
    wq, wv = O.self_attn_backward(q, v, dO)
    print(f"bwd {shape}: dq {rel_fro(np_of(dq), wq):.3e} dv {rel_fro(np_of(dv), wv):.3e}", flush=True)
    assert rel_fro(np_of(dq), wq) <= TOL[BF]
    assert rel_fro(np_of(dv), wv) <= TOL[BF]


def test_self_backward_permuted_view_fp32_out():
    """x_sparse as bdh.py makes it, (B,T,nh,N) viewed as (B,nh,T,N); fp32 grads."""
    B, T, H, N, D = 2, 70, 2, 512, 40
    x = O.bf16_round(latent((B, T, H, N), 3))
    v = O.bf16_round(normal((B, 1, T, D), 4))
    dO = O.bf16_round(normal((B, H, T, D), 5))
    xd = to_dev(x, BF).permute(0, 2, 1, 3)
    dq = torch.empty(B, H, T, N, dtype=torch.float32, device=DEV)
    dv = torch.empty(B, 1, T, D, dtype=torch.float32, device=DEV)
    ext.tril_score_v_bwd(xd, None, to_dev(v, BF), to_dev(dO, BF), dq=dq, dv=dv)
    xq = np.ascontiguousarray(x.transpose(0, 2, 1, 3))
    wq, wv = O.self_attn_backward(xq, v, dO)
    assert rel_fro(np_of(dq), wq) <= TOL[BF]
    assert rel_fro(np_of(dv), wv) <= TOL[BF]


def test_self_backward_c4_properties():
    """C4 at full size: dQ and dV are linear in dO, and doubling is exact in
    bf16 and fp32, so the bits must match; batch element 0 (all four heads:
    dV sums over them) against the oracle for both dQ and dV."""
    B, H, T, N, D = 16, 4, 1024, 8192, 256
    g = torch.Generator(device=DEV).manual_seed(0)
    q = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    v = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    d = torch.randn(B, H, T, D, generator=g, device=DEV).to(BF)
    dq1, _, dv1 = ext.tril_score_v_bwd(q, None, v, d)
    dq2, _, dv2 = ext.tril_score_v_bwd(q, None, v, d * 2)
    assert torch.equal(dq2, dq1 * 2)
    assert torch.equal(dv2, dv1 * 2)
    assert torch.isfinite(dq1).all().item()
    # batch element 0 depends only on q[0], v[0], dO[0]
    wq, wv = O.self_attn_backward(np_of(q[:1]), np_of(v[:1]), np_of(d[:1]))
    eq, ev = rel_fro(np_of(dq1[:1]), wq), rel_fro(np_of(dv1[:1]), wv)
    print(f"C4 batch 0: dQ rel {eq:.3e}, dV rel {ev:.3e}", flush=True)
    assert eq <= TOL[BF] and ev <= TOL[BF]


@pytest.mark.parametrize("shape", SHAPES)
def test_saved_scores_backward_is_bit_exact(shape):
    """The forward keeps its score tiles; the backward from them equals the
    recompute path bit for bit (same kernel, same inputs) and the oracle."""
    B, H, T, N, D, Hv = shape
    q = to_dev(O.bf16_round(latent((B, H, T, N), 7)), BF)
    v = to_dev(O.bf16_round(normal((B, Hv, T, D), 8)), BF)
    d = to_dev(O.bf16_round(normal((B, H, T, D), 9)), BF)
    assert ext.keeps_scores(q, v)
    out, scores = ext.tril_score_v_save(q, v)
    assert scores is not None
    assert torch.equal(out, ext.tril_score_v(q, q, v))
    dq_s, dv_s = ext.tril_score_v_bwd_saved(q, v, d, scores)
    dq_r, _, dv_r = ext.tril_score_v_bwd(q, None, v, d)
    assert torch.equal(dq_s, dq_r)
    assert torch.equal(dv_s, dv_r)
    wq, wv = O.self_attn_backward(np_of(q), np_of(v), np_of(d))
    assert rel_fro(np_of(dq_s), wq) <= TOL[BF]
    assert rel_fro(np_of(dv_s), wv) <= TOL[BF]


def test_saved_scores_autograd_and_refusals(monkeypatch):
    """strict_tril_attn(x, x, v, impl="hip") saves the tiles; gradients equal
    those of the recompute path.  fp32 keeps no tiles; a different x is refused."""
    import kernels as K

    B, H, T, N, D = 2, 2, 300, 512, 64
    x0 = to_dev(O.bf16_round(latent((B, H, T, N), 11)), BF)
    v0 = to_dev(O.bf16_round(normal((B, 1, T, D), 12)), BF)
    g = to_dev(O.bf16_round(normal((B, H, T, D), 13)), BF)

    def grads(save: str):
        monkeypatch.setenv("BDH_ATTN_SAVE_SCORES", save)
        x = x0.clone().requires_grad_(True)
        v = v0.clone().requires_grad_(True)
        K.strict_tril_attn(x, x, v, impl="hip", use_fn=True).backward(g)
        return x.grad, v.grad

    gx1, gv1 = grads("1")
    gx0, gv0 = grads("0")
    assert torch.equal(gx1, gx0)
    assert torch.equal(gv1, gv0)
    assert not ext.keeps_scores(x0.float(), v0.float())
    _, scores = ext.tril_score_v_save(x0, v0)
    with pytest.raises(RuntimeError):  # narrower x: the saved tiles do not belong to it
        ext.tril_score_v_bwd_saved(x0[..., :64].contiguous().float(), v0, g, scores)
