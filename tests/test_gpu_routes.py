"""GPU parity of the routes the unchanged reference callers take, and of the
BASELINE configurations at their full width.

* T=1 decode RoPE: ``bdh_rope_rotate_paired(..., out=slot, impl="hip")`` with
  the paired (..., N/2, 2) table narrowed at the decode position and the
  capacity-strided KR cache slot as ``out`` (reference bdh.py:396-405,
  kernels/rope.py:174-190), bit for bit against the eager rotation and the
  oracle.
* The unfused training route of bdh.py:405-412: ``bdh_rope_rotate(x, cos, sin,
  impl="hip")`` (HipRopeFn) -> ``bdh_attn(QR, QR, V, impl="hip")``
  (StrictTrilSelfAttnFn, score tiles kept or recomputed) -> ``backward``,
  against the oracle's fused-RoPE gradients (fp32 1e-4, bf16 2e-2) and the
  same route on torch eager autograd (on the CPU: bf16 batched products on
  transposed views have faulted ROCm GPUs).
* C1 in fp32 at full width (B=8 nh=4 T=512 N=8192 D=256): batch element 0
  against the oracle at 1e-4; exact homogeneity over all 8.
* C5 attention width (B=4 nh=8 T=2048 N=8192 D=512, V wider than 256): batch
  element 0 against the oracle at 2e-2; exact homogeneity over all 4.
* The C5 model configuration (L=8 D=512 nh=8 N=8192, T=2048) against the
  numpy model oracle at 2e-2 on one sequence.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, latent, normal, np_of, rel_fro, to_dev
from oracle import bdh_model_oracle as M

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)
import kernels  # noqa: E402
from kernels import rope as R  # noqa: E402

DEV = "cuda"
BF = torch.bfloat16


# ------------------------------------------------------------ T=1 paired RoPE
@pytest.mark.parametrize("vdt", [torch.float32, BF])
@pytest.mark.parametrize("pos", [0, 37, 255])
def test_paired_t1_rope_into_cache_slot_is_bit_exact(vdt, pos):
    """bdh.py:396-405 at a decode step: paired cis narrowed from the generate
    table at ``pos`` (bdh.py:157-191, 301-345), v (B, nh, 1, N), out the KR
    cache slot ``kr_buf.narrow(2, pos, 1)`` (bdh_cache.py:258-277)."""
    print(f"paired t1 rope vdt={vdt} pos={pos}", flush=True)
    B, nh, N, cap = 3, 4, 1024, 256
    f = kernels.get_freqs(N)
    cos, sin = kernels.rope_cos_sin(cap, 0, f)  # (1, 1, cap, N) fp32 generate table
    cp = cos.reshape(*cos.shape[:-1], -1, 2).narrow(-3, pos, 1)
    sp = sin.reshape(*sin.shape[:-1], -1, 2).narrow(-3, pos, 1)
    v = torch.from_numpy(latent((B, nh, 1, N), 7)).to(vdt)
    kr = torch.zeros(B, nh, cap, N, dtype=vdt, device=DEV)
    slot = kr.narrow(2, pos, 1)
    got = kernels.bdh_rope_rotate_paired(v.to(DEV), cp.to(DEV), sp.to(DEV), out=slot, impl="hip")
    assert got is slot
    want = R.rope_rotate_paired(v, cp, sp)  # eager, on the CPU
    assert torch.equal(slot.cpu(), want)
    ora = O.rope_rotate(v.float().numpy(), cos[..., pos:pos + 1, :].numpy(), sin[..., pos:pos + 1, :].numpy(),
                        bf16=vdt == BF)
    assert np.array_equal(slot.float().cpu().numpy(), ora)
    # nothing outside the slot was written
    assert not kr[:, :, :pos].any().item() and not kr[:, :, pos + 1:].any().item()


# ------------------------------------------------- unfused training route
def _eager_route_cpu(x, v, dO, start):
    """The same route on torch eager autograd, on the CPU."""
    xe = x.detach().cpu().clone().requires_grad_(True)
    ve = v.detach().cpu().clone().requires_grad_(True)
    f = kernels.get_freqs(x.size(-1))
    cos, sin = kernels.rope_cos_sin(x.size(2), start, f)
    qr = R.eager_rope_rotate(xe, cos, sin)
    out = kernels.bdh_attn(qr, qr, ve, impl="eager")
    out.backward(dO.detach().cpu())
    return out.detach().float().numpy(), xe.grad.float().numpy(), ve.grad.float().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, BF])
@pytest.mark.parametrize("save", ["1", "0"])
@pytest.mark.parametrize("start", [0, 5])
def test_unfused_training_route_matches_oracle_and_eager(dtype, save, start, monkeypatch):
    """bdh.py:405-412 with BDH_ROPE_IMPL=hip and BDH_ATTN_IMPL=hip: HipRopeFn,
    then bdh_attn(QR, QR, V) through StrictTrilSelfAttnFn (hip kernels for the
    forward and the merged-gradient backward), then the RoPE backward."""
    monkeypatch.setenv("BDH_ATTN_SAVE_SCORES", save)
    print(f"unfused training route dtype={dtype} save={save} start={start}", flush=True)
    B, nh, T, N, D = 2, 2, 300, 512, 64
    x = latent((B, nh, T, N), 41)
    v = normal((B, 1, T, D), 42)
    dO = normal((B, nh, T, D), 43)
    if dtype == BF:
        x, v, dO = O.bf16_round(x), O.bf16_round(v), O.bf16_round(dO)
    xd = to_dev(x, dtype).requires_grad_(True)
    vd = to_dev(v, dtype).requires_grad_(True)
    dOd = to_dev(dO, dtype)
    f = kernels.get_freqs(N).to(DEV)
    cos, sin = kernels.rope_cos_sin(T, start, f)
    before = ext.launch_count()
    qr = kernels.bdh_rope_rotate(xd, cos, sin, impl="hip")
    out = kernels.bdh_attn(qr, qr, vd, impl="hip")
    out.backward(dOd)
    torch.cuda.synchronize()
    assert ext.launch_count() >= before + 4  # rope fwd, attention fwd, attention bwd, rope bwd
    fr = O.get_freqs(N)
    want, _ = O.tril_rope_score_v(x, v, fr, start, bf16=dtype == BF)
    wdx, wdv = O.tril_rope_score_v_backward(x, v, dO, fr, start)
    tol = TOL[dtype]
    errs = {"out": rel_fro(np_of(out), want), "dx": rel_fro(np_of(xd.grad), wdx), "dv": rel_fro(np_of(vd.grad), wdv)}
    e_out, e_dx, e_dv = _eager_route_cpu(xd, vd, dOd, start)
    errs_e = {"out": rel_fro(np_of(out), e_out), "dx": rel_fro(np_of(xd.grad), e_dx),
              "dv": rel_fro(np_of(vd.grad), e_dv)}
    print(f"  vs oracle {errs}  vs eager route {errs_e}", flush=True)
    assert all(e <= tol for e in errs.values()), errs
    assert all(e <= tol for e in errs_e.values()), errs_e
    assert xd.grad.dtype == dtype and vd.grad.dtype == dtype
    assert not out[:, :, 0].any().item()


# ------------------------------------------------------- C1 fp32, full width
def test_c1_fp32_full_width():
    """C1 as BASELINE states it (fp32): fused RoPE op at B=8 nh=4 T=512 N=8192
    D=256.  Batch element 0 against the oracle at 1e-4; scaling v by 2 and x by
    2 are exact in fp32, so out(x, 2v) = 2 out and out(2x, v) = 4 out bit for
    bit over the whole batch; row 0 exactly zero."""
    print("C1 fp32 full width", flush=True)
    B, H, T, N, D = 8, 4, 512, 8192, 256
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV))
    v = torch.randn(B, 1, T, D, generator=g, device=DEV)
    f = torch.from_numpy(O.get_freqs(N)).to(DEV)
    o1 = ext.tril_rope_score_v(x, v, f, 0)
    assert o1.dtype == torch.float32
    assert torch.equal(ext.tril_rope_score_v(x, v * 2, f, 0), o1 * 2)
    assert torch.equal(ext.tril_rope_score_v(x * 2, v, f, 0), o1 * 4)
    assert not o1[:, :, 0].any().item()
    want, _ = O.tril_rope_score_v(np_of(x[:1]), np_of(v[:1]), O.get_freqs(N), 0)
    err = rel_fro(np_of(o1[:1]), want)
    print(f"  batch 0 rel {err:.3e}", flush=True)
    assert err <= TOL[torch.float32]


# ------------------------------------------------------ C5 attention width
def test_c5_attention_width():
    """C5's attention (B=4 nh=8 T=2048 N=8192 D=512), bf16 fused RoPE: V is
    wider than 256, so score x V runs once per 256 columns.  Batch element 0
    against the oracle at 2e-2; exact homogeneity over the whole batch."""
    print("C5 attention width", flush=True)
    B, H, T, N, D = 4, 8, 2048, 8192, 512
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.relu(0.32 * torch.randn(B, H, T, N, generator=g, device=DEV)).to(BF)
    v = torch.randn(B, 1, T, D, generator=g, device=DEV).to(BF)
    f = torch.from_numpy(O.get_freqs(N)).to(DEV)

    def run(xx, vv):
        o = torch.empty(B, H, T, D, dtype=torch.float32, device=DEV)
        return ext.tril_rope_score_v(xx, vv, f, 0, out=o)

    o1 = run(x, v)
    assert torch.equal(run(x, v * 2), o1 * 2)
    assert torch.equal(run(x * 2, v), o1 * 4)
    assert not o1[:, :, 0].any().item()
    want, _ = O.tril_rope_score_v(np_of(x[:1]), np_of(v[:1]), O.get_freqs(N), 0, bf16=True)
    err = rel_fro(np_of(o1[:1]), want)
    print(f"  batch 0 rel {err:.3e}", flush=True)
    assert err <= TOL[BF]


def test_c5_model_config_matches_oracle():
    """The C5 model configuration in full (L=8, D=512, nh=8, N=8192, vocab 256)
    at T=2048 on one sequence, bf16 autocast, against the numpy model oracle
    (fp32): logits within 2e-2."""
    import bdh_harness as Hh

    print("C5 model config forward", flush=True)
    p = M.init_params(8, 512, 8, 8192, 256, seed=51)
    nh, D, N = p["encoder"].shape
    cfg = Hh.BDHConfig(n_layer=8, n_embd=D, n_head=nh, mlp_internal_dim_multiplier=128, vocab_size=256)
    m = Hh.BDH(cfg)
    with torch.no_grad():
        for k in ("encoder", "encoder_v", "decoder", "lm_head"):
            getattr(m, k).copy_(torch.from_numpy(p[k]))
        m.embed.weight.copy_(torch.from_numpy(p["embed"]))
    m = m.to(DEV)
    idx = np.random.default_rng(52).integers(0, 256, (1, 2048))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got, _ = m(torch.from_numpy(idx).to(DEV), impl="hip")
    got = got.float().cpu().numpy()
    del m
    torch.cuda.empty_cache()
    want = M.bdh_forward(p, idx)
    err = rel_fro(got, want)
    print(f"  logits rel {err:.3e}", flush=True)
    assert err <= 2e-2
