"""GPU parity of the HIP kernels against the CPU oracle, through the C-ABI library.

Tolerances (relative Frobenius): fp32 <= 1e-4, bf16 <= 2e-2; integer / mask /
position behaviour exact (known answers, row 0 == 0 exactly).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, as_dtype_values, latent, normal, np_of, rel_fro, to_dev

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # collected on CPU hosts, run only on the GPU box
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)

KA = json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())
DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]


def _f32(x):
    return torch.tensor(x, dtype=torch.float32, device=DEV)


# ------------------------------------------------------------- known answers
def test_known_answers_cold_and_decode():
    k = KA["raw_tril_fwd_bwd"]
    out = ext.tril_score_v(_f32(k["q"]), _f32(k["k"]), _f32(k["v"]))
    assert torch.equal(out.cpu(), torch.tensor(k["out"]))
    k = KA["self_attn_single_query"]
    q = _f32(k["q"])
    assert torch.equal(ext.tril_score_v(q, q, _f32(k["v"])).cpu(), torch.tensor(k["out"]))
    k = KA["bench_cold"]
    assert torch.equal(ext.tril_score_v(_f32(k["q"]), _f32(k["k"]), _f32(k["v"])).cpu(), torch.tensor(k["out"]))
    for name in ("decode_raw", "bench_decode"):
        k = KA[name]
        got = ext.tril_decode(_f32(k["q"]), _f32(k["k_past"]), _f32(k["v_past"]))
        assert torch.equal(got.cpu(), torch.tensor(k["out"])), name


def test_known_answers_backward():
    k = KA["raw_tril_fwd_bwd"]
    dq, dk, dv = ext.tril_score_v_bwd(_f32(k["q"]), _f32(k["k"]), _f32(k["v"]), _f32(k["dout"]))
    assert torch.equal(dq.cpu(), torch.tensor(k["dq"]))
    assert torch.equal(dk.cpu(), torch.tensor(k["dk"]))
    assert torch.equal(dv.cpu(), torch.tensor(k["dv"]))
    k = KA["self_attn_single_query"]
    dqm, none, dv = ext.tril_score_v_bwd(_f32(k["q"]), None, _f32(k["v"]), _f32(k["dout"]))
    assert none is None
    assert torch.equal(dqm.cpu(), torch.tensor(k["dq_merged"]))
    assert torch.equal(dv.cpu(), torch.tensor(k["dv"]))


# ------------------------------------------------------------ cold forward
COLD_SHAPES = [
    # B, H, T, N, D, Hv
    (1, 1, 1, 8, 4, 1),
    (1, 2, 2, 2, 1, 1),
    (2, 3, 37, 6, 5, 3),
    (1, 2, 128, 64, 32, 1),
    (2, 2, 129, 72, 40, 1),
    (1, 1, 300, 200, 130, 1),
    (1, 2, 257, 1024, 256, 2),
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", COLD_SHAPES)
def test_cold_forward_matches_oracle(shape, dtype):
    B, H, T, N, D, Hv = shape
    q = as_dtype_values(latent((B, H, T, N), 0), dtype)
    k = as_dtype_values(latent((B, H, T, N), 7), dtype)
    v = as_dtype_values(normal((B, Hv, T, D), 1), dtype)
    want = O.tril_score_v_cpu(q, k, v)
    got = ext.tril_score_v(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype))
    assert got.dtype == dtype and got.shape == (B, H, T, D)
    g = np_of(got)
    assert rel_fro(g, want) <= TOL[dtype]
    assert not g[:, :, 0].any()  # position 0 attends to nothing: exactly zero
    # self attention (q is k) takes the shared-operand diagonal path
    got_s = np_of(ext.tril_score_v(to_dev(q, dtype), to_dev(q, dtype), to_dev(v, dtype)))
    assert rel_fro(got_s, O.tril_score_v_cpu(q, q, v)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DTYPES)
def test_cold_forward_strided_views_and_mixed_v(dtype):
    """Permuted (B,T,H,N) latent views and fp32 V with bf16 Q work without copies."""
    B, T, H, N, D = 2, 150, 3, 96, 48
    x_bthn = as_dtype_values(latent((B, T, H, N), 3), dtype)
    xt = to_dev(x_bthn, dtype).permute(0, 2, 1, 3)  # (B,H,T,N) view, stride (T*H*N, N, H*N, 1)
    v = normal((B, 1, T, D), 4)
    vt = to_dev(v, torch.float32)
    got = np_of(ext.tril_score_v(xt, xt, vt))
    want = O.tril_score_v_cpu(x_bthn.transpose(0, 2, 1, 3), x_bthn.transpose(0, 2, 1, 3),
                              as_dtype_values(v, dtype))
    assert rel_fro(got, want) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,start", [((2, 2, 40, 16, 8), 0), ((1, 3, 200, 130, 64), 5), ((1, 2, 513, 512, 256), 0)])
def test_fused_rope_forward_matches_oracle(shape, start, dtype):
    B, H, T, N, D = shape
    x = as_dtype_values(latent((B, H, T, N), 0), dtype)
    v = as_dtype_values(normal((B, 1, T, D), 1), dtype)
    freqs = O.get_freqs(N)
    want, qr_want = O.tril_rope_score_v(x, v, freqs, start, bf16=(dtype == torch.bfloat16))
    qr = torch.empty(B, H, T, N, dtype=dtype, device=DEV)
    got = ext.tril_rope_score_v(to_dev(x, dtype), to_dev(v, dtype), torch.from_numpy(freqs).to(DEV), start, qr_out=qr)
    g = np_of(got)
    assert rel_fro(g, want) <= TOL[dtype]
    assert not g[:, :, 0].any()
    assert rel_fro(np_of(qr), qr_want) <= (1e-5 if dtype == torch.float32 else 8e-3)


def test_fused_rope_forward_c1_shape_bf16():
    """The headline shape (B=8 nh=4 T=512 N=8192 D=256) on a 2-batch sample."""
    B, H, T, N, D = 2, 4, 512, 8192, 256
    x = O.bf16_round(latent((B, H, T, N), 0))
    v = O.bf16_round(normal((B, 1, T, D), 1))
    freqs = O.get_freqs(N)
    want, _ = O.tril_rope_score_v(x, v, freqs, 0, bf16=True)
    got = ext.tril_rope_score_v(to_dev(x, torch.bfloat16), to_dev(v, torch.bfloat16), torch.from_numpy(freqs).to(DEV))
    assert rel_fro(np_of(got), want) <= 2e-2


# ------------------------------------------------------------------ decode
@pytest.mark.parametrize("qdt,cdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("S,Tq,N,D,Hv", [(0, 1, 8, 4, 1), (1, 1, 16, 8, 1), (45, 1, 64, 32, 1),
                                         (70, 2, 200, 24, 3), (300, 1, 8192, 256, 1)])
def test_decode_matches_oracle_on_capacity_strided_cache(S, Tq, N, D, Hv, qdt, cdt):
    B, H, cap = 2, 3, S + 7
    kbuf = as_dtype_values(latent((B, H, cap, N), 2), cdt)
    vbuf = as_dtype_values(normal((B, Hv, cap, D), 3), cdt)
    q = as_dtype_values(latent((B, H, Tq, N), 4), qdt)
    kt, vt = to_dev(kbuf, cdt), to_dev(vbuf, cdt)
    got = np_of(ext.tril_decode(to_dev(q, qdt), kt.narrow(2, 0, S), vt.narrow(2, 0, S)))
    want = O.tril_decode_cpu(q, kbuf[:, :, :S], vbuf[:, :, :S])
    tol = TOL[torch.bfloat16] if torch.bfloat16 in (qdt, cdt) else TOL[torch.float32]
    assert rel_fro(got, want) <= tol
    if S == 0:
        assert not got.any()


def test_decode_full_c3_size_properties():
    """C3 at full size (B=64 nh=4 N=8192 D=256, bf16 cache of capacity 512, S=511):
    the decode of the query at position S over the cache equals row S of the cold
    op over the same S+1 rows (the definition of a decode step), within bf16
    tolerance; doubling V doubles the output exactly; batch element 0 against
    the oracle."""
    B, H, N, D, S, cap = 64, 4, 8192, 256, 511, 512
    g = torch.Generator(device=DEV).manual_seed(3)
    kc = torch.relu(0.32 * torch.randn(B, H, cap, N, generator=g, device=DEV)).to(torch.bfloat16)
    vc = torch.randn(B, 1, cap, D, generator=g, device=DEV).to(torch.bfloat16)
    q = kc[:, :, S:S + 1]
    got = ext.tril_decode(q, kc.narrow(2, 0, S), vc.narrow(2, 0, S))
    cold_row = ext.tril_score_v_past(q, kc, vc, S)  # queries at offset S over the S+1 rows
    assert rel_fro(np_of(got), np_of(cold_row)) <= TOL[torch.bfloat16]
    got2 = ext.tril_decode(q, kc.narrow(2, 0, S), (vc * 2).narrow(2, 0, S))
    assert torch.equal(got2, got * 2)
    want = O.tril_decode_cpu(np_of(q[:1]), np_of(kc[:1, :, :S]), np_of(vc[:1, :, :S]))
    assert rel_fro(np_of(got[:1]), want) <= TOL[torch.bfloat16]


# -------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("vdt,odt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("backward", [False, True])
def test_rope_apply_is_bit_exact(vdt, odt, backward):
    """Same cos/sin tables in, same bits out (fp32 and bf16 rounding orders)."""
    B, H, T, N = 2, 3, 33, 64
    x = as_dtype_values(normal((B, H, T, N), 5), vdt)
    c, s = O.rope_cos_sin(T, 11, O.get_freqs(N))
    fn = O.rope_rotate_backward if backward else O.rope_rotate
    want = fn(x, c, s, bf16=(vdt == torch.bfloat16))
    want = as_dtype_values(want, odt)
    out = torch.empty(B, H, T, N, dtype=odt, device=DEV)
    got = ext.rope_rotate(to_dev(x, vdt), torch.from_numpy(c).to(DEV).view(1, 1, T, N),
                          torch.from_numpy(s).to(DEV).view(1, 1, T, N), out, backward=backward)
    assert got is out
    assert np.array_equal(np_of(got), want)


@pytest.mark.parametrize("layout", ["per_head_tables", "narrow_rows", "permuted_view"])
@pytest.mark.parametrize("vdt", [torch.float32, torch.bfloat16])
def test_rope_apply_paths_are_bit_exact(layout, vdt):
    """Each kernel variant against the oracle's rounding: tables that vary per
    (b, h) (8-wide path without the broadcast), N not a multiple of 8 (scalar
    path) and the permuted x_sparse view with broadcast tables."""
    B, H, T = 2, 3, 17
    N = 12 if layout == "narrow_rows" else 64
    c, s = O.rope_cos_sin(T, 5, O.get_freqs(N))
    if layout == "per_head_tables":
        scale = (1.0 + 0.01 * np.arange(B * H, dtype=np.float32)).reshape(B, H, 1, 1)
        c4, s4 = (c.reshape(1, 1, T, N) * scale).astype(np.float32), (s.reshape(1, 1, T, N) * scale).astype(np.float32)
    else:
        c4, s4 = np.broadcast_to(c.reshape(1, 1, T, N), (B, H, T, N)), np.broadcast_to(s.reshape(1, 1, T, N), (B, H, T, N))
    x = as_dtype_values(normal((B, T, H, N) if layout == "permuted_view" else (B, H, T, N), 8), vdt)
    xv = np.ascontiguousarray(x.transpose(0, 2, 1, 3)) if layout == "permuted_view" else x
    want = O.rope_rotate(xv, c4, s4, bf16=(vdt == torch.bfloat16))
    xd = to_dev(x, vdt)
    xd = xd.permute(0, 2, 1, 3) if layout == "permuted_view" else xd
    if layout == "per_head_tables":
        cd, sd = torch.from_numpy(c4).to(DEV), torch.from_numpy(s4).to(DEV)
    else:
        cd = torch.from_numpy(c).to(DEV).view(1, 1, T, N).expand(B, H, T, N)
        sd = torch.from_numpy(s).to(DEV).view(1, 1, T, N).expand(B, H, T, N)
    got = ext.rope_rotate(xd, cd, sd)
    assert np.array_equal(np_of(got), as_dtype_values(want, vdt))


@pytest.mark.parametrize("permuted", [False, True])
@pytest.mark.parametrize("backward", [False, True])
@pytest.mark.parametrize("vdt", [torch.float32, torch.bfloat16])
def test_rope_apply_broadcast_kernel_is_bit_exact(vdt, backward, permuted):
    """The broadcast-table kernel (many time steps, tables shared by every
    (b, h) row): B*H = 40 rows (two full runs of 16 and one of 8), N = 2560
    (a last column block of 512), T = 256, contiguous and as the permuted
    x_sparse view."""
    B, H, T, N = 5, 8, 256, 2560
    c, s = O.rope_cos_sin(T, 3, O.get_freqs(N))
    x = as_dtype_values(normal((B, T, H, N) if permuted else (B, H, T, N), 9), vdt)
    xv = np.ascontiguousarray(x.transpose(0, 2, 1, 3)) if permuted else x
    fn = O.rope_rotate_backward if backward else O.rope_rotate
    want = fn(xv, c.reshape(1, 1, T, N), s.reshape(1, 1, T, N), bf16=(vdt == torch.bfloat16))
    xd = to_dev(x, vdt)
    xd = xd.permute(0, 2, 1, 3) if permuted else xd
    cd = torch.from_numpy(c).to(DEV).view(1, 1, T, N).expand(B, H, T, N)
    sd = torch.from_numpy(s).to(DEV).view(1, 1, T, N).expand(B, H, T, N)
    got = ext.rope_rotate(xd, cd, sd, backward=backward)
    assert np.array_equal(np_of(got), as_dtype_values(want, vdt))


# ---------------------------------------------------------------- backward
BWD_SHAPES = [(1, 1, 5, 4, 3, 1), (2, 3, 70, 24, 16, 1), (1, 2, 200, 136, 72, 2), (1, 2, 300, 512, 256, 1)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BWD_SHAPES)
def test_backward_matches_oracle(shape, dtype):
    B, H, T, N, D, Hv = shape
    q = as_dtype_values(latent((B, H, T, N), 0), dtype)
    k = as_dtype_values(latent((B, H, T, N), 9), dtype)
    v = as_dtype_values(normal((B, Hv, T, D), 1), dtype)
    dO = as_dtype_values(normal((B, H, T, D), 2), dtype)
    tol = TOL[dtype]
    dq, dk, dv = ext.tril_score_v_bwd(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), to_dev(dO, dtype))
    wq, wk, wv = O.analytic_tril_attn_backward_blocked(q, k, v, dO)
    assert rel_fro(np_of(dq), wq) <= tol
    assert rel_fro(np_of(dk), wk) <= tol
    assert rel_fro(np_of(dv), wv) <= tol
    dqm, _, dv2 = ext.tril_score_v_bwd(to_dev(q, dtype), None, to_dev(v, dtype), to_dev(dO, dtype))
    wqm, wv2 = O.self_attn_backward(q, v, dO)
    assert rel_fro(np_of(dqm), wqm) <= tol
    assert rel_fro(np_of(dv2), wv2) <= tol


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,start", [((1, 2, 60, 32, 16), 0), ((2, 2, 260, 256, 64), 3)])
def test_fused_rope_backward_matches_oracle(shape, start, dtype):
    B, H, T, N, D = shape
    x = as_dtype_values(latent((B, H, T, N), 0), dtype)
    v = as_dtype_values(normal((B, 1, T, D), 1), dtype)
    dO = as_dtype_values(normal((B, H, T, D), 2), dtype)
    f = O.get_freqs(N)
    dx, dv = ext.tril_rope_score_v_bwd(to_dev(x, dtype), to_dev(v, dtype), to_dev(dO, dtype),
                                       torch.from_numpy(f).to(DEV), start)
    wx, wv = O.tril_rope_score_v_backward(x, v, dO, f, start)
    assert rel_fro(np_of(dx), wx) <= TOL[dtype]
    assert rel_fro(np_of(dv), wv) <= TOL[dtype]


def test_errors_surface_as_runtime_errors():
    q = torch.zeros(1, 1, 4, 8, device=DEV)
    with pytest.raises(RuntimeError):
        ext.tril_score_v(q, q, torch.zeros(1, 2, 4, 3, device=DEV))  # v heads not in {1, H}
    with pytest.raises(RuntimeError):
        ext.tril_score_v(q.cpu(), q.cpu(), q.cpu())  # no CPU path in the HIP library
