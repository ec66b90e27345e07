"""GPU parity of queries at an offset (chunked prefill) against the CPU oracle.

The op: T new query rows after ``past`` cached rows,
``out[b,h,i] = sum_{j < past+i} <q_i, k_j> v_j``, which the reference obtains by
recomputing the strict-tril attention over past||new and keeping the last T rows
(bdh.py:446-461).  Tolerances (relative Frobenius): fp32 <= 1e-4, bf16 <= 2e-2;
the causal boundary is checked bit-exactly on small-integer inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from helpers import TOL, as_dtype_values, latent, normal, np_of, rel_fro, to_dev

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # collected on CPU hosts, run only on the GPU box
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)
import kernels  # noqa: E402

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16]

PAST_SHAPES = [
    # B, H, T, past, N, D, Hv
    (1, 1, 1, 1, 8, 4, 1),      # one new row over one past row
    (1, 2, 5, 3, 16, 8, 1),     # inside one tile
    (2, 2, 40, 128, 64, 32, 2),  # past on a tile boundary
    (1, 3, 100, 37, 72, 40, 1),  # new rows straddle a tile boundary
    (1, 2, 1, 300, 96, 64, 1),   # T = 1: decode over the past
    (2, 1, 130, 200, 130, 130, 1),
    (1, 2, 257, 511, 512, 256, 2),
    (1, 1, 64, 0, 32, 16, 1),    # past = 0 is the cold op
]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", PAST_SHAPES)
def test_past_matches_oracle(shape, dtype):
    B, H, T, past, N, D, Hv = shape
    print(f"past shape={shape} dtype={dtype}", flush=True)
    k = as_dtype_values(latent((B, H, past + T, N), 11), dtype)
    q = as_dtype_values(latent((B, H, T, N), 12), dtype)
    v = as_dtype_values(normal((B, Hv, past + T, D), 13), dtype)
    want = O.tril_score_v_past(q, k, v, past)
    got = ext.tril_score_v_past(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), past)
    assert got.dtype == dtype and got.shape == (B, H, T, D)
    assert rel_fro(np_of(got), want) <= TOL[dtype]
    # the reference's own route: the new rows are the last T keys, full attention sliced
    k[:, :, past:] = q
    want = O.tril_score_v_cpu(k, k, v)[:, :, past:]
    got = ext.tril_score_v_past(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), past)
    assert rel_fro(np_of(got), want) <= TOL[dtype]


def test_past_causal_boundary_is_exact():
    """Small integers: every product and sum is exact in fp32, so any key taken
    or dropped at the boundary j = past + i - 1 shows as a mismatch."""
    rng = np.random.default_rng(3)
    for past, T in [(1, 3), (127, 2), (128, 1), (129, 130), (250, 7)]:
        q = rng.integers(-2, 3, (1, 2, T, 16)).astype(np.float32)
        k = rng.integers(-2, 3, (1, 2, past + T, 16)).astype(np.float32)
        v = rng.integers(-2, 3, (1, 1, past + T, 8)).astype(np.float32)
        got = ext.tril_score_v_past(to_dev(q, torch.float32), to_dev(k, torch.float32),
                                    to_dev(v, torch.float32), past)
        assert np.array_equal(np_of(got), O.tril_score_v_past(q, k, v, past)), (past, T)


@pytest.mark.parametrize("dtype", DTYPES)
def test_past_on_capacity_strided_cache_and_fp32_v(dtype):
    """Keys and values read in place from a cache of larger capacity; fp32 V under bf16 q."""
    B, H, T, past, N, D, cap = 2, 2, 70, 190, 64, 48, 320
    kc = torch.zeros(B, H, cap, N, dtype=dtype, device=DEV)
    vc = torch.zeros(B, 1, cap, D, dtype=torch.float32, device=DEV)
    k = as_dtype_values(latent((B, H, past + T, N), 21), dtype)
    v = normal((B, 1, past + T, D), 22)
    kc[:, :, : past + T] = to_dev(k, dtype)
    vc[:, :, : past + T] = to_dev(v, torch.float32)
    q = as_dtype_values(latent((B, H, T, N), 23), dtype)
    got = ext.tril_score_v_past(to_dev(q, dtype), kc[:, :, : past + T], vc[:, :, : past + T], past)
    want = O.tril_score_v_past(q, k, as_dtype_values(v, dtype), past)
    assert rel_fro(np_of(got), want) <= TOL[dtype]


def test_past_c1_chunk_matches_full_recompute_bf16():
    """A C1-width chunk (N = 8192, D = 256): the last 256 rows of a 1024-row
    sequence against the oracle, and against the same rows of the full cold op
    on the GPU (the reference's recompute-and-slice)."""
    B, H, T, past, N, D = 1, 4, 256, 768, 8192, 256
    g = torch.Generator(device=DEV).manual_seed(5)
    k = torch.relu(0.32 * torch.randn(B, H, past + T, N, generator=g, device=DEV)).to(torch.bfloat16)
    v = torch.randn(B, 1, past + T, D, generator=g, device=DEV).to(torch.bfloat16)
    got = ext.tril_score_v_past(k[:, :, past:], k, v, past)
    full = ext.tril_score_v(k, k, v)[:, :, past:]
    assert rel_fro(np_of(got), np_of(full)) <= TOL[torch.bfloat16]
    kk = np_of(k)
    want = O.tril_score_v_past(kk[:, :, past:], kk, np_of(v), past)
    err = rel_fro(np_of(got), want)
    print(f"C1-width chunk past={past}: rel {err:.3e}", flush=True)
    assert err <= TOL[torch.bfloat16]


def test_past_dispatch_and_errors():
    B, H, T, past, N, D = 1, 2, 9, 20, 16, 8
    k = torch.relu(torch.randn(B, H, past + T, N, device=DEV))
    v = torch.randn(B, 1, past + T, D, device=DEV)
    q = k[:, :, past:]
    hip = kernels.bdh_attn_past(q, k, v, past, impl="hip")
    eager = kernels.bdh_attn_past(q, k, v, past, impl="eager")
    assert rel_fro(np_of(hip), np_of(eager)) <= TOL[torch.float32]
    full = kernels.bdh_attn(k, k, v, impl="eager")[:, :, past:]
    assert rel_fro(np_of(hip), np_of(full)) <= TOL[torch.float32]
    with pytest.raises(RuntimeError):
        ext.tril_score_v_past(q, k[:, :, :-1], v[:, :, :-1], past)  # k shorter than past + T
    with pytest.raises(RuntimeError):
        ext.tril_score_v_past(q, k, v, -1)
    with pytest.raises(ValueError):
        kernels.tril_score_v_past(q, k, v, past + 1)
    with pytest.raises(ValueError):
        kernels.bdh_attn_past(q.clone().requires_grad_(), k, v, past, impl="hip")


@pytest.mark.parametrize("past,T", [(1, 40), (200, 100), (256, 256), (300, 500), (511, 1), (700, 333)])
def test_past_self_view_takes_score_tile_path(past, T):
    """q = k[..., past:, :] in bf16 (the reference's QR_all case) runs the
    score-tile kernels over the new rows' tiles only; results match the oracle
    and the generic kernels (q copied, so not a view of k)."""
    B, H, N, D = 2, 2, 256, 128
    print(f"past self view past={past} T={T}", flush=True)
    k = as_dtype_values(latent((B, H, past + T, N), 31), torch.bfloat16)
    v = as_dtype_values(normal((B, 1, past + T, D), 32), torch.bfloat16)
    kd, vd = to_dev(k, torch.bfloat16), to_dev(v, torch.bfloat16)
    ext.profile_enable(True)
    try:
        got = ext.tril_score_v_past(kd[:, :, past:], kd, vd, past)
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    assert "k_sy_scores" in names and names & {"k_sy_sv", "k_sv_dma"}, names
    want = O.tril_score_v_past(k[:, :, past:], k, v, past)
    assert rel_fro(np_of(got), want) <= TOL[torch.bfloat16]
    generic = ext.tril_score_v_past(kd[:, :, past:].clone(), kd, vd, past)
    assert rel_fro(np_of(got), np_of(generic)) <= TOL[torch.bfloat16]
