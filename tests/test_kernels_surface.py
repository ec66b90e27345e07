"""CPU tests of the wider ``kernels`` import surface: every name the reference's
kernels/__init__.py:3-97 exports imports from this package, ``kernels.cuda_attn``
exists with the reference module's names, its tile pickers give the values the
reference's own tests assert, and its torch references and CPU dispatchers
agree with the oracle.  No GPU compute."""

from __future__ import annotations

import importlib
import sys

import numpy as np
import pytest
import torch

import oracle as O
from helpers import rel_fro

# The reference's kernels/__init__.py __all__ (kernels/__init__.py:55-97), as data.
REFERENCE_KERNELS_ALL = [
    "bdh_attn", "bdh_attn_decode", "resolve_attn_impl", "resolve_cold_impl",
    "resolve_decode_impl", "attn_auto_threshold", "attn_auto_cold_threshold",
    "attn_auto_enabled", "DEFAULT_ATTN_AUTO_THRESHOLD", "triton_decode_available",
    "triton_cold_skip_reason", "pick_triton_cold_tiles", "backend_info",
    "strict_tril_attn", "StrictTrilAttnFn", "StrictTrilSelfAttnFn",
    "analytic_tril_attn_backward", "analytic_tril_attn_backward_blocked",
    "tril_score_v", "tril_score_v_ref", "tril_score_v_tiled_ref", "tril_decode",
    "tril_decode_ref", "tril_decode_tiled_ref", "pick_cuda_cold_tiles",
    "pick_cuda_decode_tile_n", "has_cuda_ext", "has_cuda_kernel", "ext_status",
    "CUDA_TILE_M", "CUDA_TILE_N", "CUDA_TILE_M_MAX", "CUDA_TILE_N_MAX",
    "CUDA_TILE_M_CPU_MAX", "CUDA_TILE_N_CPU_MAX", "CUDA_DECODE_TILE_N",
    "CUDA_DECODE_TILE_N_MAX", "bdh_rope_rotate", "bdh_rope_rotate_paired",
    "resolve_rope_impl", "rope_backend_info",
]

# Names the reference's kernels/cuda_attn.py defines at module level and its tests import.
REFERENCE_CUDA_ATTN = [
    "CUDA_TILE_M", "CUDA_TILE_N", "CUDA_TILE_D", "CUDA_TILE_M_MAX", "CUDA_TILE_N_MAX",
    "CUDA_TILE_M_CPU_MAX", "CUDA_TILE_N_CPU_MAX", "CUDA_DECODE_TILE_N",
    "CUDA_DECODE_TILE_N_MAX", "CUDA_DECODE_TILE_N_CPU_MAX", "has_cuda_ext",
    "has_cuda_kernel", "pick_cuda_cold_tiles", "pick_cuda_decode_tile_n",
    "tril_score_v_ref", "tril_score_v_tiled_ref", "tril_score_v", "tril_decode_ref",
    "tril_decode_tiled_ref", "tril_decode", "ext_status",
]


def test_every_reference_kernels_name_imports():
    kernels = importlib.import_module("kernels")
    assert kernels.__file__.startswith(str(__import__("pathlib").Path(__file__).resolve().parents[1]))
    missing = [n for n in REFERENCE_KERNELS_ALL if not hasattr(kernels, n)]
    assert not missing, missing
    assert not [n for n in REFERENCE_KERNELS_ALL if n not in kernels.__all__]
    ns: dict = {}
    exec("from kernels import " + ", ".join(REFERENCE_KERNELS_ALL), ns)
    assert all(n in ns for n in REFERENCE_KERNELS_ALL)


def test_kernels_cuda_attn_module_has_reference_names():
    ca = importlib.import_module("kernels.cuda_attn")
    missing = [n for n in REFERENCE_CUDA_ATTN if not hasattr(ca, n)]
    assert not missing, missing
    assert ca.has_cuda_ext()  # the HIP library is built in-tree
    assert ca.has_cuda_kernel() == torch.cuda.is_available()
    assert ca.ext_status().startswith("native=loaded")


def test_tile_pickers_match_reference_asserts():
    """Values the reference's own tests assert (test_cuda_attn.py:287-318,
    test_cuda_decode.py:250-264, test_inc_decode.py:694-705, test_triton_attn.py:233-256)."""
    import kernels
    from kernels import cuda_attn as ca

    assert ca.CUDA_TILE_M == 16 and ca.CUDA_TILE_N == 16
    assert ca.pick_cuda_cold_tiles(32) == (16, 16)
    assert ca.pick_cuda_cold_tiles(128) == (32, 32)
    assert ca.pick_cuda_cold_tiles(512) == (128, 128)
    tm, tn = ca.pick_cuda_cold_tiles(512, Dk=64, for_smem=True)
    assert 16 <= tm <= ca.CUDA_TILE_M_MAX and 16 <= tn <= ca.CUDA_TILE_N_MAX
    assert ca.pick_cuda_cold_tiles(512, tile_m=16, tile_n=16) == (16, 16)
    assert ca.pick_cuda_cold_tiles(512, Dk=128, Dv=256) == (64, 64)
    assert ca.pick_cuda_cold_tiles(512, Dk=128, Dv=256, for_smem=True) == (32, 32)
    assert ca.pick_cuda_cold_tiles(512, Dk=128, Dv=256, tile_m=16, tile_n=16) == (16, 16)
    assert ca.pick_cuda_cold_tiles(260, 128, Dv=256) == (64, 64)
    # An explicit width rounds up the power-of-two ladder (cuda_attn.py:156-163).
    assert ca.pick_cuda_cold_tiles(512, tile_m=100, tile_n=17) == (128, 32)

    assert ca.pick_cuda_decode_tile_n(32) == 32
    assert ca.pick_cuda_decode_tile_n(64) == 32
    assert ca.pick_cuda_decode_tile_n(128) >= 64
    assert ca.pick_cuda_decode_tile_n(512) >= 64
    assert ca.pick_cuda_decode_tile_n(2048) >= 128
    assert ca.pick_cuda_decode_tile_n(4096) == 512
    assert ca.pick_cuda_decode_tile_n(4096, tile_n=64) == 64
    assert ca.pick_cuda_decode_tile_n(4096, for_smem=True) <= ca.CUDA_DECODE_TILE_N_MAX
    assert ca.pick_cuda_decode_tile_n(100) >= 32

    from kernels.attention import DEFAULT_BLOCK_COLD, pick_cold_block_size

    assert pick_cold_block_size(128) == DEFAULT_BLOCK_COLD
    assert pick_cold_block_size(256) == 128
    bm, bn, bd, bk = kernels.pick_triton_cold_tiles(T=128, N=64, D=128)
    assert (bm, bn, bd, bk) == (64, 64, 64, 64)
    assert kernels.pick_triton_cold_tiles(T=256, N=64, D=128)[:2] == (128, 128)
    assert kernels.pick_triton_cold_tiles(T=512, N=64, D=128)[:2] == (128, 128)
    assert kernels.pick_triton_cold_tiles(T=512, N=128, D=256)[:2] == (DEFAULT_BLOCK_COLD,) * 2
    assert kernels.pick_triton_cold_tiles(512, 128, 256, block_m=128, block_n=128)[:2] == (128, 128)
    assert kernels.triton_decode_available() is False
    assert "CPU-safe skip" in kernels.triton_cold_skip_reason()


@pytest.mark.parametrize("T,vh", [(1, 1), (31, 1), (260, 1), (300, 3), (600, 1)])
def test_cold_refs_and_cpu_dispatch_match_oracle(T, vh):
    """Both torch references and the CPU dispatcher against the oracle's brute
    closed form; row 0 exactly zero (tril_attn.h:1-4)."""
    from kernels import cuda_attn as ca

    g = torch.Generator().manual_seed(7 + T)
    q = torch.relu(0.32 * torch.randn(2, 3, T, 40, generator=g))
    v = torch.randn(2, vh, T, 24, generator=g)
    want = O.tril_score_v_eager(q.numpy(), q.numpy(), v.numpy())
    for fn in (ca.tril_score_v_ref, ca.tril_score_v_tiled_ref, ca.tril_score_v):
        got = fn(q, q, v)
        assert got.shape == (2, 3, T, 24)
        assert rel_fro(got.numpy(), want) <= 1e-5, fn.__name__
        assert torch.count_nonzero(got[:, :, 0]) == 0
    # Narrow explicit tiles force the chunked past branch (cuda_attn.py:361-372).
    got = ca.tril_score_v_tiled_ref(q, q, v, tile_m=16, tile_n=16)
    assert rel_fro(got.numpy(), want) <= 1e-5


def test_tiled_ref_bf16_accumulates_in_fp32():
    from kernels import cuda_attn as ca

    g = torch.Generator().manual_seed(3)
    q = torch.relu(0.32 * torch.randn(1, 2, 300, 64, generator=g)).bfloat16()
    v = torch.randn(1, 1, 300, 32, generator=g).bfloat16()
    got = ca.tril_score_v_tiled_ref(q, q, v)
    assert got.dtype == torch.bfloat16
    want = O.tril_score_v_eager(q.float().numpy(), q.float().numpy(), v.float().numpy())
    assert rel_fro(got.float().numpy(), want) <= 1e-2


@pytest.mark.parametrize("S,tq", [(0, 1), (1, 1), (37, 1), (700, 1), (300, 4)])
def test_decode_refs_and_cpu_dispatch_match_oracle(S, tq):
    from kernels import cuda_attn as ca

    g = torch.Generator().manual_seed(11 + S)
    q = torch.randn(2, 3, tq, 48, generator=g)
    kp = torch.randn(2, 3, S, 48, generator=g)
    vp = torch.randn(2, 1, S, 16, generator=g)
    want = O.tril_decode_eager(q.numpy(), kp.numpy(), vp.numpy())
    for fn in (ca.tril_decode_ref, ca.tril_decode_tiled_ref, ca.tril_decode):
        got = fn(q, kp, vp)
        assert got.shape == (2, 3, tq, 16)
        assert rel_fro(got.numpy(), want) <= 1e-5, fn.__name__
    got = ca.tril_decode_tiled_ref(q, kp, vp, tile_n=16)
    assert rel_fro(got.numpy(), want) <= 1e-5


def test_cuda_attn_validators_raise_before_dispatch():
    from kernels import cuda_attn as ca

    with pytest.raises(ValueError, match="must be 4D"):
        ca.tril_score_v(torch.zeros(2, 3), torch.zeros(2, 3), torch.zeros(2, 3))
    with pytest.raises(ValueError, match="shapes must match"):
        ca.tril_score_v(torch.zeros(1, 1, 4, 8), torch.zeros(1, 1, 5, 8), torch.zeros(1, 1, 4, 2))
    with pytest.raises(ValueError, match="incompatible"):
        ca.tril_decode(torch.zeros(1, 2, 1, 8), torch.zeros(1, 2, 3, 4), torch.zeros(1, 1, 3, 2))


def test_reference_native_module_name_routes_device_tensors():
    """``bdh_cuda_ext`` is the import name the reference's own cuda_attn.py probes;
    its ``has_cuda`` attribute is what that wrapper reads (cuda_attn.py:93-97) to send
    ``q.is_cuda`` tensors (the HIP device under PyTorch-ROCm) to the native entries."""
    ext = importlib.import_module("bdh_cuda_ext")
    assert ext.has_cuda is True and ext.has_hip is True
    q = torch.randn(1, 2, 9, 8)
    v = torch.randn(1, 1, 9, 4)
    want = O.tril_score_v_eager(q.numpy(), q.numpy(), v.numpy())
    assert rel_fro(ext.tril_score_v(q, q, v).numpy(), want) <= 1e-6
    assert "bdh-gpu-fast_amd" in sys.modules["bdh_cuda_ext"].__file__
