"""``bdh_cuda_ext``: the import name the reference's kernels/cuda_attn.py probes.

The reference loads its native module with ``import bdh_cuda_ext`` and routes
device tensors to it when ``has_cuda`` is true (kernels/cuda_attn.py:84-100,
391-414, 490-502).  On PyTorch-ROCm the device type ``cuda`` is the HIP
device, so this module exposes :mod:`bdh_hip_ext` under that name with
``has_cuda = True``: the reference's own wrapper then calls the gfx950 kernels
for ``q.is_cuda`` tensors without any edit.  Entries dispatch by device as the
reference's pybind functions do (tril_attn_bind.cpp:3-23): ROCm tensors go to
the HIP library, CPU tensors to the torch CPU entries.
"""

from __future__ import annotations

import torch

import bdh_hip_ext as _hip

has_cuda = True  # device type "cuda" is the ROCm/HIP device under PyTorch-ROCm
has_hip = True
lib_path = _hip.lib_path

tril_score_v_cpu = _hip.tril_score_v_cpu
tril_decode_cpu = _hip.tril_decode_cpu
tril_score_v_cuda = _hip.tril_score_v
tril_decode_cuda = _hip.tril_decode


def tril_score_v(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """``tril(q @ k^T, -1) @ v``: HIP kernels for ROCm tensors, torch on the CPU."""
    return _hip.tril_score_v(q, k, v) if q.is_cuda else _hip.tril_score_v_cpu(q, k, v)


def tril_decode(q: torch.Tensor, k_past: torch.Tensor, v_past: torch.Tensor) -> torch.Tensor:
    """``(q @ k_past^T) @ v_past``: HIP kernels for ROCm tensors, torch on the CPU."""
    return _hip.tril_decode(q, k_past, v_past) if q.is_cuda else _hip.tril_decode_cpu(q, k_past, v_past)


__all__ = [
    "has_cuda",
    "has_hip",
    "lib_path",
    "tril_score_v",
    "tril_score_v_cpu",
    "tril_score_v_cuda",
    "tril_decode",
    "tril_decode_cpu",
    "tril_decode_cuda",
]
