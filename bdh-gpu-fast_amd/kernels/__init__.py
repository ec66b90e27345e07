"""BDH attention + RoPE operators: the reference's ``kernels`` import surface.

Drop-in counterpart of the reference package ``kernels`` (kernels/__init__.py):
``bdh.py`` imports ``bdh_attn``, ``bdh_attn_decode``, ``resolve_attn_impl``,
``_env_autograd_enabled``, ``bdh_rope_rotate``, ``bdh_rope_rotate_paired`` and
``resolve_rope_impl`` from here unchanged.  ``BDH_ATTN_IMPL=hip`` /
``BDH_ROPE_IMPL=hip`` select the gfx950 HIP kernels; ``eager`` (default) keeps
the reference's PyTorch semantics.  The wider set of the reference's
``kernels/__init__.py:3-97`` (tile pickers, ``*_ref`` references, Triton and
native probes) is exported too.  ``tril_score_v`` / ``tril_decode`` are the
dispatchers of :mod:`kernels.cuda_attn`, as in the reference: ROCm tensors run
the HIP kernels (errors raised), CPU tensors the CPU entries.
"""

from .attention import (
    DEFAULT_BLOCK_COLD,
    DEFAULT_BLOCK_DECODE,
    eager_decode_attn,
    eager_past_attn,
    eager_tril_attn,
    pick_triton_cold_tiles,
    triton_cold_skip_reason,
    triton_decode_available,
)
from .attention_bwd import (
    StrictTrilAttnFn,
    StrictTrilSelfAttnFn,
    TrilRopeSelfAttnFn,
    analytic_tril_attn_backward,
    analytic_tril_attn_backward_blocked,
    strict_tril_attn,
)
from .attention_dispatch import (
    DEFAULT_ATTN_AUTO_THRESHOLD,
    attn_auto_cold_threshold,
    attn_auto_enabled,
    attn_auto_threshold,
    backend_info,
    bdh_attn,
    bdh_attn_decode,
    bdh_attn_past,
    bdh_attn_rope,
    resolve_attn_impl,
    resolve_cold_impl,
    resolve_decode_impl,
)
from .cuda_attn import (
    CUDA_DECODE_TILE_N,
    CUDA_DECODE_TILE_N_MAX,
    CUDA_TILE_M,
    CUDA_TILE_M_CPU_MAX,
    CUDA_TILE_M_MAX,
    CUDA_TILE_N,
    CUDA_TILE_N_CPU_MAX,
    CUDA_TILE_N_MAX,
    ext_status,
    has_cuda_ext,
    has_cuda_kernel,
    pick_cuda_cold_tiles,
    pick_cuda_decode_tile_n,
    tril_decode,
    tril_decode_ref,
    tril_decode_tiled_ref,
    tril_score_v,
    tril_score_v_ref,
    tril_score_v_tiled_ref,
)
from .hip_attn import (
    has_hip_ext,
    gated_gemm,
    gated_decoder,
    has_hip_kernel,
    relu_gemm,
    layer_norm_rows,
    relu_mul,
    small_gemm,
    tril_rope_score_v,
    tril_score_v_past,
)
from .rope import get_freqs, rope_cos_sin
from .rope_dispatch import backend_info as rope_backend_info
from .rope_dispatch import bdh_rope_rotate, bdh_rope_rotate_paired, resolve_rope_impl

__all__ = [
    "bdh_attn",
    "bdh_attn_rope",
    "bdh_attn_decode",
    "bdh_attn_past",
    "resolve_attn_impl",
    "resolve_cold_impl",
    "resolve_decode_impl",
    "attn_auto_threshold",
    "attn_auto_cold_threshold",
    "attn_auto_enabled",
    "DEFAULT_ATTN_AUTO_THRESHOLD",
    "DEFAULT_BLOCK_COLD",
    "DEFAULT_BLOCK_DECODE",
    "backend_info",
    "strict_tril_attn",
    "StrictTrilAttnFn",
    "StrictTrilSelfAttnFn",
    "TrilRopeSelfAttnFn",
    "analytic_tril_attn_backward",
    "analytic_tril_attn_backward_blocked",
    "eager_tril_attn",
    "eager_decode_attn",
    "eager_past_attn",
    "tril_score_v",
    "tril_score_v_past",
    "relu_mul",
    "gated_gemm",
    "gated_decoder",
    "relu_gemm",
    "small_gemm",
    "layer_norm_rows",
    "tril_rope_score_v",
    "tril_decode",
    "has_hip_ext",
    "has_hip_kernel",
    "ext_status",
    "get_freqs",
    "rope_cos_sin",
    "bdh_rope_rotate",
    "bdh_rope_rotate_paired",
    "resolve_rope_impl",
    "rope_backend_info",
    "triton_decode_available",
    "triton_cold_skip_reason",
    "pick_triton_cold_tiles",
    "tril_score_v_ref",
    "tril_score_v_tiled_ref",
    "tril_decode_ref",
    "tril_decode_tiled_ref",
    "pick_cuda_cold_tiles",
    "pick_cuda_decode_tile_n",
    "has_cuda_ext",
    "has_cuda_kernel",
    "CUDA_TILE_M",
    "CUDA_TILE_N",
    "CUDA_TILE_M_MAX",
    "CUDA_TILE_N_MAX",
    "CUDA_TILE_M_CPU_MAX",
    "CUDA_TILE_N_CPU_MAX",
    "CUDA_DECODE_TILE_N",
    "CUDA_DECODE_TILE_N_MAX",
]
