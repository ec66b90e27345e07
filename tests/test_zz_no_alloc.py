"""The no-allocation decode entry point (``bdh_tril_decode_noalloc``) against
``bdh_tril_decode``: same kernels, so the same bits, on two calls in a row
(the second with a smaller input, over the scratch the first left behind),
on the bf16 cache path and the generic path; inputs larger than the scratch
are refused with BDH_ERR_SCRATCH."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402

DEV = "cuda"


def _cache(B, H, cap, N, D, kdt, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.relu(0.32 * torch.randn(B, H, cap, N, generator=g, device=DEV)).to(kdt)
    v = torch.randn(B, 1, cap, D, generator=g, device=DEV).to(kdt)
    q = torch.relu(0.32 * torch.randn(B, H, 1, N, generator=g, device=DEV)).to(kdt)
    return q, k, v


@pytest.mark.parametrize("kdt,N", [(torch.bfloat16, 8192), (torch.float32, 1024)])
def test_noalloc_decode_equals_workspace_decode(kdt, N):
    print(f"noalloc decode {kdt} N={N}", flush=True)
    B, H, D, cap = 64, 4, 256, 512
    q, k, v = _cache(B, H, cap, N, D, kdt, 5)
    for S, bs in ((511, B), (130, 7)):  # second call smaller: fewer rows and chunks
        qs, ks, vs = q[:bs], k[:bs, :, :S], v[:bs, :, :S]  # capacity-strided past views
        want = ext.tril_decode(qs, ks, vs)
        out = torch.full_like(want, float("nan"))
        got = ext.tril_decode_noalloc(qs, ks, vs, out=out)
        torch.cuda.synchronize()
        assert got is out
        assert torch.equal(got, want), (S, bs)


def test_noalloc_decode_refuses_inputs_beyond_its_scratch():
    B, H, N, D, S = 64, 4, 2048, 256, 4096 + 64  # 65 chunks of 64 keys x 256 rows x 1 KB > 16 MiB
    q = torch.zeros(B, H, 1, N, dtype=torch.bfloat16, device=DEV)
    k = torch.zeros(B, H, S, N, dtype=torch.bfloat16, device=DEV)
    v = torch.zeros(B, 1, S, D, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="scratch"):
        ext.tril_decode_noalloc(q, k, v)
    # the largest that fits still runs
    out = ext.tril_decode_noalloc(q, k[:, :, :4096], v[:, :, :4096])
    torch.cuda.synchronize()
    assert not out.any().item()
