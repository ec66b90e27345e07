"""GPU checks of the encoder with its ReLU (``bdh_relu_gemm``) and of the gated form
(``bdh_gated_gemm``, x * relu(...)) on the same streaming kernel.

out[b, t, h, n] = relu(sum_k y[b, h, t, k] wt[h, n, k]) as bf16 (bdh.py:861-912,
`_encoder_relu`), against CPU references on the same bf16 inputs:
* float64 products rounded once to bf16: within 1e-2 relative Frobenius error,
  and at least 99 % of the elements bit-identical (fp32 sums in another order
  move an occasional value across a bf16 rounding boundary);
* the library's generic tile kernel (k_gated_gemm without the gate), which the
  entry point takes for shapes the streaming kernel does not: the same bounds.
Shapes: K = 256 and 512 on the streaming kernel (ragged last token blocks, N
down to one chunk), the tile kernel below its workgroup threshold and for K =
128, one token, heads sharing y through a zero head stride (the encoder) and
per-head y.
"""

from __future__ import annotations

import pytest
import torch

from helpers import rel_fro

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():
    pytest.skip("needs a ROCm GPU", allow_module_level=True)

import bdh_hip_ext as ext  # noqa: E402  (fails loudly when the library is missing)

DEV = torch.device("cuda:0")
BF = torch.bfloat16


def _inputs(B, T, nh, N, K, seed, shared):
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(B, 1 if shared else nh, T, K, generator=g).to(BF)
    wt = (0.05 * torch.randn(nh, N, K, generator=g)).to(BF)
    return y, wt


def _want(y, wt, nh):
    yy = y.double().expand(y.size(0), nh, y.size(2), y.size(3))
    lin = torch.matmul(yy, wt.double().transpose(1, 2))  # (B, nh, T, N)
    return torch.relu(lin).permute(0, 2, 1, 3).float().to(BF)


# (B, T, nh, N, K): the streaming kernel takes K = 256 / 512 when (B*T / 256) x nh >= 128
# workgroups: a ragged last token block (77 and 116 tokens), one chunk (N = 64 at K = 256),
# two (N = 64 at K = 512); the tile kernel below that (a decode step's 64 tokens, short
# prompts) and for K = 128.
STREAM_SHAPES = [(1, 32845, 1, 64, 256), (2, 8250, 2, 64, 512), (4, 8200, 4, 128, 256)]
TILE_SHAPES = [(2, 300, 4, 1024, 256), (1, 1, 2, 64, 256), (3, 129, 3, 192, 512), (2, 77, 2, 96, 128)]


@pytest.mark.parametrize("shape", STREAM_SHAPES + TILE_SHAPES)
@pytest.mark.parametrize("shared", [True, False])
def test_relu_gemm_matches_reference(shape, shared):
    B, T, nh, N, K = shape
    print(f"relu_gemm {shape} shared={shared}", flush=True)
    y, wt = _inputs(B, T, nh, N, K, seed=B * 7 + T + N + K, shared=shared)
    yd = y.to(DEV)
    yd = yd.expand(B, nh, T, K) if shared else yd
    got = ext.relu_gemm(yd, wt.to(DEV)).cpu()
    assert got.shape == (B, T, nh, N) and got.dtype == BF
    want = _want(y, wt, nh)
    e = rel_fro(got.float().numpy(), want.float().numpy())
    same = float((got == want).float().mean())
    print(f"  rel {e:.2e}, bit-identical {same:.4f}", flush=True)
    assert e <= 1e-2
    assert same >= 0.99
    assert bool((got >= 0).all())


def test_relu_gemm_encoder_view_matches_generic_kernel():
    """At C2's shape (B = 32, T = 512): the streaming kernel (N a multiple of 64)
    against the generic tile kernel on the same rows (N = 8184 goes to it), and
    repeated calls give the same bits."""
    B, T, nh, K = 32, 512, 4, 256
    y, wt = _inputs(B, T, nh, 8192, K, seed=11, shared=True)
    yd = y.to(DEV).expand(B, nh, T, K)
    wd = wt.to(DEV)
    got = ext.relu_gemm(yd, wd)
    assert torch.equal(got, ext.relu_gemm(yd, wd))
    gen = ext.relu_gemm(yd, wd[:, :8184].contiguous())
    a, b = got[..., :8184].float().cpu(), gen.float().cpu()
    assert rel_fro(a.numpy(), b.numpy()) <= 1e-2
    assert float((got[..., :8184] == gen).float().mean()) >= 0.99


def test_relu_gemm_rejects_bad_shapes():
    y, wt = (t.to(DEV) for t in _inputs(1, 8, 2, 64, 256, seed=3, shared=False))
    with pytest.raises(RuntimeError):
        ext.relu_gemm(y, wt[..., :128].contiguous())  # K mismatch
    with pytest.raises(RuntimeError):
        ext.relu_gemm(y[:, :1].contiguous(), wt)  # head count


def _want_gated(y, wt, x):
    """x * relu(y wt^T): the GEMM in float64, relu rounded to bf16, the product rounded to bf16."""
    lin = torch.matmul(y.double(), wt.double().transpose(1, 2))  # (B, nh, T, N)
    r = torch.relu(lin).float().to(BF).permute(0, 2, 1, 3)
    return (x.float() * r.float()).to(BF)


@pytest.mark.parametrize("shape", STREAM_SHAPES + TILE_SHAPES)
def test_gated_form_matches_reference(shape):
    """The gated form (x * relu(y wt^T), the encoder_v product of the layer; the
    streaming kernel for K = 256 / 512, the generic tile kernel for K = 128)
    against float64 with the two bf16 roundings: within 1e-2, 99 % bit-identical."""
    B, T, nh, N, K = shape
    print(f"gated form {shape}", flush=True)
    y, wt = _inputs(B, T, nh, N, K, seed=B * 11 + T + N + K, shared=False)
    g = torch.Generator().manual_seed(N + K)
    x = torch.relu(torch.randn(B, T, nh, N, generator=g)).to(BF)
    got = ext.gated_gemm(y.to(DEV), wt.to(DEV), x.to(DEV)).cpu()
    want = _want_gated(y, wt, x)
    e = rel_fro(got.float().numpy(), want.float().numpy())
    same = float((got == want).float().mean())
    print(f"  rel {e:.2e}, bit-identical {same:.4f}", flush=True)
    assert got.shape == (B, T, nh, N) and e <= 1e-2 and same >= 0.99


def test_gated_form_c5_width_repeats_and_matches_generic():
    """At C5's shape (B = 4, T = 2048, K = 512, 8 x 8192 columns): repeated
    calls give the same bits, and the generic tile kernel (N = 8184 goes to it)
    agrees on the shared columns."""
    B, T, nh, N, K = 4, 2048, 8, 8192, 512
    y, wt = (t.to(DEV) for t in _inputs(B, T, nh, N, K, seed=5, shared=False))
    g = torch.Generator().manual_seed(9)
    x = torch.relu(torch.randn(B, T, nh, N, generator=g)).to(BF).to(DEV)
    got = ext.gated_gemm(y, wt, x)
    for _ in range(3):
        assert torch.equal(got, ext.gated_gemm(y, wt, x))
    gen = ext.gated_gemm(y, wt[:, :8184].contiguous(), x[..., :8184].contiguous())
    a, b = got[..., :8184], gen
    assert rel_fro(a.float().cpu().numpy(), b.float().cpu().numpy()) <= 1e-2
    assert float((a == b).float().mean()) >= 0.99


@pytest.mark.parametrize("tokens", [64, 4096])
def test_few_tokens_take_the_tile_kernel(tokens):
    """The streaming kernel needs (tokens / 256) x heads >= 128 workgroups; a
    decode step's few tokens (64 here, C3's batch) take the tile kernel, a
    prefill's the streaming one (checked in the launch log); both against
    float64."""
    B, T, nh, N, K = tokens, 1, 4, 8192, 256
    if tokens == 4096:
        B, T, nh = 8, 512, 8
    y, wt = _inputs(B, T, nh, N, K, seed=tokens, shared=False)
    g = torch.Generator().manual_seed(tokens)
    x = torch.relu(torch.randn(B, T, nh, N, generator=g)).to(BF)
    ext.profile_enable(True)
    try:
        got = ext.gated_gemm(y.to(DEV), wt.to(DEV), x.to(DEV))
        torch.cuda.synchronize()
        names = {n for n, _ in ext.profile_collect()}
    finally:
        ext.profile_enable(False)
    assert names == ({"k_gated_gemm"} if tokens == 64 else {"k_gated_enc"}), names
    want = _want_gated(y, wt, x)
    assert rel_fro(got.float().cpu().numpy(), want.float().numpy()) <= 1e-2
