"""GPU checks of the gated product chained into the decoder (``bdh_gated_decoder``).

y_mlp = (x * relu(y @ wt^T)) viewed (B, T, nh*N) @ dec, the product never
stored (bdh.py:914-945, bdh_baseline.py:135-141), against CPU references on
the same bf16 inputs:
* the kernel's own rounding (each product x * relu(...) rounded to bf16 once,
  fp32 sums): within 2e-3 (only the fp32 summation order differs, and with it
  an occasional last-bit difference of a rounded product);
* float64 without the intermediate rounding: within 2e-2 (the bf16 tolerance);
* the library's two-step path (``gated_gemm``, then the decoder product): within
  1e-2.
Shapes: ragged token blocks (B*T not a multiple of 256), one token, several
heads, N from 32 to 8192, the model's permuted views, bf16 and fp32 outputs.
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


def _inputs(B, T, nh, N, seed):
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(B, nh, T, 256, generator=g).to(BF)
    wt = (0.05 * torch.randn(nh, N, 256, generator=g)).to(BF)
    x = torch.relu(torch.randn(B, T, nh, N, generator=g)).to(BF)
    dec = (0.02 * torch.randn(nh * N, 256, generator=g)).to(BF)
    return y, wt, x, dec


def _want(y, wt, x, dec, round_xy=True):
    B, T, nh, N = x.shape
    lin = torch.matmul(y.double(), wt.double().transpose(1, 2))  # (B, nh, T, N)
    xy = x.double() * torch.relu(lin).permute(0, 2, 1, 3)  # (B, T, nh, N)
    if round_xy:
        xy = xy.float().to(BF).double()
    return (xy.reshape(B, T, nh * N) @ dec.double()).float()


@pytest.mark.parametrize("shape", [(2, 300, 2, 1024), (1, 1, 1, 32), (3, 129, 4, 96), (1, 512, 4, 8192),
                                   (2, 256, 3, 64)])
@pytest.mark.parametrize("odt", [torch.float32, BF])
def test_gated_decoder_matches_references(shape, odt):
    B, T, nh, N = shape
    print(f"gated_decoder {shape} {odt}", flush=True)
    y, wt, x, dec = _inputs(B, T, nh, N, seed=B * 1000 + T + N)
    got = ext.gated_decoder(y.to(DEV), wt.to(DEV), x.to(DEV), dec.to(DEV), odt)
    assert got.shape == (B, T, 256) and got.dtype == odt
    g = got.float().cpu()
    tol = 2e-3 if odt == torch.float32 else 5e-3
    e1 = rel_fro(g.numpy(), _want(y, wt, x, dec).numpy())
    e2 = rel_fro(g.numpy(), _want(y, wt, x, dec, round_xy=False).numpy())
    print(f"  vs its rounding {e1:.2e}, vs float64 {e2:.2e}", flush=True)
    assert e1 <= tol
    assert e2 <= 2e-2


def test_gated_decoder_on_model_views_matches_two_step():
    """The harness's operands: x the encoder's (B, T, nh, N) output, y the
    LayerNorm of the attention output, the decoder as (nh*N, D); against
    ``gated_gemm`` followed by the decoder product (the path it replaces), and
    repeated calls give the same bits (the heads' partials add in order)."""
    B, T, nh, N = 4, 512, 4, 8192
    print("gated_decoder vs two-step, C2 width", flush=True)
    y, wt, x, dec = (t.to(DEV) for t in _inputs(B, T, nh, N, seed=7))
    got = ext.gated_decoder(y, wt, x, dec)
    again = ext.gated_decoder(y, wt, x, dec)
    assert torch.equal(got, again)
    xy = ext.gated_gemm(y, wt, x)
    two = xy.view(B, T, nh * N).float() @ dec.float()
    e = rel_fro(got.cpu().numpy(), two.cpu().numpy())
    print(f"  vs gated_gemm + decoder {e:.2e}", flush=True)
    assert e <= 1e-2


def test_gated_decoder_rejects_bad_shapes():
    y, wt, x, dec = (t.to(DEV) for t in _inputs(1, 8, 2, 64, seed=3))
    with pytest.raises(RuntimeError):
        ext.gated_decoder(y[..., :128].contiguous(), wt[..., :128].contiguous(), x, dec)  # K != 256
    with pytest.raises(RuntimeError):
        ext.gated_decoder(y, wt[:, :48].contiguous(), x[..., :48].contiguous(), dec[:96].contiguous())  # N % 32
