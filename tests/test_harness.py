"""CPU checks of the model oracle and of the model harness (eager attention).

The model oracle (numpy, bdh_baseline.py:109-151) is pinned by a pure-Python
loop model on tiny shapes, closed forms (T = 1; encoder_v = 0), causality and
LayerNorm's moments.  The harness (``bdh_harness.BDH``) with ``impl="eager"``
must match it at fp32 (1e-4 relative Frobenius), and its cached paths (prompt
prefill into the cache, one-token decode, multi-token chunks after a past)
must reproduce the full forward's logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import rel_fro
from oracle import bdh_model_oracle as M

import bdh_harness as H


def _model(p, mult):
    nh, D, N = p["encoder"].shape
    cfg = H.BDHConfig(n_layer=int(p["n_layer"]), n_embd=D, n_head=nh, mlp_internal_dim_multiplier=mult,
                      vocab_size=p["lm_head"].shape[1])
    assert cfg.n_latent == N
    m = H.BDH(cfg)
    with torch.no_grad():
        for k in ("encoder", "encoder_v", "decoder", "lm_head"):
            getattr(m, k).copy_(torch.from_numpy(p[k]))
        m.embed.weight.copy_(torch.from_numpy(p["embed"]))
    return m


def _closed_form(p, idx):
    """Every layer is x <- LN(x) when attention or encoder_v contributes nothing."""
    x = M.layer_norm(p["embed"][idx])
    for _ in range(int(p["n_layer"])):
        x = M.layer_norm(x)
    return x @ p["lm_head"]


def test_model_oracle_matches_loop_model():
    p = M.init_params(2, 4, 2, 4, 5, seed=1)
    for k in ("encoder", "encoder_v", "decoder"):
        p[k] = p[k] * 25.0  # O(1) activations so every term matters
    idx = np.array([[1, 4, 0], [3, 3, 2]])
    assert rel_fro(M.bdh_forward(p, idx), M.bdh_forward_loops(p, idx)) <= 1e-5


def test_model_oracle_closed_forms_and_causality():
    p = M.init_params(3, 8, 2, 8, 7, seed=2)
    idx1 = np.array([[5], [2]])
    np.testing.assert_allclose(M.bdh_forward(p, idx1), _closed_form(p, idx1), rtol=1e-5, atol=1e-6)
    q = dict(p, encoder_v=np.zeros_like(p["encoder_v"]))
    idx = np.array([[1, 2, 3, 4, 5, 6]])
    np.testing.assert_allclose(M.bdh_forward(q, idx), _closed_form(q, idx), rtol=1e-5, atol=1e-6)
    p["encoder"] *= 20
    p["encoder_v"] *= 20
    a = M.bdh_forward(p, np.array([[1, 2, 3, 4, 5, 6]]))
    b = M.bdh_forward(p, np.array([[1, 2, 3, 0, 0, 0]]))
    np.testing.assert_array_equal(a[:, :3], b[:, :3])
    assert np.abs(a[:, 3:] - b[:, 3:]).max() > 1e-3
    y = M.layer_norm(np.random.default_rng(0).standard_normal((4, 32)) * 3 + 1)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-6)
    np.testing.assert_allclose(y.var(-1), 1, atol=1e-3)


def test_harness_eager_matches_oracle():
    p = M.init_params(2, 32, 2, 64, 11, seed=3)
    m = _model(p, mult=4)
    idx = np.random.default_rng(4).integers(0, 11, (2, 20))
    got, _ = m(torch.from_numpy(idx), impl="eager")
    assert rel_fro(got.detach().numpy(), M.bdh_forward(p, idx)) <= 1e-4


def test_harness_cached_paths_match_full_forward():
    p = M.init_params(2, 32, 2, 64, 11, seed=5)
    m = _model(p, mult=4)
    idx = torch.from_numpy(np.random.default_rng(6).integers(0, 11, (2, 14)))
    full, _ = m(idx, impl="eager")
    cache = H.KVCache(m.config, 2, 14, torch.float32, "cpu")
    with torch.no_grad():
        pre, _ = m(idx[:, :6], cache=cache, impl="eager")          # prompt prefill
        step, _ = m(idx[:, 6:7], cache=cache, impl="eager")        # one-token decode
        chunk, _ = m(idx[:, 7:11], cache=cache, impl="eager")      # chunk after a past
        last, _ = m(idx[:, 11:14], cache=cache, impl="eager", last_only=True)
    assert cache.seq_len == 14
    got = torch.cat([pre, step, chunk], dim=1)
    assert rel_fro(got.numpy(), full[:, :11].detach().numpy()) <= 1e-4
    assert rel_fro(last.numpy(), full[:, 13:14].detach().numpy()) <= 1e-4


def test_sampler_and_generate_on_cpu():
    g = torch.Generator().manual_seed(0)
    logits = torch.tensor([[0.0, 5.0, 4.0, -1.0, 3.0]] * 64)
    picks = H.BDH.sample(logits, 1.0, 2, generator=g)
    assert set(picks.flatten().tolist()) <= {1, 2}
    p = M.init_params(2, 16, 2, 32, 9, seed=7)
    m = _model(p, mult=4)
    idx = torch.from_numpy(np.random.default_rng(8).integers(0, 9, (3, 5)))
    out = m.generate(idx, 4, top_k=3, impl="eager", generator=torch.Generator().manual_seed(1))
    assert out.shape == (3, 9) and torch.equal(out[:, :5], idx)
    again = m.generate(idx, 4, top_k=3, impl="eager", generator=torch.Generator().manual_seed(1))
    assert torch.equal(out, again)
    with pytest.raises(ValueError):
        H.KVCache(m.config, 1, 2, torch.float32, "cpu").slot(0, 3)
