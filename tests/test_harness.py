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


def test_loss_grads_oracle_pinned_by_forward_and_finite_differences():
    """``bdh_loss_grads`` (float64 autograd of the model formula): its logits
    equal the numpy oracle's, and every parameter's gradient matches central
    finite differences of its own loss on sampled entries."""
    p = M.init_params(2, 4, 2, 8, 7, seed=23)
    for k in ("encoder", "encoder_v", "decoder"):
        p[k] = p[k] * 25.0  # O(1) activations so every term matters
    rng = np.random.default_rng(24)
    idx, tgt = rng.integers(0, 7, (2, 6)), rng.integers(0, 7, (2, 6))
    loss, g, logits = M.bdh_loss_grads(p, idx, tgt, return_logits=True)
    assert rel_fro(logits, M.bdh_forward(p, idx)) <= 1e-5
    h = 1e-6
    for name in M.PARAM_NAMES:
        assert g[name].shape == p[name].shape
        for flat in rng.choice(p[name].size, 4, replace=False):
            up = {k: (np.array(v, np.float64) if k in M.PARAM_NAMES else v) for k, v in p.items()}
            dn = {k: (np.array(v, np.float64) if k in M.PARAM_NAMES else v) for k, v in p.items()}
            up[name].flat[flat] += h
            dn[name].flat[flat] -= h
            fd = (M.bdh_loss_grads(up, idx, tgt)[0] - M.bdh_loss_grads(dn, idx, tgt)[0]) / (2 * h)
            assert abs(fd - g[name].flat[flat]) <= 1e-6 + 1e-4 * abs(fd), (name, flat, fd, g[name].flat[flat])


def test_harness_eager_train_step_matches_oracle_gradients():
    """The harness's training step (eager attention, fp32 on the CPU): loss and
    every parameter gradient against the float64 oracle at 1e-4."""
    p = M.init_params(2, 32, 2, 64, 11, seed=25)
    m = _model(p, mult=4)
    rng = np.random.default_rng(26)
    idx, tgt = rng.integers(0, 11, (2, 40)), rng.integers(0, 11, (2, 40))
    _, loss = m(torch.from_numpy(idx), torch.from_numpy(tgt), impl="eager")
    loss.backward()
    want_loss, want = M.bdh_loss_grads(p, idx, tgt)
    assert abs(loss.item() - want_loss) <= 1e-5 * abs(want_loss)
    got = {"embed": m.embed.weight.grad, **{k: getattr(m, k).grad for k in M.PARAM_NAMES if k != "embed"}}
    for k in M.PARAM_NAMES:
        assert rel_fro(got[k].numpy(), want[k]) <= 1e-4, k


def test_relu_margin_detects_inputs_near_zero():
    """``relu_margin`` is the smallest |ReLU input| / RMS of the forward: zero when
    an encoder product is exactly 0 (an embedding row orthogonal to an encoder
    column), positive otherwise, and equal for a prefix of a longer draw (causal)."""
    p = M.init_params(1, 8, 2, 8, 5, seed=27)
    idx = np.array([[1, 3, 2, 4]])
    m = M.relu_margin(p, idx)
    assert 0 < m < 1
    assert M.relu_margin(p, np.array([[1, 3, 2, 4, 0, 1]])) <= m
    q = dict(p, encoder=p["encoder"].copy())
    q["encoder"][0, :, 3] = 0.0  # one latent column of head 0 is identically zero
    assert M.relu_margin(q, idx) == 0.0
