"""numpy restatement of the reference BDH forward, for checking the model harness.

TEST INFRASTRUCTURE ONLY: tests and ``bench.py``'s ``cpu_baseline`` are the
only callers.  fp32 throughout (the reference's CPU math).

Follows bdh_baseline.py:109-151 (the reference's plain model, which
bdh.py:947-1072 equals bit for bit at dropout 0 per the reference's
tests/test_vs_baseline.py:201-234):

    x = LN(embed[idx])                                       (B, T, D)
    per layer:
        x_sparse = relu(x @ encoder)                         (B, nh, T, N)
        yKV      = LN(tril(R(x_sparse) R(x_sparse)^T, -1) @ x)
        y_sparse = relu(yKV @ encoder_v)                     (B, nh, T, N)
        yMLP     = (x_sparse * y_sparse) as (B, T, nh*N), index h*N + n, @ decoder
        x        = LN(x + LN(yMLP))
    logits = x @ lm_head

LayerNorm has no affine and eps 1e-5 (bdh_baseline.py:92).  R is BDH's RoPE
with positions 0..T-1 (bdh_baseline.py:53-66).

Pinned (tests/test_harness.py) by: a pure-Python loop model on tiny shapes;
the T = 1 closed form (attention is empty, so every layer reduces to
x <- LN(x)); the encoder_v = 0 closed form; causality (logits at t do not
depend on later tokens); LayerNorm's mean 0 / variance 1.

``bdh_loss_grads`` is the same formula in float64 torch on the CPU, for the
gradients of the training loss (cross entropy over all positions, as
bdh_baseline.py:147-150 and train.py:997-1034 compute it) by autograd.  Its
logits are pinned to ``bdh_forward`` and its gradients to central finite
differences (tests/test_harness.py).
"""

from __future__ import annotations

import math
from typing import Dict

import numpy as np

from . import tril_attn_oracle as A

__all__ = ["layer_norm", "bdh_forward", "bdh_forward_loops", "bdh_loss_grads", "init_params"]


def layer_norm(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """LayerNorm over the last axis without affine (bdh_baseline.py:92)."""
    x = np.asarray(x, np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return ((x - mu) / np.sqrt(var + eps)).astype(np.float32)


def init_params(n_layer: int, D: int, nh: int, N: int, V: int, seed: int = 0) -> Dict[str, np.ndarray]:
    """N(0, 0.02^2) weights of the shapes of bdh_baseline.py:80-102."""
    rng = np.random.default_rng(seed)

    def w(*shape):
        return (0.02 * rng.standard_normal(shape)).astype(np.float32)

    return {"embed": w(V, D), "encoder": w(nh, D, N), "encoder_v": w(nh, D, N),
            "decoder": w(nh * N, D), "lm_head": w(D, V), "n_layer": n_layer}


def bdh_forward(p: Dict[str, np.ndarray], idx: np.ndarray) -> np.ndarray:
    """Logits (B, T, V) of bdh_baseline.py:109-151 (dropout off)."""
    idx = np.asarray(idx)
    B, T = idx.shape
    nh, D, N = p["encoder"].shape
    freqs = A.get_freqs(N)
    x = layer_norm(p["embed"][idx])  # (B, T, D)
    for _ in range(int(p["n_layer"])):
        xs = np.maximum(np.matmul(x[:, None], p["encoder"][None]), 0).astype(np.float32)  # (B, nh, T, N)
        ykv, _ = A.tril_rope_score_v(xs, x[:, None], freqs, 0)
        ykv = layer_norm(ykv)
        ys = np.maximum(np.matmul(ykv, p["encoder_v"][None]), 0).astype(np.float32)
        xy = (xs * ys).transpose(0, 2, 1, 3).reshape(B, T, nh * N)
        y = layer_norm(np.matmul(xy, p["decoder"]))
        x = layer_norm(x + y)
    return np.matmul(x, p["lm_head"]).astype(np.float32)


def bdh_forward_loops(p: Dict[str, np.ndarray], idx) -> np.ndarray:
    """The same model with explicit loops over every index (tiny shapes only), in float64."""
    idx = [list(r) for r in np.asarray(idx)]
    B, T = len(idx), len(idx[0])
    nh, D, N = p["encoder"].shape
    V = p["lm_head"].shape[1]
    f = [float(v) for v in A.get_freqs(N)]

    def ln(vec):
        mu = sum(vec) / len(vec)
        var = sum((a - mu) ** 2 for a in vec) / len(vec)
        return [(a - mu) / math.sqrt(var + 1e-5) for a in vec]

    def rot(row, t):
        out = [0.0] * N
        for i in range(0, N, 2):
            a0 = (t * f[i] % 1.0) * 2 * math.pi
            a1 = (t * f[i + 1] % 1.0) * 2 * math.pi
            out[i] = row[i] * math.cos(a0) - row[i + 1] * math.sin(a0)
            out[i + 1] = row[i + 1] * math.cos(a1) + row[i] * math.sin(a1)
        return out

    E, W, Wv, Dec, H = (p[k].astype(np.float64) for k in ("embed", "encoder", "encoder_v", "decoder", "lm_head"))
    logits = np.zeros((B, T, V))
    for b in range(B):
        x = [ln([E[idx[b][t], d] for d in range(D)]) for t in range(T)]
        for _ in range(int(p["n_layer"])):
            xs = [[[max(0.0, sum(x[t][d] * W[h, d, n] for d in range(D))) for n in range(N)]
                   for t in range(T)] for h in range(nh)]
            new_x = []
            ys_all = []
            for h in range(nh):
                r = [rot(xs[h][t], t) for t in range(T)]
                ykv = []
                for i in range(T):
                    acc = [0.0] * D
                    for j in range(i):
                        s = sum(r[i][n] * r[j][n] for n in range(N))
                        for d in range(D):
                            acc[d] += s * x[j][d]
                    ykv.append(ln(acc))
                ys_all.append([[max(0.0, sum(ykv[t][d] * Wv[h, d, n] for d in range(D))) for n in range(N)]
                               for t in range(T)])
            for t in range(T):
                ymlp = [sum(xs[h][t][n] * ys_all[h][t][n] * Dec[h * N + n, d] for h in range(nh) for n in range(N))
                        for d in range(D)]
                y = ln(ymlp)
                new_x.append(ln([x[t][d] + y[d] for d in range(D)]))
            x = new_x
        for t in range(T):
            for v in range(V):
                logits[b, t, v] = sum(x[t][d] * H[d, v] for d in range(D))
    return logits.astype(np.float32)


PARAM_NAMES = ("embed", "encoder", "encoder_v", "decoder", "lm_head")


def bdh_loss_grads(p: Dict[str, np.ndarray], idx, targets, *, return_logits: bool = False):
    """Loss and parameter gradients of bdh_baseline.py:109-151 in float64 (CPU torch autograd).

    The loss is the mean cross entropy over every position (bdh_baseline.py:147-150).
    RoPE's cos/sin are the oracle's fp32 tables (constants of the parameters),
    the rotation and every product in float64.  Returns ``(loss, grads)`` with
    ``grads[name]`` a float64 array of each parameter's shape (``embed`` is the
    embedding table), plus the logits when ``return_logits``.
    """
    import torch

    idx = torch.as_tensor(np.asarray(idx), dtype=torch.long)
    tgt = torch.as_tensor(np.asarray(targets), dtype=torch.long)
    B, T = idx.shape
    nh, D, N = p["encoder"].shape
    w = {k: torch.tensor(np.asarray(p[k], np.float64), requires_grad=True) for k in PARAM_NAMES}
    cos, sin = (torch.from_numpy(a.astype(np.float64)) for a in A.rope_cos_sin(T, 0, A.get_freqs(N)))

    def ln(t):
        mu = t.mean(-1, keepdim=True)
        var = ((t - mu) ** 2).mean(-1, keepdim=True)
        return (t - mu) / torch.sqrt(var + 1e-5)

    def rot(t):
        t0, t1 = t[..., 0::2], t[..., 1::2]
        y0 = t0 * cos[:, 0::2] - t1 * sin[:, 0::2]
        y1 = t1 * cos[:, 1::2] + t0 * sin[:, 1::2]
        return torch.stack((y0, y1), -1).flatten(-2)

    x = ln(w["embed"][idx])
    mask = torch.ones(T, T, dtype=torch.float64).tril(-1)
    for _ in range(int(p["n_layer"])):
        xs = torch.relu(torch.matmul(x[:, None], w["encoder"][None]))  # (B, nh, T, N)
        r = rot(xs)
        ykv = ln(torch.matmul(torch.matmul(r, r.transpose(-2, -1)) * mask, x[:, None]))
        ys = torch.relu(torch.matmul(ykv, w["encoder_v"][None]))
        xy = (xs * ys).permute(0, 2, 1, 3).reshape(B, T, nh * N)
        x = ln(x + ln(torch.matmul(xy, w["decoder"])))
    logits = torch.matmul(x, w["lm_head"])
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.size(-1)), tgt.reshape(-1))
    loss.backward()
    grads = {k: w[k].grad.numpy() for k in PARAM_NAMES}
    if return_logits:
        return float(loss.detach()), grads, logits.detach().numpy()
    return float(loss.detach()), grads


def relu_margin(p: Dict[str, np.ndarray], idx) -> float:
    """Smallest |z| / rms(z) over the inputs z of every ReLU of the forward
    (x_sparse and y_sparse of each layer), in float64.

    A ReLU input closer to zero than the rounding of its fp32 product can take
    the other branch in another summation order, and that one element then
    moves the gradients upstream of it far beyond fp32 roundoff.  An fp32
    gradient comparison is well posed when this margin is well above the
    products' relative rounding (~1e-7 here).
    """
    idx = np.asarray(idx)
    nh, D, N = p["encoder"].shape
    f64 = {k: np.asarray(p[k], np.float64) for k in PARAM_NAMES}
    cos, sin = (a.astype(np.float64) for a in A.rope_cos_sin(idx.shape[1], 0, A.get_freqs(N)))

    def ln(t):
        mu = t.mean(-1, keepdims=True)
        return (t - mu) / np.sqrt(((t - mu) ** 2).mean(-1, keepdims=True) + 1e-5)

    def margin(z):
        return float(np.abs(z).min() / np.sqrt((z * z).mean()))

    T = idx.shape[1]
    mask = np.tril(np.ones((T, T)), -1)
    x = ln(f64["embed"][idx])
    worst = np.inf
    for _ in range(int(p["n_layer"])):
        z = np.matmul(x[:, None], f64["encoder"][None])
        worst = min(worst, margin(z))
        xs = np.maximum(z, 0)
        r = np.empty_like(xs)
        r[..., 0::2] = xs[..., 0::2] * cos[:, 0::2] - xs[..., 1::2] * sin[:, 0::2]
        r[..., 1::2] = xs[..., 1::2] * cos[:, 1::2] + xs[..., 0::2] * sin[:, 1::2]
        ykv = ln(np.matmul(np.matmul(r, np.swapaxes(r, -1, -2)) * mask, x[:, None]))
        zv = np.matmul(ykv, f64["encoder_v"][None])
        # rows whose attention is empty (position 0) are exact zeros in every order
        live = np.abs(zv).max(-1) > 0
        worst = min(worst, margin(zv[live]) if live.any() else np.inf)
        xy = (xs * np.maximum(zv, 0)).transpose(0, 2, 1, 3).reshape(idx.shape[0], T, nh * N)
        x = ln(x + ln(np.matmul(xy, f64["decoder"])))
    return worst
