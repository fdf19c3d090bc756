"""Pins of the oracle's program-level functions (CPU only).

The C oracle restates the configuration programs in binary32/binary64 with
the canonical tree everywhere; these tests hold it against what the
mathematics fixes, computed independently in float64 numpy:

  softmax adjoint   d/dx of <g, softmax(x)> by central finite differences.
  linreg_step       grad = X^T (X w - y) / n and loss = mean((X w - y)^2),
                    and grad = d loss / d w / 2 by finite differences.
  transformer_block an independent float64 forward pass (pre-LN, causal
                    mask, per-head softmax attention, exact GELU via erf)
                    within the f32 rounding of the oracle.
  mlp_train_step    the loss against a float64 forward pass that uses the
                    oracle's own dropout mask, and every parameter update
                    (w - w') / lr against central finite differences of that
                    float64 loss: a dropped term, sign or transposition in
                    the backward pass fails these.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def setup_module(_m):
    O.build()


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-300))


def test_softmax_adjoint_is_the_vjp():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 7))
    g = rng.standard_normal((3, 7))
    y = O.softmax_rows(x)
    dx = O.softmax_adjoint_rows(y, g)

    def f(z):
        e = np.exp(z - z.max(1, keepdims=True))
        return float((g * e / e.sum(1, keepdims=True)).sum())

    eps = 1e-6
    fd = np.zeros_like(x)
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            zp, zm = x.copy(), x.copy()
            zp[i, j] += eps
            zm[i, j] -= eps
            fd[i, j] = (f(zp) - f(zm)) / (2 * eps)
    assert rel(dx, fd) < 1e-7


def test_linreg_step_closed_form_and_gradient():
    rng = np.random.default_rng(1)
    X, w = rng.standard_normal((257, 9)), rng.standard_normal(9)
    y = X @ w + rng.normal(0, 0.1, 257)
    grad, loss = O.linreg_step(X, w, y)
    r = X @ w - y
    assert rel(grad, X.T @ r / 257) < 1e-13
    assert abs(loss - np.mean(r * r)) <= 1e-13 * loss
    eps = 1e-6
    for k in range(9):
        wp, wm = w.copy(), w.copy()
        wp[k] += eps
        wm[k] -= eps
        d = (np.mean((X @ wp - y) ** 2) - np.mean((X @ wm - y) ** 2)) / (2 * eps)
        assert abs(2 * grad[k] - d) <= 1e-6 * max(1.0, abs(d))


def layer_norm64(x, g, b, eps=1e-5):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * g + b


def gelu64(x):
    return x * 0.5 * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))


def transformer64(x, p, heads):
    B, S, D = x.shape
    dh = D // heads
    x = x.astype(np.float64)
    P = {k: v.astype(np.float64) for k, v in p.items()}
    h = layer_norm64(x, P["ln1_g"], P["ln1_b"])
    q, k, v = h @ P["wq"] + P["bq"], h @ P["wk"] + P["bk"], h @ P["wv"] + P["bv"]
    o = np.zeros_like(q)
    mask = np.tril(np.ones((S, S), bool))
    for hd in range(heads):
        sl = slice(hd * dh, (hd + 1) * dh)
        s = q[:, :, sl] @ k[:, :, sl].transpose(0, 2, 1) / math.sqrt(dh)
        s = np.where(mask, s, -np.inf)
        e = np.exp(s - s.max(-1, keepdims=True))
        o[:, :, sl] = (e / e.sum(-1, keepdims=True)) @ v[:, :, sl]
    x1 = x + o @ P["wo"] + P["bo"]
    h2 = layer_norm64(x1, P["ln2_g"], P["ln2_b"])
    return x1 + gelu64(h2 @ P["w1"] + P["b1"]) @ P["w2"] + P["b2"]


def test_transformer_block_against_float64_forward():
    rng = np.random.default_rng(2)
    B, S, D, F, heads = 2, 16, 128, 256, 2
    x = rng.standard_normal((B, S, D)).astype(np.float32)
    p = {}
    for name, shape in (("wq", (D, D)), ("wk", (D, D)), ("wv", (D, D)), ("wo", (D, D)), ("w1", (D, F)), ("w2", (F, D))):
        p[name] = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    for name, n in (("bq", D), ("bk", D), ("bv", D), ("bo", D), ("b1", F), ("b2", D), ("ln1_b", D), ("ln2_b", D)):
        p[name] = (rng.standard_normal(n) * 0.1).astype(np.float32)
    p["ln1_g"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    p["ln2_g"] = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    got = O.transformer_block(x, p, heads)
    assert rel(got, transformer64(x, p, heads)) < 2e-6


def mlp_loss64(x, onehot, w1, b1, w2, b2, mask_scale):
    z1 = x @ w1 + b1
    h = np.maximum(z1, 0) * mask_scale
    z2 = h @ w2 + b2
    z2 = z2 - z2.max(1, keepdims=True)
    logp = z2 - np.log(np.exp(z2).sum(1, keepdims=True))
    return float(-(logp * onehot).sum(1).mean())


def test_mlp_train_step_loss_and_updates_against_finite_differences():
    rng = np.random.default_rng(3)
    B, I, H, Ocls = 16, 12, 8, 5
    x = rng.uniform(0, 1, (B, I)).astype(np.float32)
    onehot = np.eye(Ocls, dtype=np.float32)[rng.integers(0, Ocls, B)]
    w1 = (rng.standard_normal((I, H)) * 0.5).astype(np.float32)
    b1 = (rng.standard_normal(H) * 0.1).astype(np.float32)
    w2 = (rng.standard_normal((H, Ocls)) * 0.5).astype(np.float32)
    b2 = (rng.standard_normal(Ocls) * 0.1).astype(np.float32)
    key, rate, lr = 44, np.float32(0.25), np.float32(0.5)
    loss, w1n, b1n, w2n, b2n = O.mlp_train_step(x, onehot, w1, b1, w2, b2, key, rate, lr)
    # the mask and scale of [05-OP-37]: u = (f32) unit(key, i); kept -> 1/(1-rate)
    units = np.array([np.float32(O.unit(key, i)) for i in range(B * H)], np.float32).reshape(B, H)
    mask_scale = np.where(units < rate, 0.0, 1.0 / (1.0 - float(rate)))
    P = [a.astype(np.float64) for a in (w1, b1, w2, b2)]
    args = lambda ps: (x.astype(np.float64), onehot.astype(np.float64), *ps, mask_scale)  # noqa: E731
    assert abs(loss - mlp_loss64(*args(P))) <= 1e-5 * abs(loss)
    eps = 1e-6
    for pi, new in enumerate((w1n, b1n, w2n, b2n)):
        upd = (P[pi] - new.astype(np.float64)) / float(lr)
        flat = P[pi].reshape(-1)
        for idx in range(0, flat.size, max(1, flat.size // 10)):
            plus = [q.copy() for q in P]
            minus = [q.copy() for q in P]
            plus[pi].reshape(-1)[idx] += eps
            minus[pi].reshape(-1)[idx] -= eps
            fd = (mlp_loss64(*args(plus)) - mlp_loss64(*args(minus))) / (2 * eps)
            assert abs(upd.reshape(-1)[idx] - fd) <= 2e-4 * max(abs(fd), 1e-2), (pi, idx, upd.reshape(-1)[idx], fd)
