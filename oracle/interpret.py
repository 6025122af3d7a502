"""TEST INFRASTRUCTURE ONLY: Float64 meaning of the hot path's programs.

Restates what src/Compiler/program/interpret.jl computes for each program
when fed Float64 (plan-free, products by matrix multiply, half factors
widened and the result rounded once, interpret.jl:58-63).  Arrays are numpy
in the memory order the kernels see.  For the row programs an array of
shape (rows, n), C order, is the reference's n x rows column-major array:
each numpy row is one of the reference's columns, the axis dims = 1 folds.

Pinning (tests/test_oracle_*.py):
- softmax_grad, layernorm_grad, softmax_fwd, layernorm_fwd: central finite
  differences of the loss in float64, torch CPU autograd (a library
  routine), invariants (a softmax column sums to 1; its gradient's column
  sums are 0; a LayerNorm column has mean 0, mean square v/(v+eps); its
  gradient is orthogonal to 1 and to y).
- tanh_layer_grad: closed form z = w'x + b (config 1), finite differences,
  torch autograd, and the reference's own doctest sum(abs2, [1,2,3,4]) = 30.
"""
from __future__ import annotations

import numpy as np


def _f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


def logsumexp_rows(x: np.ndarray) -> np.ndarray:
    """LOGSUMEXP over each row, shifted by lse_shift (folds.jl:194, 263)."""
    x = _f64(x)
    m = x.max(axis=1, keepdims=True)
    sh = np.where(np.isfinite(m), m, 0.0)
    with np.errstate(divide="ignore"):
        return (sh + np.log(np.exp(x - sh).sum(axis=1, keepdims=True)))


def softmax_fwd(x: np.ndarray) -> np.ndarray:
    """softmax_columns(x) = exp.(x .- logsumexp(x; dims = 1)) (test/fixtures/programs.jl:8)."""
    x = _f64(x)
    return np.exp(x - logsumexp_rows(x))


def softmax_grad(x: np.ndarray, g: np.ndarray):
    """loss = sum(softmax_columns(x) .* g) and d loss / d x (programs.jl:74)."""
    y = softmax_fwd(x)
    g = _f64(g)
    dot = (y * g).sum(axis=1, keepdims=True)
    return float(dot.sum()), y * (g - dot)


def layernorm_fwd(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """layernorm(x, 1) (test/fixtures/programs.jl:13-17): two passes, weight 1, bias 0."""
    x = _f64(x)
    n = x.shape[1]
    m = x.sum(axis=1, keepdims=True) / n
    v = ((x - m) ** 2).sum(axis=1, keepdims=True) / n
    return (x - m) / np.sqrt(v + eps)


def layernorm_grad(x: np.ndarray, g: np.ndarray, eps: float = 1e-5):
    """loss = sum(layernorm(x) .* g) and d loss / d x."""
    x = _f64(x)
    g = _f64(g)
    n = x.shape[1]
    m = x.sum(axis=1, keepdims=True) / n
    v = ((x - m) ** 2).sum(axis=1, keepdims=True) / n
    r = 1.0 / np.sqrt(v + eps)
    y = (x - m) * r
    gy = (g * y).sum(axis=1, keepdims=True)
    dx = r * (g - g.mean(axis=1, keepdims=True) - y * gy / n)
    return float(gy.sum()), dx


def tanh_layer_grad(w: np.ndarray, b: np.ndarray, x: np.ndarray):
    """Config 1: loss(w, b, x) = sum(abs2, tanh.(w' * x .+ b)) and (dw, db, dx).

    w is d x h, b h, x d x c as Julia matrices (numpy arrays indexed [i, j]
    the way Julia indexes them; memory order does not matter here)."""
    w, b, x = _f64(w), _f64(b), _f64(x)
    z = w.T @ x + b[:, None]
    y = np.tanh(z)
    loss = float((y * y).sum())
    dz = 2.0 * y * (1.0 - y * y)
    return loss, x @ dz.T, dz.sum(axis=1), w @ dz


GELU_C = 0.7978846
GELU_A = 0.044715


def gelu(x):
    """gelu(x) = x/2 (1 + tanh(0.7978846 (x + 0.044715 x^3))) (test/fixtures/programs.jl:19)."""
    return x / 2 * (1 + np.tanh(GELU_C * (x + GELU_A * x ** 3)))


def gelu_grad(x):
    t = np.tanh(GELU_C * (x + GELU_A * x ** 3))
    return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * GELU_C * (1 + 3 * GELU_A * x * x)


def mlp_grad(W1, b1, W2, b2, x):
    """Config 3: loss = sum(abs2, W2 * gelu.(W1 * x .+ b1) .+ b2) and its gradient
    w.r.t. (W1, b1, W2, b2, x), Julia matrices (W1 hidden x d_in, x d_in x batch,
    W2 d_out x hidden) in float64: the program's meaning with products widened
    and nothing rounded between (interpret.jl:58-63)."""
    W1, b1, W2, b2, x = (np.asarray(a, dtype=np.float64) for a in (W1, b1, W2, b2, x))
    z = W1 @ x + b1[:, None]
    h = gelu(z)
    y = W2 @ h + b2[:, None]
    loss = float((y * y).sum())
    dy = 2 * y
    dW2 = dy @ h.T
    db2 = dy.sum(axis=1)
    dz = (W2.T @ dy) * gelu_grad(z)
    dW1 = dz @ x.T
    db1 = dz.sum(axis=1)
    dx = W1.T @ dz
    return loss, dW1, db1, dW2, db2, dx


def attention_fwd(q, k, v, causal=True, scale=None):
    """attention(q, k, v; causal, scale) of test/fixtures/operations.jl:21-70 in
    float64.  Arrays are numpy (batch, positions, heads, d): the memory of the
    reference's (d, heads, positions, batch) column-major arrays.  Query head h
    reads key/value head h // (heads // kv_heads).  Returns (o, lse), lse
    (batch, positions, heads)."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    B, S, H, D = q.shape
    Hk = k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    kk = np.repeat(k, H // Hk, axis=2)
    vv = np.repeat(v, H // Hk, axis=2)
    s = np.einsum("bmhd,bnhd->bhmn", q, kk) * scale
    if causal:
        mask = np.arange(S)[None, :] > np.arange(S)[:, None]  # key n after query m
        s = np.where(mask[None, None], -np.inf, s)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    o = np.einsum("bhmn,bnhd->bmhd", e / l, vv)
    lse = (m + np.log(l))[..., 0].transpose(0, 2, 1)
    return o, lse


def attention_bwd(q, k, v, dout, causal=True, scale=None):
    """Gradients of sum(attention(q, k, v) .* dout) w.r.t. q, k, v in float64
    (kv_heads == heads), same layout as attention_fwd."""
    q, k, v, dout = (np.asarray(a, dtype=np.float64) for a in (q, k, v, dout))
    B, S, H, D = q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    s = np.einsum("bmhd,bnhd->bhmn", q, k) * scale
    if causal:
        mask = np.arange(S)[None, :] > np.arange(S)[:, None]
        s = np.where(mask[None, None], -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    g = np.einsum("bmhd->bhmd", dout)
    dv = np.einsum("bhmn,bhmd->bnhd", p, g)
    dp = np.einsum("bhmd,bnhd->bhmn", g, v)
    ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True))
    dq = np.einsum("bhmn,bnhd->bmhd", ds, k) * scale
    dk = np.einsum("bhmn,bmhd->bnhd", ds, q) * scale
    return dq, dk, dv
