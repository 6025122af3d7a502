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


def product(a, b, d=None):
    """contract(A, B, (1, 3, 4), (3, 2, 4), (1, 2, 4)) (+ D): A (m, k[, batch])
    times B (k, n[, batch]) per batch, Julia axes, factors widened to float64
    and nothing rounded (program/interpret.jl:58-63; ext/cuBLASExt.jl:23-25)."""
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    c = np.einsum("mk...,kn...->mn...", a, b)
    return c if d is None else c + np.asarray(d, dtype=np.float64)


def linear_bias_gelu_grad(w, x, b):
    """The fixture "linear, bias, GELU" (test/fixtures/programs.jl:83):
    loss = sum(abs2, gelu.(w * x .+ b)) and its gradient w.r.t. (w, x, b)."""
    w, x, b = (np.asarray(v, dtype=np.float64) for v in (w, x, b))
    z = w @ x + b[:, None]
    y = gelu(z)
    dz = 2 * y * gelu_grad(z)
    return float((y * y).sum()), dz @ x.T, w.T @ dz, dz.sum(axis=1)


def tanh_mlp_grad(x, w1, b1, w2, b2):
    """The fixture "MLP" (test/fixtures/programs.jl:17,79): loss =
    sum(abs2, w2 * tanh.(w1 * x .+ b1) .+ b2) and its gradient w.r.t.
    (x, w1, b1, w2, b2), with tanh' = 1 - y^2 (program/differentiate.jl:106-155)."""
    x, w1, b1, w2, b2 = (np.asarray(v, dtype=np.float64) for v in (x, w1, b1, w2, b2))
    h = np.tanh(w1 @ x + b1[:, None])
    y = w2 @ h + b2[:, None]
    dy = 2 * y
    dz = (w2.T @ dy) * (1 - h * h)
    return float((y * y).sum()), w1.T @ dz, dz @ x.T, dz.sum(axis=1), dy @ h.T, dy.sum(axis=1)


def attention_visible(B, S, Sk, causal=True, starts=None, lengths=None):
    """Which keys each query sees, (batch, 1, queries, keys): key n (0-based) is
    seen by query m of batch b when n < lengths[b], n >= starts[b, m] - 1
    (1-based starts: documents packed in sequences) and, causal, n <= m --
    the masks of test/cuda/attention.jl:218-271 and the causal formula of
    test/fixtures/operations.jl:21-70."""
    n = np.arange(Sk)[None, None, None, :]
    m = np.arange(S)[None, None, :, None]
    seen = np.ones((B, 1, S, Sk), dtype=bool)
    if causal:
        seen &= n <= m
    if starts is not None:
        seen &= n >= np.asarray(starts).reshape(B, 1, S, 1) - 1
    if lengths is not None:
        seen &= n < np.asarray(lengths).reshape(B, 1, 1, 1)
    return seen


def attention_fwd(q, k, v, causal=True, scale=None, starts=None, lengths=None):
    """attention(q, k, v; causal, scale) of test/fixtures/operations.jl:21-70 in
    float64.  Arrays are numpy (batch, positions, heads, d): the memory of the
    reference's (d, heads, positions, batch) column-major arrays; k and v may
    hold another number of positions than q.  Query head h reads key/value
    head h // (heads // kv_heads).  starts (batch, positions), lengths (batch):
    the device-held masks of attention_visible.  Returns (o, lse), lse
    (batch, positions, heads)."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    B, S, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    kk = np.repeat(k, H // Hk, axis=2)
    vv = np.repeat(v, H // Hk, axis=2)
    s = np.einsum("bmhd,bnhd->bhmn", q, kk) * scale
    s = np.where(attention_visible(B, S, Sk, causal, starts, lengths), s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore", divide="ignore"):
        o = np.einsum("bhmn,bnhd->bmhd", e / l, vv)
        lse = (m + np.log(l))[..., 0].transpose(0, 2, 1)
    return o, lse


def attention_bwd(q, k, v, dout, causal=True, scale=None, starts=None, lengths=None):
    """Gradients of sum(attention(q, k, v) .* dout) w.r.t. q, k, v in float64,
    same layout and masks as attention_fwd.  With grouped heads the key and
    value gradients sum over the query heads of a group
    (test/cuda/attention.jl:132-140)."""
    q, k, v, dout = (np.asarray(a, dtype=np.float64) for a in (q, k, v, dout))
    B, S, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    k = np.repeat(k, H // Hk, axis=2)
    v = np.repeat(v, H // Hk, axis=2)
    s = np.einsum("bmhd,bnhd->bhmn", q, k) * scale
    s = np.where(attention_visible(B, S, Sk, causal, starts, lengths), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    g = np.einsum("bmhd->bhmd", dout)
    dv = np.einsum("bhmn,bhmd->bnhd", p, g)
    dp = np.einsum("bhmd,bnhd->bhmn", g, v)
    ds = p * (dp - (dp * p).sum(axis=-1, keepdims=True))
    dq = np.einsum("bhmn,bnhd->bmhd", ds, k) * scale
    dk = np.einsum("bhmn,bmhd->bnhd", ds, q) * scale
    # Query head h = hk * (H // Hk) + g reads kv head hk: sum over g.
    dk = dk.reshape(B, Sk, Hk, H // Hk, D).sum(axis=3)
    dv = dv.reshape(B, Sk, Hk, H // Hk, D).sum(axis=3)
    return dq, dk, dv


# ---- config 5: gated DeltaNet -------------------------------------------------------
# Arrays are numpy (batch, positions, heads, d) for q, k, v, o and (batch,
# positions, heads) for the log-gates a and the strengths beta: the memory of
# the program's (d, heads, positions, batch) and (heads, positions, batch)
# column-major arrays.


def deltanet_sequential(q, k, v, a, beta):
    """The gated delta rule token by token (examples/deltanet.jl:89-101):
    S = exp(a) (I - beta k k') S + beta k v', o = S' q, S starting at zero."""
    q, k, v, a, beta = (np.asarray(x, dtype=np.float64) for x in (q, k, v, a, beta))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    o = np.zeros((B, T, H, dv))
    S = np.zeros((B, H, dk, dv))
    for t in range(T):
        kt, vt, qt = k[:, t], v[:, t], q[:, t]                      # (B, H, d)
        bt, gt = beta[:, t][..., None, None], np.exp(a[:, t])[..., None, None]
        kS = np.einsum("bhk,bhkv->bhv", kt, S)
        S = gt * (S - bt * kt[..., :, None] * kS[..., None, :]) + bt * kt[..., :, None] * vt[..., None, :]
        o[:, t] = np.einsum("bhkv,bhk->bhv", S, qt)
    return o


def _chunks(x, C):
    """(B, T, H, ...) -> (B, H, N, C, ...)."""
    B, T, H = x.shape[:3]
    y = x.reshape((B, T // C, C, H) + x.shape[3:])
    return np.moveaxis(y, 3, 1)


def _unchunks(y):
    """(B, H, N, C, ...) -> (B, T, H, ...)."""
    B, H, N, C = y.shape[:4]
    return np.moveaxis(y, 1, 3).reshape((B, N * C, H) + y.shape[4:])


def _chunk_prep(q, k, v, a, beta, C):
    """The chunk-local quantities of examples/deltanet.jl:58-86 (WY form)."""
    Q, K, V = _chunks(q, C), _chunks(k, C), _chunks(v, C)          # (B, H, N, C, d)
    A_, Bt = _chunks(a, C), _chunks(beta, C)                      # (B, H, N, C)
    ca = np.cumsum(A_, axis=-1)
    gam = np.exp(ca[..., :, None] - ca[..., None, :])            # Gamma[i, j] = exp(ca_i - ca_j)
    strict = np.tril(np.ones((C, C)), -1)
    lower = np.tril(np.ones((C, C)))
    G = K @ np.swapaxes(K, -1, -2)
    Am = Bt[..., :, None] * gam * G * strict
    T_ = np.linalg.inv(np.eye(C) + Am)
    X = (Bt * np.exp(ca))[..., None] * K
    Y = Bt[..., None] * V
    W, Ut = T_ @ X, T_ @ Y
    QK = Q @ np.swapaxes(K, -1, -2)
    P = gam * QK * lower
    Qg = np.exp(ca)[..., None] * Q
    Kd = np.exp(ca[..., -1:] - ca)[..., None] * K
    g = np.exp(ca[..., -1])
    return dict(Q=Q, K=K, V=V, Bt=Bt, ca=ca, gam=gam, G=G, T=T_, X=X, Y=Y, W=W, Ut=Ut, QK=QK, P=P, Qg=Qg, Kd=Kd,
                g=g, strict=strict, lower=lower)


def deltanet_chunked(q, k, v, a, beta, C=64, keep=False):
    """The chunked form (examples/deltanet.jl:58-86): within a chunk products,
    across chunks the state S carried: U = U~ - W S, O = Qg S + P U,
    S <- g S + Kd' U."""
    c = _chunk_prep(q, k, v, a, beta, C)
    B, H, N = c["Q"].shape[:3]
    dk, dv = c["K"].shape[-1], c["V"].shape[-1]
    S = np.zeros((B, H, dk, dv))
    O = np.zeros(c["V"].shape)
    Ss, Us = [], []
    for n in range(N):
        Ss.append(S)
        U = c["Ut"][:, :, n] - c["W"][:, :, n] @ S
        Us.append(U)
        O[:, :, n] = c["Qg"][:, :, n] @ S + c["P"][:, :, n] @ U
        S = c["g"][:, :, n][..., None, None] * S + np.swapaxes(c["Kd"][:, :, n], -1, -2) @ U
    o = _unchunks(O)
    if keep:
        c.update(S=np.stack(Ss, axis=2), U=np.stack(Us, axis=2))
        return o, c
    return o


def deltanet_grad(q, k, v, a, beta, do, C=64):
    """Gradients of sum(deltanet(q, k, v, a, beta) .* do) w.r.t. q, k, v, a
    and beta, in float64: the reverse of the chunked form (state gradient
    swept back over chunks, then each chunk's products, the WY inverse
    T = (I + A)^-1 (dA = -T' dT T'), the decays exp(ca_i - ca_j) and the
    within-chunk cumulative sum of a)."""
    o, c = deltanet_chunked(q, k, v, a, beta, C, keep=True)
    dO = _chunks(np.asarray(do, dtype=np.float64), C)
    B, H, N = dO.shape[:3]
    dk = c["K"].shape[-1]
    dv = dO.shape[-1]
    tr = lambda x: np.swapaxes(x, -1, -2)  # noqa: E731
    dS = np.zeros((B, H, dk, dv))
    dU = np.zeros_like(c["U"])
    dSn = np.zeros_like(c["S"])  # gradient at each chunk's end state S_{n+1}
    for n in reversed(range(N)):
        dSn[:, :, n] = dS
        du = tr(c["P"][:, :, n]) @ dO[:, :, n] + c["Kd"][:, :, n] @ dS
        dU[:, :, n] = du
        dS = tr(c["Qg"][:, :, n]) @ dO[:, :, n] + c["g"][:, :, n][..., None, None] * dS - tr(c["W"][:, :, n]) @ du
    S, U = c["S"], c["U"]
    dQg = dO @ tr(S)
    dP = (dO @ tr(U)) * c["lower"]
    dKd = U @ tr(dSn)
    dg = np.einsum("bhnkv,bhnkv->bhn", S, dSn)
    dW = -dU @ tr(S)
    dUt = dU
    T_ = c["T"]
    dT = dW @ tr(c["X"]) + dUt @ tr(c["Y"])
    dX = tr(T_) @ dW
    dY = tr(T_) @ dUt
    dA = -(tr(T_) @ dT @ tr(T_)) * c["strict"]
    Bt, ca, gam, G, K, Q, V = c["Bt"], c["ca"], c["gam"], c["G"], c["K"], c["Q"], c["V"]
    dG = dA * Bt[..., :, None] * gam
    dQK = dP * gam
    dQ = np.exp(ca)[..., None] * dQg + dQK @ K
    dK = tr(dQK) @ Q + (dG + tr(dG)) @ K + (Bt * np.exp(ca))[..., None] * dX + np.exp(ca[..., -1:] - ca)[..., None] * dKd
    dV = Bt[..., None] * dY
    dBt = (dA * gam * G).sum(-1) + np.exp(ca) * (K * dX).sum(-1) + (V * dY).sum(-1)
    dgam = dA * Bt[..., :, None] * G + dP * c["QK"]
    w = dgam * gam
    dca = w.sum(-1) - w.sum(-2)
    dca += Bt * np.exp(ca) * (K * dX).sum(-1)
    dca += np.exp(ca) * (Q * dQg).sum(-1)
    kd = np.exp(ca[..., -1:] - ca) * (K * dKd).sum(-1)
    dca -= kd
    dca[..., -1] += kd.sum(-1) + dg * c["g"]
    da = np.flip(np.cumsum(np.flip(dca, -1), -1), -1)
    return _unchunks(dQ), _unchunks(dK), _unchunks(dV), _unchunks(da), _unchunks(dBt)
