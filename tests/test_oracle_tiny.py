"""Config 1's oracle: loss(w, b, x) = sum(abs2, tanh.(w'x .+ b)) and its
gradient, against torch autograd, central differences and brute force."""
import numpy as np
import torch

from oracle import floor, interpret
from oracle.data import data, relative


def _inputs():
    return data(32, 64), data(64, scale=0.3), data(32, 16, scale=0.7)


def test_matches_torch_autograd():
    w, b, x = _inputs()
    loss, dw, db, dx = interpret.tanh_layer_grad(w, b, x)
    wt, bt, xt = (torch.tensor(a, requires_grad=True) for a in (w, b, x))
    lt = (torch.tanh(wt.T @ xt + bt[:, None]) ** 2).sum()
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12 * loss
    for a, t in ((dw, wt), (db, bt), (dx, xt)):
        assert relative(a, t.grad.numpy()) < 1e-12


def test_brute_force_loss_and_central_difference():
    rng = np.random.default_rng(2)
    w, b, x = rng.normal(size=(3, 4)), rng.normal(size=4), rng.normal(size=(3, 2))
    loss = 0.0
    for j in range(4):
        for c in range(2):
            z = sum(w[i, j] * x[i, c] for i in range(3)) + b[j]
            loss += np.tanh(z) ** 2
    l, dw, db, dx = interpret.tanh_layer_grad(w, b, x)
    assert abs(l - loss) < 1e-13
    h = 1e-6
    for arr, grad in ((w, dw), (b, db), (x, dx)):
        fd = np.zeros_like(arr)
        for idx in np.ndindex(*arr.shape):
            p = arr.copy()
            p[idx] += h
            lp = interpret.tanh_layer_grad(*(p if a is arr else a for a in (w, b, x)))[0]
            p[idx] -= 2 * h
            lm = interpret.tanh_layer_grad(*(p if a is arr else a for a in (w, b, x)))[0]
            fd[idx] = (lp - lm) / (2 * h)
        assert relative(grad, fd) < 1e-7


def test_floor_float32_is_close_to_float64():
    w, b, x = _inputs()
    l32, dw32, db32, dx32 = floor.tanh_layer_grad(w, b, x)
    l64, dw64, db64, dx64 = interpret.tanh_layer_grad(w, b, x)
    assert abs(l32 - l64) < 1e-5 * l64
    for a, r in ((dw32, dw64), (db32, db64), (dx32, dx64)):
        assert relative(a, r) < 1e-5
