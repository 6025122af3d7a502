"""The row programs' oracle (softmax and LayerNorm, forward and gradient)
against what fixes it: torch CPU autograd, central differences in float64,
and the invariants of each function; the Float32 floor against the Float64
interpreter."""
import numpy as np
import pytest
import torch

from oracle import floor, interpret
from oracle.data import data, relative


def _ln_torch(x, eps):
    m = x.mean(dim=1, keepdim=True)
    v = ((x - m) ** 2).mean(dim=1, keepdim=True)
    return (x - m) / torch.sqrt(v + eps)


@pytest.mark.parametrize("rows,n", [(6, 8), (3, 700), (5, 33)])
def test_softmax_grad_matches_torch_autograd(rows, n):
    x = data(n, rows).T.copy()
    g = data(n, rows, scale=0.7).T.copy()
    loss, dx = interpret.softmax_grad(x, g)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    lt = (torch.softmax(xt, dim=1) * torch.tensor(g)).sum()
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12 * max(1, abs(loss))
    assert relative(dx, xt.grad.numpy()) < 1e-12


@pytest.mark.parametrize("rows,n", [(6, 8), (3, 700), (5, 33)])
def test_layernorm_grad_matches_torch_autograd(rows, n):
    x = data(n, rows).T.copy()
    g = data(n, rows, scale=0.7).T.copy()
    loss, dx = interpret.layernorm_grad(x, g, 1e-5)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    lt = (_ln_torch(xt, 1e-5) * torch.tensor(g)).sum()
    lt.backward()
    assert abs(loss - lt.item()) < 1e-11 * max(1, abs(loss))
    assert relative(dx, xt.grad.numpy()) < 1e-11
    assert relative(interpret.layernorm_fwd(x), torch.nn.functional.layer_norm(
        torch.tensor(x), (n,), eps=1e-5).numpy()) < 1e-12


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
def test_gradients_match_central_differences(which):
    rng = np.random.default_rng(3)
    x = rng.normal(size=(2, 9))
    g = rng.normal(size=(2, 9))
    f = interpret.softmax_grad if which == "softmax" else interpret.layernorm_grad
    _, dx = f(x, g)
    h = 1e-6
    fd = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd[idx] = (f(xp, g)[0] - f(xm, g)[0]) / (2 * h)
    assert relative(dx, fd) < 1e-7


def test_invariants():
    rng = np.random.default_rng(0)
    x = rng.normal(size=(4, 64)) * 3
    g = rng.normal(size=(4, 64))
    y = interpret.softmax_fwd(x)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-14)
    _, dx = interpret.softmax_grad(x, g)
    assert np.allclose(dx.sum(axis=1), 0.0, atol=1e-13)  # sum_j y_j (g_j - <y,g>) = 0
    y = interpret.layernorm_fwd(x)
    assert np.allclose(y.mean(axis=1), 0.0, atol=1e-13)
    _, dx = interpret.layernorm_grad(x, g)
    assert np.allclose(dx.sum(axis=1), 0.0, atol=1e-12)
    # sum(dx .* y) = r * sum(g .* y) * (1 - mean(y .^ 2)), mean(y .^ 2) = v / (v + eps).
    v = x.var(axis=1)
    r = 1 / np.sqrt(v + 1e-5)
    expect = r * (g * y).sum(axis=1) * (1e-5 / (v + 1e-5))
    assert np.allclose((dx * y).sum(axis=1), expect, rtol=1e-6, atol=1e-13)


def test_all_minus_inf_column_and_shift():
    # An all -Inf column sums to zero (lse_shift); its softmax is NaN as
    # exp(-Inf - (-Inf)) is, on every implementation.
    x = np.array([[0.0, 1.0, 2.0], [-np.inf, -np.inf, -np.inf]])
    with np.errstate(invalid="ignore"):
        lse = interpret.logsumexp_rows(x)
    assert lse[1, 0] == -np.inf and np.isclose(lse[0, 0], np.log(np.exp([0, 1, 2]).sum()))


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
@pytest.mark.parametrize("rows,n", [(6, 8), (7, 700), (3, 8192), (2, 9001)])
def test_floor_float32_is_close_to_float64(which, rows, n):
    rng = np.random.default_rng(1)
    x = rng.normal(size=(rows, n)).astype(np.float32)
    g = rng.normal(size=(rows, n)).astype(np.float32)
    if which == "softmax":
        l32, d32 = floor.softmax_grad(x, g)
        l64, d64 = interpret.softmax_grad(x, g)
        y32, y64 = floor.softmax_fwd(x), interpret.softmax_fwd(x)
    else:
        l32, d32 = floor.layernorm_grad(x, g)
        l64, d64 = interpret.layernorm_grad(x, g)
        y32, y64 = floor.layernorm_fwd(x), interpret.layernorm_fwd(x)
    assert relative(d32, d64) < 2e-5
    assert relative(y32, y64) < 2e-5
    assert abs(l32 - l64) < 1e-4 * max(1.0, np.abs(d64).sum() / rows)


def test_bench_parity_reference_matches_the_oracle():
    """bench.py checks config 2's sampled rows against its own float64 torch
    gradient (it leaves the oracle to its CPU baseline): that gradient is
    the oracle's, to rounding."""
    import numpy as np
    import torch

    import bench
    from oracle import interpret
    from oracle.data import relative
    rng = np.random.default_rng(11)
    x, g = rng.standard_normal((4, 300)) * 2, rng.standard_normal((4, 300))
    for name, f in (("softmax", interpret.softmax_grad), ("layernorm", interpret.layernorm_grad)):
        got = bench.rows_grad_exact(name, torch.from_numpy(x), torch.from_numpy(g)).numpy()
        assert relative(got, f(x, g)[1]) < 1e-12, name
