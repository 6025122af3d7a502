"""Config 5's oracle: the chunked gated DeltaNet equals the rule token by
token, and its hand-derived gradient equals torch autograd of that rule."""
import numpy as np
import pytest
import torch

from oracle import interpret
from oracle.data import relative


def _inputs(B, T, H, d, seed):
    rng = np.random.default_rng(seed)
    unit = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)  # noqa: E731
    q, k = unit(rng.normal(size=(B, T, H, d))), unit(rng.normal(size=(B, T, H, d)))
    v = rng.normal(size=(B, T, H, d))
    a = -np.log1p(np.exp(rng.normal(size=(B, T, H))))          # log of exp(-softplus(x))
    beta = 1 / (1 + np.exp(-rng.normal(size=(B, T, H))))
    return q, k, v, a, beta


@pytest.mark.parametrize("C", [4, 8, 16])
def test_chunked_equals_token_by_token(C):
    q, k, v, a, beta = _inputs(2, 32, 3, 8, 0)
    assert relative(interpret.deltanet_chunked(q, k, v, a, beta, C), interpret.deltanet_sequential(q, k, v, a, beta)) < 1e-12


def _torch_sequential(q, k, v, a, beta):
    B, T, H, d = q.shape
    S = torch.zeros(B, H, d, v.shape[-1], dtype=q.dtype)
    out = []
    for t in range(T):
        kt, vt, qt = k[:, t], v[:, t], q[:, t]
        bt, gt = beta[:, t][..., None, None], torch.exp(a[:, t])[..., None, None]
        kS = torch.einsum("bhk,bhkv->bhv", kt, S)
        S = gt * (S - bt * kt[..., :, None] * kS[..., None, :]) + bt * kt[..., :, None] * vt[..., None, :]
        out.append(torch.einsum("bhkv,bhk->bhv", S, qt))
    return torch.stack(out, dim=1)


@pytest.mark.parametrize("C", [4, 8])
def test_gradient_matches_autograd_of_the_rule(C):
    q, k, v, a, beta = _inputs(1, 16, 2, 6, 1)
    do = np.random.default_rng(2).normal(size=v.shape)
    ts = [torch.tensor(x, requires_grad=True) for x in (q, k, v, a, beta)]
    (_torch_sequential(*ts) * torch.tensor(do)).sum().backward()
    ours = interpret.deltanet_grad(q, k, v, a, beta, do, C)
    for name, g, t in zip(("dq", "dk", "dv", "da", "dbeta"), ours, ts):
        assert relative(g, t.grad.numpy()) < 1e-10, name


def test_no_decay_no_strength_leaves_state_empty():
    # beta = 0: nothing is written, every output is zero.
    q, k, v, a, _ = _inputs(1, 8, 1, 4, 3)
    assert np.all(interpret.deltanet_sequential(q, k, v, a, np.zeros_like(a)) == 0)
