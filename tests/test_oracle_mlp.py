"""Config 3's oracle (the 2-layer MLP's loss and gradient) and the bf16
rounding it feeds the kernels, against torch: autograd in float64, and
torch's own float32 -> bfloat16 conversion."""
import numpy as np
import torch

from oracle import interpret
from oracle.data import bf16_bits, bf16_round, bf16_value, relative


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(size=10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
                                  3.3895314e38], dtype=np.float32)]).astype(np.float32)
    ours = bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(bf16_value(ours), torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    # Ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7.
    assert bf16_round(np.float32(1.0 + 2.0 ** -8)) == 1.0


def test_mlp_grad_matches_torch_autograd():
    rng = np.random.default_rng(1)
    h, d, b, o = 12, 6, 5, 4
    W1, b1, W2, b2, x = (rng.normal(size=s) for s in ((h, d), h, (o, h), o, (d, b)))
    loss, dW1, db1, dW2, db2, dx = interpret.mlp_grad(W1, b1, W2, b2, x)
    t = [torch.tensor(a, requires_grad=True) for a in (W1, b1, W2, b2, x)]
    gelu = lambda z: z / 2 * (1 + torch.tanh(0.7978846 * (z + 0.044715 * z ** 3)))  # noqa: E731
    y = t[2] @ gelu(t[0] @ t[4] + t[1][:, None]) + t[3][:, None]
    lt = (y * y).sum()
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12 * loss
    for ours, tt in zip((dW1, db1, dW2, db2, dx), t):
        assert relative(ours, tt.grad.numpy()) < 1e-12


def test_gelu_grad_central_difference():
    z = np.linspace(-6, 6, 101)
    eps = 1e-6
    fd = (interpret.gelu(z + eps) - interpret.gelu(z - eps)) / (2 * eps)
    assert np.max(np.abs(fd - interpret.gelu_grad(z))) < 1e-8
