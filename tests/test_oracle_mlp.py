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


def test_fixture_programs_with_products_match_torch_autograd():
    """"linear, bias, GELU" and "MLP" (test/fixtures/programs.jl:79,83) at
    their shapes: loss and every gradient against torch's float64 autograd."""
    from oracle.data import data
    w, x, b = data(9, 7, scale=0.2), data(7, 10), data(9)
    loss, dw, dx, db = interpret.linear_bias_gelu_grad(w, x, b)
    t = [torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=True) for a in (w, x, b)]
    gelu = lambda z: z / 2 * (1 + torch.tanh(0.7978846 * (z + 0.044715 * z ** 3)))  # noqa: E731
    lt = (gelu(t[0] @ t[1] + t[2][:, None]) ** 2).sum()
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12 * abs(loss)
    for ours, tt in zip((dw, dx, db), t):
        assert relative(ours, tt.grad.numpy()) < 1e-12
    args = (data(6, 10), data(7, 6, scale=0.1), data(7), data(6, 7, scale=0.2), data(6))
    loss, *grads = interpret.tanh_mlp_grad(*args)
    t = [torch.tensor(np.asarray(a, dtype=np.float64), requires_grad=True) for a in args]
    y = t[3] @ torch.tanh(t[1] @ t[0] + t[2][:, None]) + t[4][:, None]
    (y ** 2).sum().backward()
    assert abs(loss - (y ** 2).sum().item()) < 1e-12 * abs(loss)
    for ours, tt in zip(grads, t):
        assert relative(ours, tt.grad.numpy()) < 1e-12


def test_batched_product_and_accumulate():
    """product over a batch axis against numpy's matmul per slice, and D + A B."""
    rng = np.random.default_rng(2)
    a, b, d = rng.normal(size=(3, 4, 2)), rng.normal(size=(4, 5, 2)), rng.normal(size=(3, 5, 2))
    c = interpret.product(a, b, d)
    for z in range(2):
        assert np.allclose(c[:, :, z], a[:, :, z] @ b[:, :, z] + d[:, :, z], rtol=1e-14, atol=1e-14)
