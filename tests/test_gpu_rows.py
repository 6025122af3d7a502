"""Op class (a) on the GPU: fused softmax / LayerNorm forward and gradient
against the oracle, at the reference tests' inputs, ragged and streamed
sizes, and config 2's full size (sampled rows + invariants)."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import data, relative

pytestmark = pytest.mark.gpu

TOL = 1e-5  # fused fp32 pointwise/reduction: 1e-5 relative (norm-wise, as agree())


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def _run(target, which, x, g):
    import tempest_hip as th
    rows, n = x.shape
    prog = th.programs.softmax_columns(rows, n) if which == "softmax" else th.programs.layernorm(rows, n)
    ex = th.prepare(prog, target, _dev(x), _dev(g))
    ex.execute()
    loss, dx = ex.outputs()
    torch.cuda.synchronize()
    return loss.item(), dx.cpu().numpy()


CASES = [
    # (rows, n, source): the reference's fixtures (test/fixtures/programs.jl:74,77;
    # test/cuda/folds.jl:20-24) and sizes that take each kernel shape.
    (6, 8, "data"), (700, 256, "data"), (40, 9000, "data"), (100, 3000, "data"),
    (5, 1, "normal"), (3, 7, "normal"), (9, 1027, "normal"), (4, 4096, "normal"),
    (3, 16384, "normal"), (2, 16385, "normal"), (2, 40000, "normal"), (1, 6, "normal"),
]


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
@pytest.mark.parametrize("rows,n,source", CASES)
def test_grad_matches_oracle(target, which, rows, n, source):
    announce("rows grad", which, rows, n, source)
    if source == "data":
        x = data(n, rows).T
        g = data(n, rows, scale=0.7).T
    else:
        rng = np.random.default_rng(rows * 7919 + n)
        x = rng.normal(size=(rows, n)) * 2
        g = rng.normal(size=(rows, n))
    x = x.astype(np.float32)
    g = g.astype(np.float32)
    loss, dx = _run(target, which, x, g)
    f = interpret.softmax_grad if which == "softmax" else interpret.layernorm_grad
    ref_loss, ref_dx = f(x, g)
    assert relative(dx, ref_dx) < TOL
    scale = max(1.0, np.abs(ref_dx).sum() / rows)
    assert abs(loss - ref_loss) <= TOL * scale


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
@pytest.mark.parametrize("rows,n", [(6, 8), (33, 8192), (3, 2047), (2, 16384)])
def test_forward_matches_oracle(target, which, rows, n):
    import tempest_hip.launch as L
    announce("rows fwd", which, rows, n)
    rng = np.random.default_rng(n)
    x = (rng.normal(size=(rows, n)) * 3).astype(np.float32)
    xd = _dev(x)
    yd = torch.empty_like(xd)
    l = (L.softmax_fwd(rows, n, n, xd.data_ptr(), yd.data_ptr()) if which == "softmax"
         else L.layernorm_fwd(rows, n, n, 1e-5, xd.data_ptr(), yd.data_ptr()))
    l()
    torch.cuda.synchronize()
    ref = interpret.softmax_fwd(x) if which == "softmax" else interpret.layernorm_fwd(x)
    assert relative(yd.cpu().numpy(), ref) < TOL


def test_strided_rows_and_unaligned_fall_back_to_scalar_loads(target):
    import tempest_hip.launch as L
    announce("rows strided")
    rows, n, ld = 5, 100, 103
    rng = np.random.default_rng(1)
    big = rng.normal(size=(rows, ld)).astype(np.float32)
    gb = rng.normal(size=(rows, ld)).astype(np.float32)
    xd, gd = _dev(big), _dev(gb)
    dx = torch.zeros_like(xd)
    loss = torch.zeros(1, device="cuda")
    l = L.softmax_grad(rows, n, ld, xd.data_ptr(), gd.data_ptr(), dx.data_ptr(), loss.data_ptr())
    assert "v1" in l.describe()
    l()
    torch.cuda.synchronize()
    ref_loss, ref_dx = interpret.softmax_grad(big[:, :n], gb[:, :n])
    out = dx.cpu().numpy()
    assert relative(out[:, :n], ref_dx) < TOL
    assert np.all(out[:, n:] == 0)  # nothing written past n


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
def test_config2_full_size_sampled_rows_and_invariants(target, which):
    """32768 x 8192 (config 2): rows are independent, so sampled rows are
    checked against the Float64 oracle exactly, and every row's invariants
    (softmax: dx sums to 0; LayerNorm: dx sums to 0) at full size."""
    import tempest_hip as th
    announce("config2 full", which)
    rows, n = 32768, 8192
    gen = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(rows, n, device="cuda", generator=gen)
    g = torch.randn(rows, n, device="cuda", generator=gen)
    prog = th.programs.softmax_columns(rows, n) if which == "softmax" else th.programs.layernorm(rows, n)
    c = th.compile(prog, target, x, g)
    loss, dx = c(x, g)
    sample = torch.tensor([0, 1, 4097, 12345, 20000, 32766, 32767], device="cuda")
    xs, gs, ds = (t.index_select(0, sample).cpu().numpy() for t in (x, g, dx))
    f = interpret.softmax_grad if which == "softmax" else interpret.layernorm_grad
    _, ref = f(xs, gs)
    assert relative(ds, ref) < TOL
    row_sums = dx.double().sum(dim=1).abs().max().item()
    assert row_sums < 1e-3
    # The loss against the Float64 loss over the whole array, computed on the GPU in float64.
    xd, gd = x.double(), g.double()
    if which == "softmax":
        ref_loss = (torch.softmax(xd, dim=1) * gd).sum().item()
    else:
        ref_loss = (torch.nn.functional.layer_norm(xd, (n,), eps=1e-5) * gd).sum().item()
    assert abs(loss - ref_loss) <= TOL * max(1.0, abs(ref_loss)) + 1e-3
