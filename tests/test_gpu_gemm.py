"""Op class (b) on the GPU: the bf16 product in every operand layout, its
fused epilogues, and config 3 (the 2-layer MLP's gradient) against the
oracle at small sizes and against a float32 torch reference at full size."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import bf16_round, relative

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2  # bf16 products: 2e-2 relative (norm-wise) of the fp32/fp64 reference


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).cuda()


def _operand(mat, contiguous_inner: bool):
    """A Julia matrix (rows x cols) stored with its second index fastest
    (True) or its first index fastest (False); returns (tensor, row stride, col stride)."""
    r, c = mat.shape
    if contiguous_inner:
        return _bf16(mat), c, 1
    return _bf16(mat.T), 1, r


LAYOUTS = [("k", "k"), ("k", "mn"), ("mn", "k"), ("mn", "mn")]


def _run_gemm(m, n, k, la, lb, c_f32=True, bias=None, ldc=None, seed=0, tile=1):
    import tempest_hip.launch as L
    rng = np.random.default_rng(seed)
    A = bf16_round(rng.normal(size=(m, k)).astype(np.float32))
    B = bf16_round(rng.normal(size=(k, n)).astype(np.float32))
    # A (m x k): k-contiguous = second index fastest.
    ta, a_m, a_k = _operand(A, la == "k")
    # B (k x n): k-contiguous = first index fastest.
    tb, b_k, b_n = _operand(B, lb != "k")
    ldc = ldc or m
    c = torch.zeros(n, ldc, dtype=torch.float32 if c_f32 else torch.bfloat16, device="cuda")
    tbias = None
    if bias is not None:
        tbias = _bf16(bias)
    l = L.gemm(m, n, k, ta.data_ptr(), a_m, a_k, tb.data_ptr(), b_k, b_n, c.data_ptr(), ldc,
               c_dtype=L.F32 if c_f32 else L.BF16, bias=tbias.data_ptr() if tbias is not None else 0, tile=tile)
    if tile == L.TILE_256:
        assert "gemm_bf16" in l.describe()
    l()
    torch.cuda.synchronize()
    out = c.float().cpu().numpy()[:, :m].T
    ref = A.astype(np.float64) @ B.astype(np.float64)
    if bias is not None:
        ref = ref + bf16_round(bias)[:, None]
    return out, ref, c


@pytest.mark.parametrize("la,lb", LAYOUTS)
@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (512, 768, 320), (72, 136, 40), (8, 8, 8), (1024, 256, 2048)])
@pytest.mark.parametrize("tile", [1, 0])  # the 256 x 256 kernel; the library's choice
def test_product_fp32_result_is_exact_to_accumulation(target, m, n, k, la, lb, tile):
    announce("gemm f32", m, n, k, la, lb, tile)
    out, ref, _ = _run_gemm(m, n, k, la, lb, c_f32=True, tile=tile)
    assert relative(out, ref) < 1e-5


@pytest.mark.parametrize("la,lb", LAYOUTS)
def test_product_bf16_result_with_bias_and_ldc(target, la, lb):
    announce("gemm bf16 bias", la, lb)
    m, n, k = 264, 520, 200
    bias = np.random.default_rng(3).normal(size=m).astype(np.float32)
    out, ref, c = _run_gemm(m, n, k, la, lb, c_f32=False, bias=bias, ldc=272)
    assert relative(out, ref) < 4e-3  # one bf16 rounding of the result
    assert torch.all(c[:, m:] == 0)  # nothing written between m and ldc


def test_shapes_route_to_the_kernel_that_takes_them(target):
    """The library's choice: a product too small to fill the device with
    256 x 256 tiles runs on a middle tile, also at m not a multiple of 8; one
    with no unit stride on the general kernel; a fused epilogue there is
    refused; a tile named that does not take the product is refused."""
    import tempest_hip.launch as L
    from tempest_hip import HIPError
    t = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    p = t.data_ptr()
    assert "gemm_mid" in L.gemm(64, 64, 64, p, 64, 1, p, 1, 64, p, 64).describe()
    assert "gemm_bf16_store" in L.gemm(64, 64, 64, p, 64, 1, p, 1, 64, p, 64, tile=L.TILE_256).describe()
    assert "gemm_mid" in L.gemm(60, 64, 64, p, 64, 1, p, 1, 64, p, 64).describe()
    assert "gemm_general" in L.gemm(60, 64, 64, p, 64, 1, p, 1, 64, p, 64, tile=L.TILE_GENERAL).describe()
    assert "gemm_general" in L.gemm(64, 64, 32, p, 64, 2, p, 1, 64, p, 64).describe()
    with pytest.raises(HIPError, match="fused epilogues"):
        L.gemm(60, 64, 64, p, 64, 1, p, 1, 64, p, 64, epilogue=L.GELU, bias=p, aux_out=p)
    with pytest.raises(HIPError, match="256 x 256 kernel takes"):
        L.gemm(60, 64, 64, p, 64, 1, p, 1, 64, p, 64, tile=L.TILE_256)
    with pytest.raises(HIPError, match="middle tiles take"):
        L.gemm(64, 64, 32, p, 64, 2, p, 1, 64, p, 64, tile=L.TILE_64X64)


def _mlp_inputs(batch, d_in, hidden, d_out, seed):
    rng = np.random.default_rng(seed)
    W1 = bf16_round((rng.normal(size=(hidden, d_in)) / np.sqrt(d_in)).astype(np.float32))
    b1 = bf16_round((rng.normal(size=hidden) / np.sqrt(d_in)).astype(np.float32))
    W2 = bf16_round((rng.normal(size=(d_out, hidden)) / np.sqrt(hidden)).astype(np.float32))
    b2 = bf16_round((rng.normal(size=d_out) / np.sqrt(hidden)).astype(np.float32))
    x = bf16_round(rng.normal(size=(d_in, batch)).astype(np.float32))
    return W1, b1, W2, b2, x


def _col(a):
    """A Julia array as the bf16 tensor holding its column-major bytes."""
    return _bf16(np.ascontiguousarray(a.T) if a.ndim == 2 else a)


def _julia(t, dims):
    return t.float().cpu().numpy().reshape(tuple(reversed(dims))).T if len(dims) == 2 else t.float().cpu().numpy()


@pytest.mark.parametrize("batch,d_in,hidden,d_out", [(256, 256, 512, 256), (264, 136, 520, 72)])
def test_mlp_program_matches_oracle(target, batch, d_in, hidden, d_out):
    import tempest_hip as th
    announce("mlp small", batch, d_in, hidden, d_out)
    W1, b1, W2, b2, x = _mlp_inputs(batch, d_in, hidden, d_out, 7)
    args = [_col(a) for a in (W1, b1, W2, b2, x)]
    comp = th.compile(th.programs.mlp(batch, d_in, hidden, d_out), target, *args)
    loss, dW1, db1, dW2, db2, dx = comp(*args)
    ref = interpret.mlp_grad(W1, b1, W2, b2, x)
    assert abs(loss - ref[0]) <= BF16_TOL * abs(ref[0])
    got = [_julia(dW1, (hidden, d_in)), _julia(db1, (hidden,)), _julia(dW2, (d_out, hidden)),
           _julia(db2, (d_out,)), _julia(dx, (d_in, batch))]
    for name, g, r in zip(("dW1", "db1", "dW2", "db2", "dx"), got, ref[1:]):
        assert relative(g, r) < BF16_TOL, name


def test_mlp_config3_full_size_against_fp32(target):
    """Config 3 at its size against torch in float32 on the same bf16 inputs
    (the floating-point reference of the same ops)."""
    import tempest_hip as th
    announce("mlp config3 full")
    batch, d_in, hidden, d_out = 4096, 4096, 16384, 4096
    gen = torch.Generator(device="cuda").manual_seed(3)
    bf = torch.bfloat16
    W1 = (torch.randn(d_in, hidden, device="cuda", generator=gen) / d_in ** 0.5).to(bf)   # Julia hidden x d_in
    b1 = (torch.randn(hidden, device="cuda", generator=gen) / d_in ** 0.5).to(bf)
    W2 = (torch.randn(hidden, d_out, device="cuda", generator=gen) / hidden ** 0.5).to(bf)  # Julia d_out x hidden
    b2 = (torch.randn(d_out, device="cuda", generator=gen) / hidden ** 0.5).to(bf)
    x = torch.randn(batch, d_in, device="cuda", generator=gen).to(bf)                      # Julia d_in x batch
    comp = th.compile(th.programs.mlp(batch, d_in, hidden, d_out), target, W1, b1, W2, b2, x)
    loss, dW1, db1, dW2, db2, dx = comp(W1, b1, W2, b2, x)
    # Reference in Julia orientation, float32: W1j = W1.T etc.
    W1j, W2j, xj = W1.float().T, W2.float().T, x.float().T
    z = W1j @ xj + b1.float()[:, None]
    gelu = lambda v: v / 2 * (1 + torch.tanh(0.7978846 * (v + 0.044715 * v ** 3)))  # noqa: E731
    hh = gelu(z)
    y = W2j @ hh + b2.float()[:, None]
    ref_loss = (y.double() ** 2).sum().item()
    dy = 2 * y
    t = torch.tanh(0.7978846 * (z + 0.044715 * z ** 3))
    dz = (W2j.T @ dy) * (0.5 * (1 + t) + 0.5 * z * (1 - t * t) * 0.7978846 * (1 + 3 * 0.044715 * z * z))
    refs = {"dW2": dy @ hh.T, "db2": dy.sum(1), "dW1": dz @ xj.T, "db1": dz.sum(1), "dx": W1j.T @ dz}
    got = {"dW2": dW2.float().T, "db2": db2.float(), "dW1": dW1.float().T, "db1": db1.float(), "dx": dx.float().T}
    assert abs(loss - ref_loss) <= BF16_TOL * abs(ref_loss)
    for k, r in refs.items():
        rel = ((got[k] - r).norm() / r.norm()).item()
        assert rel < BF16_TOL, (k, rel)
