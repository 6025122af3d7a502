"""Products beyond the bf16 tile kernel's shapes, and the tile kernel's batch,
split K and accumulate.  The general kernel: every product of the reference's
fixture programs at its own shape (test/fixtures/programs.jl:79-96), fp32
factors, transposed operands through strides, a batch axis, D + A B, and bf16
or fp16 factors at shapes that are not multiples of 8.  A whole fixture
program ("linear, bias, GELU") with its gradient, its products on the general
kernel and its pointwise work and folds on the generated floor.  The tile
kernel: a batch of products, K split over parts (512 x 512 x 65536, which
alone would fill four CUs), and D + A B in place.  All against the float64
oracle on the same inputs."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import data, relative

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5   # fp32 factors, fp32 sums: 1e-5 relative, norm-wise
TOL_HALF = 1e-2  # half factors: products exact, one rounding of the result (2^-8 relative)


def _col(a, dtype=torch.float32):
    """A Julia (column-major) array on the device: memory = a.ravel(order='F')."""
    return torch.from_numpy(np.asarray(a, dtype=np.float64).ravel(order="F").copy()).to(dtype).cuda()


def _back(t, shape):
    return t.double().cpu().numpy().reshape(shape, order="F")


def _product(a, b, shape_a, shape_b, transpose_a=False, transpose_b=False, dtype=torch.float32,
             factors=None, result=None, d=None, batch=1):
    """C = op(A) op(B) (+ D) through th_build_gemm, A and B Julia arrays; op
    = transpose where asked, by strides."""
    import tempest_hip.launch as L
    fac = factors if factors is not None else L.F32
    res = result if result is not None else fac
    tdt = {L.F32: torch.float32, L.BF16: torch.bfloat16, L.F16: torch.float16}
    ta, tb = _col(a, tdt[fac]), _col(b, tdt[fac])
    ra, ca = shape_a[0], shape_a[1]
    rb, cb = shape_b[0], shape_b[1]
    m, k = (ca, ra) if transpose_a else (ra, ca)
    k2, n = (cb, rb) if transpose_b else (rb, cb)
    assert k == k2
    a_m, a_k = (ra, 1) if transpose_a else (1, ra)
    b_k, b_n = (rb, 1) if transpose_b else (1, rb)
    c = torch.zeros(m * n * batch, dtype=tdt[res], device="cuda")
    dd = _col(d, tdt[res]) if d is not None else None
    l = L.gemm(m, n, k, ta.data_ptr(), a_m, a_k, tb.data_ptr(), b_k, b_n, c.data_ptr(), m, c_dtype=res,
               factors=fac, batch=batch, a_batch=ra * ca, b_batch=rb * cb, c_batch=m * n,
               d=dd.data_ptr() if dd is not None else 0)
    l()
    torch.cuda.synchronize()
    return _back(c, (m, n, batch) if batch > 1 else (m, n)), l


def test_products_of_the_fixture_programs(target):
    """Each product of the reference's fixtures at its own shape, fp32."""
    import tempest_hip.launch as L
    cases = [
        ("MLP w1 * x", data(7, 6, scale=0.1), data(6, 10), False, False, None),
        ("MLP w2 * h", data(6, 7, scale=0.2), np.tanh(data(7, 10)), False, False, None),
        ("adjoint product a' * b", data(6, 4), data(6, 5, scale=0.3), True, False, None),
        ("product spelled as a broadcast sum", data(5, 7, scale=0.3), data(7, 6), False, False, None),
        ("linear w * x", data(9, 7, scale=0.2), data(7, 10), False, False, None),
        ("residual epilogue w * x .+ x", data(7, 7, scale=0.2), data(7, 10), False, False, data(7, 10)),
        ("scaling prologue w * (x .* 0.5)", data(9, 7, scale=0.2), data(7, 10) * 0.5, False, False, None),
        ("products of transposes a' * b'", data(7, 5, scale=0.2), data(6, 7), True, True, None),
        ("matrix vector", data(5, 4), data(4, 1, scale=0.5), False, False, None),
        ("a constant times x", data(5, 4, scale=0.2), data(4, 3), False, False, None),
        ("a constant times a vector", data(5, 4, scale=0.2), data(4, 1, scale=0.5), False, False, None),
        ("x' times a constant", data(5, 3), data(5, 4, scale=0.2), True, False, None),
    ]
    for name, a, b, ta, tb, d in cases:
        announce("general product", name)
        got, l = _product(a, b, a.shape, b.shape, ta, tb, d=d)
        assert "gemm_general" in l.describe(), name
        want = interpret.product(a.T if ta else a, b.T if tb else b, d)
        assert relative(got, want) < TOL_F32, (name, relative(got, want))


def test_batched_products(target):
    """"batched product" (3 x 4 x 2 by 4 x 5 x 2) and a batch with a constant."""
    a, b = data(3, 4, 2), data(4, 5, 2, scale=0.3)
    announce("general batched product")
    got, _ = _product(a, b, (3, 4), (4, 5), batch=2)
    assert relative(got, interpret.product(a, b)) < TOL_F32
    c = data(3, 5, 2)
    got, _ = _product(data(3, 5, 2) * 0 + c, b.transpose(1, 0, 2).copy(), (3, 5), (5, 4), batch=2)
    assert relative(got, interpret.product(c, b.transpose(1, 0, 2))) < TOL_F32
    # "batched product with a constant" and "constant batched product": the
    # closed-over BATCH = data(4, 3, 2; scale = 0.3) as either factor.
    const = data(4, 3, 2, scale=0.3)
    a3 = data(3, 4, 2)
    got, _ = _product(a3, const, (3, 4), (4, 3), batch=2)
    assert relative(got, interpret.product(a3, const)) < TOL_F32
    b3 = data(3, 5, 2)
    got, _ = _product(const, b3, (4, 3), (3, 5), batch=2)
    assert relative(got, interpret.product(const, b3)) < TOL_F32


@pytest.mark.parametrize("factors,result", [("bf16", "bf16"), ("bf16", "f32"), ("f16", "f16"), ("f16", "f32")])
def test_half_factors_at_ragged_shapes(target, factors, result):
    """bf16 and fp16 factors (cuBLASProducts' FACTOR_TYPES) at 37 x 29 x 53,
    the result in the factors' type or widened to fp32."""
    import tempest_hip.launch as L
    from oracle.data import bf16_round
    f = {"bf16": L.BF16, "f16": L.F16, "f32": L.F32}
    rng = np.random.default_rng(3)
    a, b = rng.standard_normal((37, 53)), rng.standard_normal((53, 29))
    if factors == "bf16":
        a, b = bf16_round(a.astype(np.float32)).astype(np.float64), bf16_round(b.astype(np.float32)).astype(np.float64)
    else:
        a, b = a.astype(np.float16).astype(np.float64), b.astype(np.float16).astype(np.float64)
    announce("general half product", factors, result)
    got, _ = _product(a, b, a.shape, b.shape, factors=f[factors], result=f[result])
    tol = TOL_F32 if result == "f32" else TOL_HALF
    assert relative(got, interpret.product(a, b)) < tol


def test_linear_bias_gelu_program_and_gradient(target):
    """"linear, bias, GELU" (test/fixtures/programs.jl:83): loss =
    sum(abs2, gelu.(w * x .+ b)) with w 9 x 7, x 7 x 10, b 9, and its
    gradient: Z = w x and dw = dZ x', dx = w' dZ on the general kernel; the
    GELU, its derivative, dZ, db and the loss on the generated floor."""
    import tempest_hip.launch as L
    from tempest_hip.floor import FloorGroup
    w, x, b = data(9, 7, scale=0.2), data(7, 10), data(9)
    announce("linear bias gelu program")
    tw, tx, tb = _col(w), _col(x), _col(b)
    Z, dZ = torch.zeros(90, device="cuda"), torch.zeros(90, device="cuda")
    db, rows, loss = torch.zeros(9, device="cuda"), torch.zeros(9, device="cuda"), torch.zeros(1, device="cuda")
    dw, dx = torch.zeros(63, device="cuda"), torch.zeros(70, device="cuda")
    L.gemm(9, 10, 7, tw.data_ptr(), 1, 9, tx.data_ptr(), 1, 7, Z.data_ptr(), 9, c_dtype=L.F32, factors=L.F32)()
    # The rows of the result: z = Z + b; y = gelu(z); dz = 2 y gelu'(z);
    # db and the row's sum of y^2 fold over the columns.
    g = FloorGroup("reduction", (9, 10), reduced=(1,), name="gelu and its gradient")
    for k, n in (("Z", 90), ("b", 9), ("dZ", 90), ("db", 9), ("rows", 9)):
        g.value(k, "f32", n)
    z = g.load("Z", (1, 9)) + g.load("b", (1, 0))
    t = g.apply("tanh", 0.7978846 * (z + 0.044715 * z * z * z))
    y = z / 2.0 * (1.0 + t)
    dg = 0.5 * (1.0 + t) + 0.5 * z * (1.0 - t * t) * 0.7978846 * (1.0 + 3.0 * 0.044715 * z * z)
    dz = 2.0 * y * dg
    g.output("dZ", dz, (1, 9))
    g.output("db", g.fold("sum", dz).value, (1, 0), full=False)
    g.output("rows", g.fold("sum", y * y).value, (1, 0), full=False)
    h = FloorGroup("reduction", (9,), reduced=(0,), name="loss")
    h.value("rows", "f32", 9)
    h.value("loss", "f32", 1)
    h.output("loss", h.fold("sum", h.load("rows", (1,))).value, (0,), full=False)
    ptrs = {"Z": Z, "b": tb, "dZ": dZ, "db": db, "rows": rows, "loss": loss}
    g.build({k: ptrs[k].data_ptr() for k in g.values})()
    h.build({k: ptrs[k].data_ptr() for k in h.values})()
    # dw = dZ x' (9 x 10 by 10 x 7), dx = w' dZ (7 x 9 by 9 x 10).
    L.gemm(9, 7, 10, dZ.data_ptr(), 1, 9, tx.data_ptr(), 7, 1, dw.data_ptr(), 9, c_dtype=L.F32, factors=L.F32)()
    L.gemm(7, 10, 9, tw.data_ptr(), 9, 1, dZ.data_ptr(), 1, 9, dx.data_ptr(), 7, c_dtype=L.F32, factors=L.F32)()
    torch.cuda.synchronize()
    rl, rdw, rdx, rdb = interpret.linear_bias_gelu_grad(w, x, b)
    assert abs(loss.item() - rl) <= TOL_F32 * abs(rl)
    assert relative(_back(dw, (9, 7)), rdw) < TOL_F32
    assert relative(_back(dx, (7, 10)), rdx) < TOL_F32
    assert relative(db.double().cpu().numpy(), rdb) < TOL_F32


def _bf16(shape, gen, scale=1.0):
    return (torch.randn(*shape, device="cuda", generator=gen) * scale).to(torch.bfloat16)


def test_tile_kernel_batch(target):
    """Three 512 x 256 products summing 384, k-contiguous A, mn-contiguous B,
    on the tile kernel (grid z the batch)."""
    import tempest_hip.launch as L
    announce("tile kernel batch")
    gen = torch.Generator(device="cuda").manual_seed(4)
    A = _bf16((3, 512, 384), gen)   # A_z(i, l) at z*512*384 + i*384 + l: k-contiguous
    B = _bf16((3, 384, 256), gen)   # B_z(l, j) at z*384*256 + l*256 + j: n-contiguous
    C = torch.zeros(3, 256, 512, dtype=torch.bfloat16, device="cuda")  # column-major m x n
    l = L.gemm(512, 256, 384, A.data_ptr(), 384, 1, B.data_ptr(), 256, 1, C.data_ptr(), 512, batch=3,
               a_batch=512 * 384, b_batch=384 * 256, c_batch=512 * 256, splits=1, tile=L.TILE_256)
    assert "gemm_bf16_store" in l.describe() and "gemm_general" not in l.describe()
    l()
    torch.cuda.synchronize()
    want = torch.matmul(A.double(), B.double())  # (3, 512, 256)
    got = C.double().transpose(1, 2)
    assert relative(got.cpu().numpy(), want.cpu().numpy()) < 1e-2


@pytest.mark.parametrize("c_dtype", ["f32", "bf16"])
def test_tile_kernel_split_k(target, c_dtype):
    """512 x 512 x 65536: four tiles alone; K split into parts so that the
    launch takes 256 workgroups, the parts summed in order by a second launch."""
    import tempest_hip.launch as L
    announce("tile kernel split k", c_dtype)
    gen = torch.Generator(device="cuda").manual_seed(5)
    A = _bf16((512, 65536), gen)      # k-contiguous
    B = _bf16((512, 65536), gen)      # B(l, j) at j*65536 + l: k-contiguous
    cd = L.F32 if c_dtype == "f32" else L.BF16
    C = torch.zeros(512, 512, dtype=torch.float32 if c_dtype == "f32" else torch.bfloat16, device="cuda")
    l = L.gemm(512, 512, 65536, A.data_ptr(), 65536, 1, B.data_ptr(), 1, 65536, C.data_ptr(), 512, c_dtype=cd)
    desc = l.describe()
    assert "gemm_bf16_parts_f32" in desc and "sum_splits" in desc, desc
    assert l.work().blocks >= 256
    l()
    torch.cuda.synchronize()
    want = (A.double() @ B.double().T).T  # column-major C(i, j) at i + 512 j
    tol = 1e-4 if c_dtype == "f32" else 1e-2  # bf16 factors: within 2e-2; fp32 sums of 65536 terms
    assert relative(C.double().cpu().numpy(), want.cpu().numpy()) < tol


def test_tile_kernel_accumulates(target):
    """C = D + A B on the tile kernel: into a separate D and in place (D = C,
    a gradient accumulating over a value's uses), with K split as well."""
    import tempest_hip.launch as L
    announce("tile kernel accumulate")
    gen = torch.Generator(device="cuda").manual_seed(6)
    A = _bf16((512, 1024), gen)
    B = _bf16((512, 1024), gen)
    D = torch.randn(512, 512, device="cuda", generator=gen)
    C = torch.zeros(512, 512, device="cuda")
    prod = (A.double() @ B.double().T).T
    l = L.gemm(512, 512, 1024, A.data_ptr(), 1024, 1, B.data_ptr(), 1, 1024, C.data_ptr(), 512, c_dtype=L.F32,
               d=D.data_ptr(), splits=2, tile=L.TILE_256)
    l()
    torch.cuda.synchronize()
    assert relative(C.double().cpu().numpy(), (prod + D.double()).cpu().numpy()) < 1e-5
    Cb = D.to(torch.bfloat16)
    start = Cb.double().clone()
    l2 = L.gemm(512, 512, 1024, A.data_ptr(), 1024, 1, B.data_ptr(), 1, 1024, Cb.data_ptr(), 512, c_dtype=L.BF16,
                d=Cb.data_ptr(), splits=1, tile=L.TILE_256)
    l2()
    torch.cuda.synchronize()
    assert relative(Cb.double().cpu().numpy(), (prod + start).cpu().numpy()) < 1e-2
