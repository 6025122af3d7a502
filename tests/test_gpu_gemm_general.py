"""Products beyond the bf16 tile kernel's shapes, and the tile kernel's batch,
split K and accumulate.  fp32 factors on their own 128 x 128 kernel (vector
loads along a unit stride, edges element by element, K split into parts), on
the 32 x 32 kernel for small products, and as split bf16 (bf16x3) on the bf16
tile kernels, at sizes, against float64.  The general kernel: every product of the reference's
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
        assert "gemm_f32" in l.describe(), name
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


def _f32_operands(m, n, k, a_kfast, b_kfast, seed, batch=1):
    """fp32 A (m x k) and B (k x n) for each of `batch` products, on the
    device in the layout asked: A k-contiguous (A(i, l) at i k + l) or
    m-contiguous (l m + i); B k-contiguous (j k + l) or n-contiguous (l n + j).
    Returns the float64 values, the tensors and the strides."""
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((batch, m, k)).astype(np.float32)
    B = rng.standard_normal((batch, k, n)).astype(np.float32)
    ta = torch.from_numpy(np.ascontiguousarray(A if a_kfast else A.transpose(0, 2, 1))).cuda()
    tb = torch.from_numpy(np.ascontiguousarray(B.transpose(0, 2, 1) if b_kfast else B)).cuda()
    st = {"a_m": k if a_kfast else 1, "a_k": 1 if a_kfast else m, "b_k": 1 if b_kfast else n, "b_n": k if b_kfast else 1,
          "a_batch": m * k, "b_batch": k * n}
    return A.astype(np.float64), B.astype(np.float64), ta, tb, st


def _run_f32(m, n, k, ta, tb, st, batch=1, d=None, bf16x3=False, splits=0, tile=0):
    import tempest_hip.launch as L
    c = torch.zeros(batch, n, m, device="cuda")  # column-major m x n per product
    l = L.gemm(m, n, k, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), m,
               c_dtype=L.F32, factors=L.F32, batch=batch, a_batch=st["a_batch"], b_batch=st["b_batch"],
               c_batch=m * n, d=(d.data_ptr() if d is not None else 0), bf16x3=bf16x3, splits=splits, tile=tile)
    l()
    torch.cuda.synchronize()
    return c.double().cpu().numpy().transpose(0, 2, 1), l


@pytest.mark.parametrize("m,n,k,a_kfast,b_kfast", [
    (512, 384, 1024, True, True), (512, 384, 1024, False, False), (512, 384, 1024, True, False),
    (512, 384, 1024, False, True), (1000, 700, 333, True, False), (129, 257, 17, False, True),
    (2048, 1024, 1536, False, False), (1, 300, 5, True, True)])
@pytest.mark.parametrize("splits", [0, 1])
def test_f32_kernel_at_size(target, m, n, k, a_kfast, b_kfast, splits):
    """fp32 factors, every operand layout, interior tiles (16-byte loads) and
    ragged edges (element loads, bounds-checked): with the parts left to the
    library (the 32 x 32 kernel for products under 64 tiles of 128 x 128 and
    K <= 2048, else the 128 x 128 one) and in one part (the 128 x 128 kernel)."""
    announce("fp32 kernel", m, n, k, a_kfast, b_kfast, splits)
    A, B, ta, tb, st = _f32_operands(m, n, k, a_kfast, b_kfast, m + n + k)
    got, l = _run_f32(m, n, k, ta, tb, st, splits=splits)
    small = splits == 0 and ((m + 127) // 128) * ((n + 127) // 128) < 64 and k <= 2048
    assert ("gemm_f32_32x32" if small else "gemm_f32_128x128") in l.describe(), l.describe()
    assert relative(got[0], A[0] @ B[0]) < TOL_F32


def test_f32_kernel_splits_k_batches_and_adds(target):
    """256 x 256 x 8192 (four tiles alone) split into parts summed in order;
    a batch of three with D + A B; D + A B in place (D = C)."""
    announce("fp32 kernel split k")
    A, B, ta, tb, st = _f32_operands(256, 256, 8192, True, False, 11)
    got, l = _run_f32(256, 256, 8192, ta, tb, st)
    assert "gemm_f32_sum_parts" in l.describe() and l.work().blocks >= 256, l.describe()
    assert relative(got[0], A[0] @ B[0]) < 3e-5  # fp32 sums of 8192 terms
    # Eight tiles over a short K ("linear, bias, GELU" of the reference's
    # coverage suite, 256 x 384 x 512): 128 blocks of 32 x 32, no parts; and
    # the same asked for in parts of at least 32 (twelve, 96 workgroups).
    A, B, ta, tb, st = _f32_operands(256, 512, 384, False, False, 13)
    got, l = _run_f32(256, 512, 384, ta, tb, st)
    assert "gemm_f32_32x32" in l.describe() and l.work().blocks == 128, l.describe()
    assert relative(got[0], A[0] @ B[0]) < TOL_F32
    got, l = _run_f32(256, 512, 384, ta, tb, st, splits=12)
    assert "gemm_f32_sum_parts" in l.describe() and l.work().blocks == 96, l.describe()
    assert relative(got[0], A[0] @ B[0]) < TOL_F32
    A, B, ta, tb, st = _f32_operands(384, 200, 640, False, True, 12, batch=3)
    D = torch.randn(3, 200, 384, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3))
    got, _ = _run_f32(384, 200, 640, ta, tb, st, batch=3, d=D)
    want = A @ B + D.double().cpu().numpy().transpose(0, 2, 1)
    assert relative(got, want) < TOL_F32
    # In place: C starts as D and the product is added to it.
    import tempest_hip.launch as L
    c = D.clone()
    start = c.double().cpu().numpy().transpose(0, 2, 1)
    L.gemm(384, 200, 640, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), 384,
           c_dtype=L.F32, factors=L.F32, batch=3, a_batch=st["a_batch"], b_batch=st["b_batch"], c_batch=384 * 200,
           d=c.data_ptr(), splits=2)()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().transpose(0, 2, 1), A @ B + start) < TOL_F32


# bf16x3: each fp32 factor hi + lo with hi = bf16(x), lo = bf16(x - hi), and
# C = A_hi B_hi + A_hi B_lo + A_lo B_hi summed in fp32.  What it leaves out
# per product a b: a_lo b_lo (|a_lo| <= 2^-9 |a|, so <= 2^-18 |a b|) and the
# rounding of x - hi to lo (<= 2^-9 |x - hi| <= 2^-17 |x|), about 2^-16 of
# |a b| at worst; random signs keep the norm-wise error of a sum of such
# terms near that, well inside the 2e-4 the reference's fp32 product tests
# hold (test/cuda/products.jl) and ~100x below bf16 factors' error.
TOL_BF16X3 = 2e-4


@pytest.mark.parametrize("m,n,k,a_kfast,b_kfast", [
    (1024, 768, 2048, True, True), (1024, 768, 2048, False, False), (1024, 768, 2048, True, False),
    (1024, 768, 2048, False, True), (1000, 700, 333, False, True), (37, 29, 53, True, False)])
def test_bf16x3_products(target, m, n, k, a_kfast, b_kfast):
    """fp32 factors as split bf16 on the bf16 tile kernels: within the fp32
    products' tolerance, and far closer than bf16 factors."""
    from oracle.data import bf16_round
    announce("bf16x3", m, n, k, a_kfast, b_kfast)
    A, B, ta, tb, st = _f32_operands(m, n, k, a_kfast, b_kfast, 7 * m + k)
    got, l = _run_f32(m, n, k, ta, tb, st, bf16x3=True)
    desc = l.describe()
    assert "split_bf16x3" in desc and ("gemm_bf16" in desc or "gemm_mid" in desc) and "gemm_f32" not in desc, desc
    want = A[0] @ B[0]
    err = relative(got[0], want)
    plain = relative(bf16_round(A[0].astype(np.float32)).astype(np.float64) @
                     bf16_round(B[0].astype(np.float32)).astype(np.float64), want)
    assert err < TOL_BF16X3, err
    assert err < plain / 30, (err, plain)


def test_bf16x3_batch_split_and_in_place(target):
    """A batch of two with D + A B, K split, and D + A B in place."""
    import tempest_hip.launch as L
    announce("bf16x3 batch")
    A, B, ta, tb, st = _f32_operands(512, 512, 4096, True, False, 13, batch=2)
    D = torch.randn(2, 512, 512, device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
    got, l = _run_f32(512, 512, 4096, ta, tb, st, batch=2, d=D, bf16x3=True, splits=4)
    assert "sum_splits" in l.describe()
    want = A @ B + D.double().cpu().numpy().transpose(0, 2, 1)
    assert relative(got, want) < TOL_BF16X3
    c = D.clone()
    start = c.double().cpu().numpy().transpose(0, 2, 1)
    L.gemm(512, 512, 4096, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), 512,
           c_dtype=L.F32, factors=L.F32, batch=2, a_batch=st["a_batch"], b_batch=st["b_batch"], c_batch=512 * 512,
           d=c.data_ptr(), bf16x3=True)()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().transpose(0, 2, 1), A @ B + start) < TOL_BF16X3


def test_bf16x3_tuned_and_refusals(target):
    """th_gemm_tune measures the bf16 tiles for a bf16x3 product; an epilogue,
    a bias or a half result is refused."""
    import tempest_hip.launch as L
    from tempest_hip import HIPError
    announce("bf16x3 tune")
    A, B, ta, tb, st = _f32_operands(768, 640, 1536, True, True, 14)
    c = torch.zeros(640, 768, device="cuda")
    args = (768, 640, 1536, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), 768)
    tile, splits, sec = L.gemm_tune(*args, c_dtype=L.F32, factors=L.F32, bf16x3=True)
    assert tile in (L.TILE_256, L.TILE_128X128, L.TILE_128X64, L.TILE_64X128, L.TILE_64X64) and sec > 0
    L.gemm(*args, c_dtype=L.F32, factors=L.F32, bf16x3=True, tile=tile, splits=splits)()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().T, A[0] @ B[0]) < TOL_BF16X3
    with pytest.raises(HIPError, match="bf16x3"):
        L.gemm(*args, c_dtype=L.BF16, factors=L.F32, bf16x3=True)
    with pytest.raises(HIPError, match="bf16x3"):
        L.gemm(*args, c_dtype=L.F32, factors=L.F32, bf16x3=True, tile=L.TILE_GENERAL)
