"""The product's middle tiles (128 x 128, 128 x 64, 64 x 128, 64 x 64 on the
half-precision matrix cores) and the measured choice among every kernel and
split (th_gemm_tune), against the float64 product of the same factors: every
tile and operand layout, bf16 and fp16 factors, ragged m, n, k, a batch, D + A
B (also in place), a bias, parts of K; the tuner's choice is one of the
kernels that take the product, is kept for the process, and builds a launch
whose result matches."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import bf16_round, relative

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5   # half factors, fp32 sums and an fp32 result: products exact
TOL_HALF = 1e-2  # one rounding of the result to bf16 / fp16 (2^-8, 2^-11 relative)

MID = [2, 3, 4, 5]  # TILE_128X128, TILE_128X64, TILE_64X128, TILE_64X64


def _half(x, f16):
    x = np.asarray(x, dtype=np.float32)
    return (x.astype(np.float16) if f16 else bf16_round(x)).astype(np.float64)


def _dev(a, f16):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(
        torch.float16 if f16 else torch.bfloat16).cuda()


def _case(m, n, k, a_kc, b_kc, f16, seed, batch=1):
    """A (m x k) and B (k x n) per product, stored k-contiguous or not, with
    leading dimensions padded to multiples of 8; device tensors and strides."""
    rng = np.random.default_rng(seed)
    A = _half(rng.standard_normal((batch, m, k)), f16)
    B = _half(rng.standard_normal((batch, k, n)), f16)
    ld = lambda x: (x + 7) // 8 * 8  # noqa: E731
    if a_kc:  # (i, l) at i * lda + l
        lda = ld(k)
        host = np.zeros((batch, m, lda))
        host[:, :, :k] = A
        a_m, a_k, a_batch = lda, 1, m * lda
    else:  # (i, l) at i + l * lda
        lda = ld(m)
        host = np.zeros((batch, k, lda))
        host[:, :, :m] = A.transpose(0, 2, 1)
        a_m, a_k, a_batch = 1, lda, k * lda
    ta = _dev(host, f16)
    if b_kc:  # (l, j) at l + j * ldb
        ldb = ld(k)
        host = np.zeros((batch, n, ldb))
        host[:, :, :k] = B.transpose(0, 2, 1)
        b_k, b_n, b_batch = 1, ldb, n * ldb
    else:  # (l, j) at l * ldb + j
        ldb = ld(n)
        host = np.zeros((batch, k, ldb))
        host[:, :, :n] = B
        b_k, b_n, b_batch = ldb, 1, k * ldb
    tb = _dev(host, f16)
    return A, B, ta, tb, dict(a_m=a_m, a_k=a_k, b_k=b_k, b_n=b_n, a_batch=a_batch, b_batch=b_batch)


def _run(m, n, k, a_kc, b_kc, f16, tile, result_f32=True, batch=1, splits=0, d=None, bias=None, seed=0):
    import tempest_hip.launch as L
    A, B, ta, tb, st = _case(m, n, k, a_kc, b_kc, f16, seed, batch)
    rt = torch.float32 if result_f32 else (torch.float16 if f16 else torch.bfloat16)
    ldc = m + 3
    c = torch.zeros(batch, n, ldc, dtype=rt, device="cuda")
    # The oracle's contraction, batch last as Julia lays it out.
    want = interpret.product(A.transpose(1, 2, 0), B.transpose(1, 2, 0)).transpose(2, 0, 1)
    kw = {}
    if d is not None:
        dd = d if isinstance(d, torch.Tensor) else torch.from_numpy(d.astype(np.float32)).to(rt).cuda()
        kw.update(d=dd.data_ptr(), d_ld=ldc, d_batch=n * ldc)
        want = want + dd.double().cpu().numpy()[:, :, :m].transpose(0, 2, 1)
    if bias is not None:
        tbias = torch.from_numpy(bias.astype(np.float32)).to(torch.bfloat16).cuda()
        kw.update(bias=tbias.data_ptr())
        want = want + bf16_round(bias.astype(np.float32)).astype(np.float64)[None, :, None]
    l = L.gemm(m, n, k, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), ldc,
               c_dtype=L.F32 if result_f32 else (L.F16 if f16 else L.BF16), factors=L.F16 if f16 else L.BF16,
               batch=batch, a_batch=st["a_batch"], b_batch=st["b_batch"], c_batch=n * ldc, splits=splits, tile=tile,
               **kw)
    l()
    torch.cuda.synchronize()
    got = c.double().cpu().numpy()[:, :, :m].transpose(0, 2, 1)
    assert torch.all(c[:, :, m:] == 0)  # nothing past m in the leading dimension
    return got, want, l


@pytest.mark.parametrize("tile", MID)
@pytest.mark.parametrize("a_kc,b_kc", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("f16", [False, True])
def test_middle_tiles_every_layout(target, tile, a_kc, b_kc, f16):
    """Ragged 203 x 137 x 101: partial tiles along m and n, a partial last
    step along K and partial 16-byte chunks."""
    announce("gemm mid", tile, a_kc, b_kc, f16)
    got, want, l = _run(203, 137, 101, a_kc, b_kc, f16, tile)
    assert "gemm_mid" in l.describe()
    assert relative(got, want) < TOL_F32


@pytest.mark.parametrize("tile", MID)
def test_middle_tiles_half_result_batch_bias_and_added(target, tile):
    """A batch of 3, a bf16 result with a bias, and D + A B with D a separate
    array and in place (D = C)."""
    rng = np.random.default_rng(tile)
    announce("gemm mid batch", tile)
    got, want, _ = _run(130, 70, 96, True, False, False, tile, result_f32=False, batch=3,
                        bias=rng.standard_normal(130))
    assert relative(got, want) < TOL_HALF
    dd = rng.standard_normal((3, 70, 133))
    got, want, _ = _run(130, 70, 96, False, True, True, tile, result_f32=True, batch=3, d=dd)
    assert relative(got, want) < TOL_F32
    # In place: C starts as D and receives D + A B.
    import tempest_hip.launch as L
    A, B, ta, tb, st = _case(64, 48, 40, True, True, False, 9)
    c = torch.from_numpy(rng.standard_normal((48, 64)).astype(np.float32)).cuda()
    before = c.double().cpu().numpy().T.copy()
    L.gemm(64, 48, 40, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), 64,
           c_dtype=L.F32, d=c.data_ptr(), tile=tile)()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().T, interpret.product(A[0], B[0], before)) < TOL_F32


@pytest.mark.parametrize("tile", [2, 5])
def test_middle_tiles_split_k(target, tile):
    """K in 3 uneven parts (each a multiple of 32, the last shorter), summed
    by the second launch with the bias, into bf16 and fp32 results."""
    rng = np.random.default_rng(11)
    announce("gemm mid split", tile)
    got, want, l = _run(96, 80, 1000, True, True, False, tile, splits=3)
    assert "sum_splits" in l.describe()
    assert relative(got, want) < TOL_F32
    got, want, _ = _run(96, 80, 1000, False, False, False, tile, result_f32=False, splits=3,
                        bias=rng.standard_normal(96))
    assert relative(got, want) < TOL_HALF


def test_automatic_choice_fills_the_device(target):
    """512 x 512 x 512 gives 4 tiles of 256: the library takes the 64 x 64
    middle tile (64 workgroups; K too short to split); 4096 x 4096 x 256
    keeps 256 x 256."""
    import tempest_hip.launch as L
    announce("gemm auto")
    t = torch.zeros(4096 * 4096, dtype=torch.bfloat16, device="cuda")
    p = t.data_ptr()
    small = L.gemm(512, 512, 512, p, 512, 1, p, 1, 512, p, 512)
    assert "gemm_mid" in small.describe() and small.work().blocks == 64
    big = L.gemm(4096, 4096, 256, p, 256, 1, p, 1, 256, p, 4096)
    assert "gemm_bf16" in big.describe()


@pytest.mark.parametrize("m,n,k", [(512, 512, 512), (256, 256, 8192), (2048, 2048, 1024)])
def test_tuner_measures_and_keeps_its_choice(target, m, n, k):
    """th_gemm_tune returns a kernel that takes the product, a split it
    supports and a positive time; asked again it returns the same without
    measuring; the launch it names computes the product."""
    import time
    import tempest_hip.launch as L
    announce("gemm tune", m, n, k)
    A, B, ta, tb, st = _case(m, n, k, True, False, False, 5)
    c = torch.zeros(n, m, dtype=torch.float32, device="cuda")
    args = (m, n, k, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(), m)
    tile, splits, seconds = L.gemm_tune(*args, c_dtype=L.F32)
    assert tile in (L.TILE_256, *MID, L.TILE_GENERAL) and splits >= 1 and seconds > 0
    print(f"  {m}x{n}x{k}: {L.TILE_NAMES[tile]}, {splits} part(s), {seconds * 1e6:.1f} us", flush=True)
    t0 = time.perf_counter()
    assert L.gemm_tune(*args, c_dtype=L.F32) == (tile, splits, seconds)
    assert time.perf_counter() - t0 < 0.05
    c.zero_()
    L.gemm(*args, c_dtype=L.F32, tile=tile, splits=splits)()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().T, interpret.product(A[0], B[0])) < TOL_F32


def test_tuner_refuses_to_measure_in_place(target):
    import tempest_hip.launch as L
    from tempest_hip import HIPError
    t = torch.zeros(64 * 64, dtype=torch.float32, device="cuda")
    h = torch.zeros(64 * 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(HIPError, match="in place"):
        L.gemm_tune(64, 64, 64, h.data_ptr(), 64, 1, h.data_ptr(), 1, 64, t.data_ptr(), 64, c_dtype=L.F32,
                    d=t.data_ptr())


def test_every_tile_agrees_on_one_product(target):
    """The same product on every kernel that takes it: each within the
    tolerance of the float64 product (the sums' order differs by tile)."""
    import tempest_hip.launch as L
    announce("gemm all tiles")
    A, B, ta, tb, st = _case(512, 384, 640, True, True, False, 21)
    want = interpret.product(A[0], B[0])
    for tile in (L.TILE_256, *MID, L.TILE_GENERAL):
        c = torch.zeros(384, 512, dtype=torch.float32, device="cuda")
        L.gemm(512, 384, 640, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(),
               512, c_dtype=L.F32, tile=tile)()
        torch.cuda.synchronize()
        assert relative(c.double().cpu().numpy().T, want) < TOL_F32, L.TILE_NAMES[tile]


def test_environment_asks_for_measured_choices(target, monkeypatch):
    """TEMPEST_HIP_TUNE=1: a product left to the library takes the tuner's
    tile and split, and still computes the product."""
    import tempest_hip.launch as L
    announce("gemm tune env")
    A, B, ta, tb, st = _case(768, 640, 1536, False, True, True, 31)
    c = torch.zeros(640, 768, dtype=torch.float32, device="cuda")
    args = (768, 640, 1536, ta.data_ptr(), st["a_m"], st["a_k"], tb.data_ptr(), st["b_k"], st["b_n"], c.data_ptr(),
            768)
    tile, splits, _ = L.gemm_tune(*args, c_dtype=L.F32, factors=L.F16)
    monkeypatch.setenv("TEMPEST_HIP_TUNE", "1")
    l = L.gemm(*args, c_dtype=L.F32, factors=L.F16)
    kernel = {L.TILE_256: "gemm_bf16", L.TILE_GENERAL: "gemm_general"}.get(tile, "gemm_mid")
    assert kernel in l.describe() and (splits > 1) == ("sum_splits" in l.describe())
    l()
    torch.cuda.synchronize()
    assert relative(c.double().cpu().numpy().T, interpret.product(A[0], B[0])) < TOL_F32
