"""The floor's exponential (th_exp: a hardware exp2 with an fma-carried
correction) against float64 over a dense sweep of fp32: every 64th bit
pattern whose exponential is a normal float, in ulps of the fp32 result; and
the special values.  The bound is the test's, stated below."""
import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

MAX_ULP = 1.5  # th_exp measured 1.22 ulp at worst over this sweep (MI355X); bound in the fp32 result's last place


def _exp(target, x: np.ndarray) -> np.ndarray:
    from tempest_hip.floor import FloorGroup
    n = x.size
    g = FloorGroup("pointwise", (n,))
    g.value("x", "f32", n)
    g.value("y", "f32", n)
    g.output("y", g.apply("exp", g.load("x", [1])), [1])
    tx = torch.from_numpy(x).cuda()
    ty = torch.full_like(tx, float("nan"))
    l = g.build({"x": tx.data_ptr(), "y": ty.data_ptr()})
    l()
    torch.cuda.synchronize()
    return ty.cpu().numpy()


def test_exp_relative_error_over_a_dense_sweep(target):
    announce("th_exp sweep")
    # Every 64th bit pattern of [smallest x with a normal exp(x), largest
    # finite], both signs: ~35M points, each binade of x equally dense.
    lo = np.float32(np.log(np.float64(np.finfo(np.float32).tiny))) + np.float32(1e-5)
    hi = np.float32(np.log(np.float64(np.finfo(np.float32).max))) - np.float32(1e-5)
    pos = np.arange(0, np.float32(hi).view(np.uint32), 64, dtype=np.uint32).view(np.float32)
    neg = (np.arange(0, np.float32(-lo).view(np.uint32), 64, dtype=np.uint32) | np.uint32(0x80000000)).view(np.float32)
    x = np.concatenate([pos, neg, np.array([lo, hi], dtype=np.float32)])
    y = _exp(target, x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(y - ref) / ulp
    worst = int(np.argmax(err))
    print(f"th_exp: {x.size} points, max {err[worst]:.3f} ulp at x = {x[worst]!r}, "
          f"mean {err.mean():.3f} ulp, {np.mean(err > 1):.2e} beyond 1 ulp", flush=True)
    assert err[worst] <= MAX_ULP, (x[worst], y[worst], ref[worst])


def test_exp_special_values(target):
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 100.0, -100.0, -200.0, 1.0, -1.0], dtype=np.float32)
    y = _exp(target, x)
    assert y[0] == 1.0 and y[1] == 1.0                     # exactly
    assert y[2] == np.inf and y[3] == 0.0 and np.isnan(y[4])
    assert y[5] == np.inf                                  # beyond the largest float
    # Below the normal range the result is 0 or subnormal, within a subnormal step.
    tiny = np.finfo(np.float32).tiny
    assert 0 <= y[6] < tiny and abs(y[6] - np.exp(-100.0)) < tiny and y[7] == 0.0
    assert abs(y[8] - np.e) <= 2 * np.spacing(np.float32(np.e))
    assert abs(y[9] - np.exp(-1.0)) <= 2 * np.spacing(np.float32(np.exp(-1.0)))
