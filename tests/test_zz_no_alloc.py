"""th_softmax_grad_noalloc, the softmax gradient that allocates nothing, against
th_build_softmax_grad's launch (the same kernels): bit-identical dx and loss,
through the C ABI, on two calls in a row (the second smaller, so what the
first left in the shared scratch must not leak into it), and a refusal of rows
beyond the scratch's size."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu

MAX_ROWS = 1 << 20


def _built(rows, n, x, g):
    from tempest_hip import _lib
    dx = torch.empty_like(x)
    loss = torch.empty(1, device=x.device)
    h = ctypes.c_void_p()
    _lib.call("th_build_softmax_grad", rows, n, n, x.data_ptr(), g.data_ptr(), dx.data_ptr(), loss.data_ptr(),
              ctypes.byref(h))
    try:
        _lib.call("th_launch_run", h)
        _lib.call("th_quiesce")
    finally:
        _lib.call("th_launch_destroy", h)
    return dx, loss


def _noalloc(rows, n, x, g):
    from tempest_hip import _lib
    dx = torch.full_like(x, float("nan"))
    loss = torch.full((1,), float("nan"), device=x.device)
    _lib.call("th_softmax_grad_noalloc", rows, n, n, x.data_ptr(), g.data_ptr(), dx.data_ptr(), loss.data_ptr())
    _lib.call("th_quiesce")
    return dx, loss


def test_noalloc_matches_the_built_launch_twice(target):
    torch.cuda.synchronize()
    gen = torch.Generator(device="cuda").manual_seed(5)
    # The second call is smaller: 300 rows of the first call's 4096 partials
    # stay in the scratch, and its loss must not sum them.  n = 1000 takes the
    # resident kernel, n = 20000 the streamed one.
    for rows, n in ((4096, 1000), (300, 20000), (7, 9)):
        announce("noalloc softmax grad", rows, n)
        x = torch.randn(rows, n, device="cuda", generator=gen) * 2
        g = torch.randn(rows, n, device="cuda", generator=gen)
        ref_dx, ref_loss = _built(rows, n, x, g)
        dx, loss = _noalloc(rows, n, x, g)
        torch.cuda.synchronize()
        assert torch.equal(dx, ref_dx), (rows, n)
        assert torch.equal(loss, ref_loss), (rows, n, loss.item(), ref_loss.item())
        assert np.isfinite(loss.item())


def test_noalloc_refuses_rows_beyond_its_scratch(target):
    from tempest_hip import HIPError, _lib
    x = torch.zeros(8, device="cuda")
    with pytest.raises(HIPError, match="rows must be in 1..1048576"):
        _lib.call("th_softmax_grad_noalloc", MAX_ROWS + 1, 1, 1, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                  x.data_ptr())
    with pytest.raises(HIPError, match="rows must be"):
        _lib.call("th_softmax_grad_noalloc", 0, 1, 1, x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr())
