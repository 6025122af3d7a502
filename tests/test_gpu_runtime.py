"""The runtime on the GPU: config 1 (the tanh layer's gradient), compile and
call, execute vs replay, retargeting a captured graph to moved arrays, the
arena, timings and device rates."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import data, relative

pytestmark = pytest.mark.gpu


def _col(a):
    """A Julia (column-major) array as the torch tensor holding its bytes."""
    a = np.asfortranarray(a, dtype=np.float32)
    return torch.from_numpy(np.ascontiguousarray(a.T)).cuda()


def _julia(t, dims):
    return t.detach().cpu().numpy().reshape(tuple(reversed(dims))).T


@pytest.mark.parametrize("d,h,c", [(32, 64, 16), (1, 1, 1), (7, 13, 5), (64, 128, 32)])
def test_tanh_layer_grad_matches_oracle(target, d, h, c):
    import tempest_hip as th
    announce("tanh layer", d, h, c)
    w, b, x = data(d, h), data(h, scale=0.3), data(d, c, scale=0.7)
    args = [_col(w), _col(b), _col(x)]
    comp = th.compile(th.programs.tanh_layer(d, h, c), target, *args)
    loss, dw, db, dx = comp(*args)
    rl, rdw, rdb, rdx = interpret.tanh_layer_grad(w, b, x)
    assert abs(loss - rl) <= 1e-5 * abs(rl)
    assert relative(_julia(dw, (d, h)), rdw) < 1e-5
    assert relative(db.cpu().numpy(), rdb) < 1e-5
    assert relative(_julia(dx, (d, c)), rdx) < 1e-5


def test_tanh_layer_refuses_what_does_not_fit(target):
    import tempest_hip.launch as L
    from tempest_hip import HIPError
    with pytest.raises(HIPError, match="64 KiB"):
        L.tanh_layer_grad(128, 128, 64, 0, 0, 0, 0, 0, 0, 0)


def test_compiled_call_checks_its_signature(target):
    import tempest_hip as th
    w, b, x = (torch.zeros(s, device="cuda") for s in ((64, 32), (64,), (16, 32)))
    comp = th.compile(th.programs.tanh_layer(), target, w, b, x)
    with pytest.raises(ValueError):
        comp(w, b, torch.zeros(17, 32, device="cuda"))


def test_replay_equals_execute_and_follows_moved_arrays(target):
    """replay! after capture reads the arrays the call passes, wherever they
    are (runtime.jl:1076-1139; test/cuda/repointing.jl), and gives what
    execute! gives (test/runtime/executable.jl:8-20)."""
    import tempest_hip as th
    announce("replay retarget")
    rows, n = 64, 512
    gen = torch.Generator(device="cuda").manual_seed(5)
    xs = [torch.randn(rows, n, device="cuda", generator=gen) for _ in range(3)]
    gs = [torch.randn(rows, n, device="cuda", generator=gen) for _ in range(3)]
    prog = th.programs.softmax_columns(rows, n)
    comp = th.compile(prog, target, xs[0], gs[0])
    ex = th.prepare(prog, target, xs[0], gs[0])
    for x, g in zip(xs, gs):
        loss, dx = comp(x, g)  # the graph retargeted to x, g
        ex.point(x, g).execute()
        l2, dx2 = ex.outputs()
        torch.cuda.synchronize()
        assert torch.equal(dx, dx2) and loss == l2.item()
        ref_loss, ref = interpret.softmax_grad(x.cpu().numpy(), g.cpu().numpy())
        assert relative(dx.cpu().numpy(), ref) < 1e-5
    # Replaying again on the same arrays patches nothing and repeats the result.
    loss_a, dx_a = comp(xs[2], gs[2])
    loss_b, dx_b = comp(xs[2], gs[2])
    assert torch.equal(dx_a, dx_b) and loss_a == loss_b


def test_bind_copies_into_own_buffers(target):
    import tempest_hip as th
    rows, n = 8, 64
    x = torch.randn(rows, n, device="cuda")
    g = torch.randn(rows, n, device="cuda")
    ex = th.prepare(th.programs.layernorm(rows, n), target, x, g, point=False)
    assert ex.addresses["x"] != x.data_ptr()
    ex.execute()
    _, dx1 = ex.outputs()
    dx1 = dx1.clone()
    x2 = torch.randn(rows, n, device="cuda")
    ex.bind(x2, g).capture().replay()
    _, dx2 = ex.outputs()
    _, ref = interpret.layernorm_grad(x2.cpu().numpy(), g.cpu().numpy())
    assert relative(dx2.cpu().numpy(), ref) < 1e-5
    assert not torch.equal(dx1, dx2)


def test_graph_replays_are_stable(target):
    """A captured graph replayed several times, with eager work and
    synchronisations between, gives the eager result every time."""
    import tempest_hip as th
    rows, n = 128, 2048
    x = torch.randn(rows, n, device="cuda")
    g = torch.randn(rows, n, device="cuda")
    ex = th.prepare(th.programs.softmax_columns(rows, n), target, x, g)
    ex.execute()
    l0, d0 = (t.clone() for t in ex.outputs())
    ex.capture()
    for _ in range(4):
        ex.outputs()[1].zero_()
        torch.cuda.synchronize()
        ex.replay()
        torch.cuda.synchronize()
        assert torch.equal(ex.outputs()[1], d0) and torch.equal(ex.outputs()[0], l0)


def test_arena_slots_are_aligned_and_disjoint(target):
    from tempest_hip.runtime import Arena
    sizes = [100, 1, 4096, 300]
    a = Arena(sizes)
    assert all(p % 256 == 0 for p in a.addresses)
    for (p, s), q in zip(zip(a.addresses, sizes), a.addresses[1:]):
        assert p + s <= q
    assert a.bytes >= sum(sizes)
    a.destroy()


def test_timing_and_rates(target):
    import tempest_hip.launch as L
    rates = target.device_rates()
    assert rates["blocks"] >= 1 and rates["bandwidth"] > 1e11 and rates["cache"] > 2**20
    assert "gfx950" in target.device_name()
    x = torch.randn(1024, 4096, device="cuda")
    g = torch.randn_like(x)
    dx = torch.empty_like(x)
    loss = torch.empty(1, device="cuda")
    l = L.softmax_grad(1024, 4096, 4096, x.data_ptr(), g.data_ptr(), dx.data_ptr(), loss.data_ptr())
    t = target.time_launch(l)
    assert 0 < t < 0.1
    w = l.work()
    assert w.bytes == 3 * 4 * 1024 * 4096 and w.kernels == 2
