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
    # The launch gap is measured: one kernel's share of a long replayed graph
    # of empty launches, not a constant.
    assert 5e-8 < rates["launch"] < 5e-5, rates["launch"]
    assert rates["launch"] == target.device_rates()["launch"]
    # The cached rate is measured too: reads the caches serve, beyond 1 TB/s.
    assert rates["cached"] > 1e12, rates["cached"]
    print("launch gap", rates["launch"], "cached B/s", rates["cached"], flush=True)
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


def test_read_rate_measures_streams(target):
    """th_read_rate: both read patterns stream at a physical rate (between 1 and
    8.2 TB/s, HBM3E's 8 TB/s with its rounding); a bad mode is refused."""
    import ctypes
    from tempest_hip import _lib
    announce("read rate")
    for mode in (0, 1):
        b = ctypes.c_double()
        _lib.call("th_read_rate", mode, ctypes.byref(b))
        assert 1e12 < b.value < 8.2e12, (mode, b.value)
    with pytest.raises(_lib.HIPError):
        _lib.call("th_read_rate", 2, ctypes.byref(ctypes.c_double()))


def test_lds_rate_measures_reads_and_products(target):
    import ctypes
    from tempest_hip import _lib
    announce("lds rate")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    got = {}
    for mode in range(4):
        b, f, c = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        _lib.call("th_lds_rate", mode, 2, ctypes.byref(b), ctypes.byref(f), ctypes.byref(c))
        assert 0.5e9 < c.value < 3.0e9, c.value
        per_clk = b.value / c.value / cus
        # Between a tenth of a bank pass and the 256 bytes a clock the 64 banks give.
        assert 10 < per_clk <= 300, (mode, per_clk)
        assert (f.value > 0) == (mode >= 2)
        got[mode] = per_clk
    print("LDS B/clk/CU", got, flush=True)
    for bad in ((4, 1), (-1, 1), (0, 3), (0, 0)):
        with pytest.raises(_lib.HIPError):
            _lib.call("th_lds_rate", bad[0], bad[1], ctypes.byref(ctypes.c_double()), ctypes.byref(ctypes.c_double()),
                      ctypes.byref(ctypes.c_double()))


def test_slots_taken_one_by_one_lie_in_one_reservation(target):
    """A pool's reserved range (th_pool_*): the config-3 MLP program's slots
    and a second executable's, allocated one at a time as `planned` does
    (runtime.jl:415), all inside [base, base + reserved), the results the
    arena's; freed blocks are reused."""
    import tempest_hip as th
    announce("slot pool")
    pool = th.Pool(reserve=8 << 30)
    base, reserved, mapped = pool.info()
    assert reserved >= 8 << 30 and mapped <= reserved
    rows, n = 300, 1000
    gen = torch.Generator(device="cuda").manual_seed(8)
    x, g = torch.randn(rows, n, device="cuda", generator=gen), torch.randn(rows, n, device="cuda", generator=gen)
    prog = th.programs.mlp(512, 256, 1024, 256)
    inputs = [(torch.randn(*reversed(prog.values[k].dims), device="cuda", generator=gen) * 0.05).to(torch.bfloat16)
              for k in prog.inputs]
    ex = th.prepare(prog, target, *inputs, pool=pool)
    ref = th.prepare(prog, target, *inputs)
    for e in (ex, ref):
        e.execute()
    torch.cuda.synchronize()
    slots = [ex.addresses[name] for name, v in prog.values.items() if v.role == "stored"]
    assert slots and all(base <= a < base + reserved for a in slots)
    for a, b in zip(ex.outputs(), ref.outputs()):
        if isinstance(a, torch.Tensor):
            assert torch.equal(a, b)
        else:
            assert a == b
    # The slots and the products' workspaces (the GELU backward's row sums,
    # the loss partials) were taken again once the workspaces were known; the
    # first blocks went back to the pool.
    assert len(ex.arena.addresses) == len(ex.storage.sizes) + sum(1 for w in ex.workspaces if w) > len(ex.storage.sizes)
    ex.arena.destroy()
    again = th.runtime.PoolSlots(pool, ex.storage.sizes)
    assert again.addresses[0] == base  # every block freed, first fit from the start
    softmax = th.prepare(th.programs.softmax_columns(rows, n), target, x, g, pool=pool)
    softmax.execute()
    torch.cuda.synchronize()
    print("pool (base, reserved, mapped)", pool.info(), flush=True)
    assert all(base <= a < base + reserved for a in softmax.arena.addresses)
    again.destroy()


def test_grouped_products_are_one_launch(target):
    """Products alike but for where their operands start (cuBLASProducts'
    build over bindings, ext/cuBLASExt.jl:262-326): one launch of three, each
    product's values numbered after the previous ones'."""
    import ctypes
    import tempest_hip.launch as L
    from tempest_hip import _lib
    announce("grouped products")
    gen = torch.Generator(device="cuda").manual_seed(9)
    As = [torch.randn(256, 512, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(3)]
    Bs = [torch.randn(256, 512, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(3)]
    Cs = [torch.zeros(256, 256, device="cuda") for _ in range(3)]
    descs = (_lib.GemmDesc * 3)()
    for i in range(3):
        descs[i] = _lib.GemmDesc(m=256, n=256, k=512, c_dtype=L.F32, a=As[i].data_ptr(), a_m=512, a_k=1,
                                 b=Bs[i].data_ptr(), b_k=1, b_n=512, c=Cs[i].data_ptr(), c_ld=256, splits=1)
    out = ctypes.c_void_p()
    _lib.call("th_build_gemm_grouped", descs, 3, ctypes.byref(out))
    l = L.Launch(out, tuple(f"{v}{i}" for i in range(3) for v in ("a", "b", "c", "bias", "aux", "aux_out",
                                                                     "row_sums", "loss", "d")))
    assert l.work().kernels == 3 and l.work().values == 27
    # Product 1 moved to product 2's output: repointed by its own value number.
    spare = torch.zeros(256, 256, device="cuda")
    l.repoint("c1", spare.data_ptr())
    l()
    torch.cuda.synchronize()
    for i, c in enumerate((Cs[0], spare, Cs[2])):
        want = (As[i].double() @ Bs[i].double().T).T
        assert relative(c.double().cpu().numpy(), want.cpu().numpy()) < 1e-5
    assert not Cs[1].any()


def test_workspaces_lie_in_the_arena(target):
    """A launch's workspace (attention's statistics and stored dS') is sized by
    th_launch_workspace and placed in the executable's arena beside the slots;
    the results are those of the launch that allocates its own at the first
    run, and of one given a caller's buffer."""
    import tempest_hip as th
    import tempest_hip.launch as L
    announce("workspace in arena")
    B, H, S = 1, 2, 256
    gen = torch.Generator(device="cuda").manual_seed(11)
    q, k, v, g = (torch.randn(B, S, H, 128, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    prog = th.programs.attention(B, H, S)
    ex = th.prepare(prog, target, q, k, v, g)
    rows = B * S * H
    ws = [l.workspace() for l in ex.launches]
    assert ws[0] == 0
    stats = (rows * 3 * 4 + 255) // 256 * 256
    assert ws[1] == stats + 2 * B * H * S * S
    assert "1 workspaces" in ex.explain()
    lo, hi = min(ex.arena.addresses), max(ex.arena.addresses)
    assert ex.arena.bytes >= sum(ex.storage.sizes) + ws[1]
    ex.execute()
    torch.cuda.synchronize()
    got = [t.clone() for t in ex.outputs()]
    # The same backward with its own workspace (allocated at its first run),
    # then with a workspace of the caller's.
    o, lse = got[0], torch.empty(H * S * B, device="cuda")
    fwd = L.attention_fwd(B, H, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr())
    fwd()
    outs = [torch.empty_like(q) for _ in range(3)]
    bwd = L.attention_bwd(B, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          g.data_ptr(), *(t.data_ptr() for t in outs))
    bwd()
    torch.cuda.synchronize()
    for a, b in zip(outs, got[1:]):
        assert torch.equal(a, b)
    buf = torch.empty(bwd.workspace() + 256, dtype=torch.uint8, device="cuda")
    addr = (buf.data_ptr() + 255) // 256 * 256
    bwd.set_workspace(addr)
    for t in outs:
        t.zero_()
    bwd()
    torch.cuda.synchronize()
    for a, b in zip(outs, got[1:]):
        assert torch.equal(a, b)
    from tempest_hip import HIPError
    with pytest.raises(HIPError, match="256-byte"):
        bwd.set_workspace(addr + 16)
    with pytest.raises(HIPError, match="no workspace"):
        fwd.set_workspace(addr)


def test_workspaces_come_from_the_pool(target):
    """With a pool, the workspaces are blocks of its reserved range too."""
    import tempest_hip as th
    announce("workspace in pool")
    B, H, S = 1, 2, 256
    gen = torch.Generator(device="cuda").manual_seed(12)
    q, k, v, g = (torch.randn(B, S, H, 128, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    pool = th.Pool(reserve=4 << 30)
    base, reserved, _ = pool.info()
    prog = th.programs.attention(B, H, S)
    ex = th.prepare(prog, target, q, k, v, g, pool=pool)
    ref = th.prepare(prog, target, q, k, v, g)
    assert all(base <= a < base + reserved for a in ex.arena.addresses)
    assert len(ex.arena.addresses) == len(ex.storage.sizes) + 1
    for e in (ex, ref):
        e.execute()
    torch.cuda.synchronize()
    for a, b in zip(ex.outputs(), ref.outputs()):
        assert torch.equal(a, b)


def test_deltanet_gradient_keeps_o_in_its_workspace(target):
    """th_build_deltanet with o null keeps o in the workspace: the gradients
    are those of the build given an o."""
    import tempest_hip.launch as L
    announce("deltanet o in workspace")
    B, H, T = 1, 2, 128
    gen = torch.Generator(device="cuda").manual_seed(13)
    q, k, v, dout = (torch.randn(B, T, H, 128, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    q = torch.nn.functional.normalize(q.float(), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(k.float(), dim=-1).to(torch.bfloat16)
    a = -torch.nn.functional.softplus(torch.randn(B, T, H, device="cuda", generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=gen))
    results = []
    for give_o in (True, False):
        o = torch.zeros_like(q)
        grads = [torch.zeros_like(q) for _ in range(3)] + [torch.zeros_like(a), torch.zeros_like(beta)]
        l = L.deltanet(B, H, T, q.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), beta.data_ptr(),
                       o.data_ptr() if give_o else 0, dout.data_ptr(), *(t.data_ptr() for t in grads))
        assert l.workspace() > 0
        l()
        torch.cuda.synchronize()
        results.append(grads)
    for x, y in zip(*results):
        assert torch.equal(x, y)


def test_builds_from_several_threads(target):
    """Builds run as tasks side by side (runtime.jl:649-680): products, floor
    groups and row programs built from eight threads at once give launches
    whose results equal those built one at a time."""
    from concurrent.futures import ThreadPoolExecutor
    import tempest_hip.launch as L
    from tempest_hip.floor import FloorGroup
    announce("threaded builds")
    gen = torch.Generator(device="cuda").manual_seed(21)
    m = 256
    a = torch.randn(m, m, device="cuda", generator=gen).to(torch.bfloat16)
    bm = torch.randn(m, m, device="cuda", generator=gen).to(torch.bfloat16)
    x = torch.randn(64, 1000, device="cuda", generator=gen)
    g = torch.randn_like(x)

    def build(i):
        kind = i % 3
        if kind == 0:
            c = torch.empty(m, m, device="cuda", dtype=torch.float32)
            return (c,), L.gemm(m, m, m, a.data_ptr(), 1, m, bm.data_ptr(), 1, m, c.data_ptr(), m, c_dtype=L.F32)
        if kind == 1:
            fg = FloorGroup("reduction", (1000, 64), reduced=(0,))
            fg.value("x", "f32", 64000)
            fg.value("r", "f32", 64)
            fg.output("r", fg.fold("sum", fg.apply("exp", fg.load("x", [1, 1000])) * (1.0 + i)).value, [0, 1],
                      full=False)
            r = torch.empty(64, device="cuda")
            return (r,), fg.build({"x": x.data_ptr(), "r": r.data_ptr()})
        # Every buffer a launch writes stays referenced while it runs: a
        # dropped one goes back to torch's allocator and is handed out again.
        dx, loss = torch.empty_like(x), torch.empty(1, device="cuda")
        return (dx, loss), L.softmax_grad(64, 1000, 1000, x.data_ptr(), g.data_ptr(), dx.data_ptr(),
                                          loss.data_ptr())

    with ThreadPoolExecutor(max_workers=8) as ex:
        threaded = list(ex.map(build, range(24)))
    serial = [build(i) for i in range(24)]
    for (t1, l1), (t2, l2) in zip(threaded, serial):
        l1()
        l2()
    torch.cuda.synchronize()
    for (t1, _), (t2, _) in zip(threaded, serial):
        for u, v in zip(t1, t2):
            assert torch.equal(u, v)


def test_copy_launch_records_and_retargets(target):
    """th_build_copy, the `Copy` step as a launch (runtime.jl:47-64): run
    directly, replayed in a graph, and retargeted to other buffers in place;
    16-byte words where the ends and the length allow, bytes otherwise."""
    import ctypes
    from tempest_hip import _lib
    announce("copy launch")
    gen = torch.Generator(device="cuda").manual_seed(9)
    for nbytes, off in ((4 << 20, 0), (1000003, 0), (4096, 3)):
        src = torch.randint(0, 256, (nbytes + 16,), dtype=torch.uint8, device="cuda", generator=gen)
        dst = torch.zeros(nbytes + 16, dtype=torch.uint8, device="cuda")
        h = ctypes.c_void_p()
        _lib.call("th_build_copy", dst.data_ptr() + off, src.data_ptr() + off, ctypes.c_uint64(nbytes), ctypes.byref(h))
        g = ctypes.c_void_p()
        try:
            _lib.call("th_launch_run", h)
            _lib.call("th_quiesce")
            assert torch.equal(dst[off:off + nbytes], src[off:off + nbytes])
            assert not dst[off + nbytes:].any() and not dst[:off].any()
            handles = (ctypes.c_void_p * 1)(h.value)
            _lib.call("th_graph_capture", handles, 1, ctypes.byref(g))
            src2 = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=gen)
            dst2 = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
            _lib.call("th_launch_repoint", h, 0, ctypes.c_void_p(dst2.data_ptr()))
            _lib.call("th_launch_repoint", h, 1, ctypes.c_void_p(src2.data_ptr()))
            _lib.call("th_graph_retarget", g, 0)
            _lib.call("th_graph_replay", g)
            _lib.call("th_quiesce")
            assert torch.equal(dst2, src2)
        finally:
            if g.value:
                _lib.call("th_graph_release", g)
            _lib.call("th_launch_destroy", h)


def test_pool_destroyed_before_its_blocks(target):
    """A pool destroyed while a block is taken keeps its range until that
    block is freed (a host's collector may finalize the pool first), and
    takes no new block meanwhile."""
    import ctypes
    from tempest_hip import HIPError, _lib
    announce("pool destroyed before its blocks")
    p = ctypes.c_void_p()
    _lib.call("th_pool_create", ctypes.c_uint64(1 << 30), ctypes.byref(p))
    a = ctypes.c_void_p()
    _lib.call("th_pool_alloc", p, ctypes.c_uint64(1 << 20), ctypes.c_uint64(256), ctypes.byref(a))
    _lib.call("th_pool_destroy", p)
    host = np.arange(1 << 18, dtype=np.float32)
    back = np.zeros_like(host)
    _lib.call("th_upload", a, host.ctypes.data, ctypes.c_size_t(host.nbytes))
    _lib.call("th_download", back.ctypes.data, a, ctypes.c_size_t(back.nbytes))
    assert np.array_equal(host, back)
    b = ctypes.c_void_p()
    with pytest.raises(HIPError, match="destroyed"):
        _lib.call("th_pool_alloc", p, ctypes.c_uint64(256), ctypes.c_uint64(256), ctypes.byref(b))
    _lib.call("th_pool_free", p, a)
