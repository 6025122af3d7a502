"""The generated floor on the GPU: every fixture program's groups against the
oracle; config 2's programs through the floor at ragged, streamed, split and
full sizes against the row oracle; column folds with lanes and parts; a
whole-array fold split into parts; graphs, repointing and a compiled call."""
import numpy as np
import pytest
import torch

import floor_cases as FC
from conftest import announce
from oracle import interpret
from oracle.data import bf16_round, data, relative

pytestmark = pytest.mark.gpu

TOL = 1e-5       # fp32 pointwise/reduction, norm-wise relative (as agree())
TOL_BF16 = 1e-2  # values stored as bfloat16 (one rounding: 2^-9 relative)


def _tensors(case):
    out = {}
    ints = {"i32": np.int32, "i64": np.int64}
    for k, n in case.lengths().items():
        dt = case.dtypes.get(k)
        if dt in ints:
            out[k] = torch.from_numpy(np.asarray(case.inputs[k], dtype=ints[dt])).cuda()
            continue
        if k in case.inputs:
            v = np.asarray(case.inputs[k], dtype=np.float32)
        else:
            v = np.zeros(n, dtype=np.float32)
        t = torch.from_numpy(v).cuda()
        out[k] = t.to(torch.bfloat16) if dt == "bf16" else t
    return out


@pytest.mark.parametrize("make", FC.CASES, ids=[c.__name__ for c in FC.CASES])
def test_fixture_programs(target, make):
    case = make()
    announce("floor fixture", case.name)
    ts = _tensors(case)
    launches = [g.build({k: ts[k].data_ptr() for k in g.values}) for g in case.groups]
    for l in launches:
        l()
    torch.cuda.synchronize()
    want = FC.run_oracle(case)
    for k in case.results:
        got = ts[k].float().cpu().numpy().astype(np.float64)
        tol = TOL_BF16 if case.dtypes.get(k) == "bf16" else TOL
        assert relative(got, want[k]) < tol, (case.name, k, relative(got, want[k]))
        if case.dtypes.get(k) == "bf16":
            # One rounding of the fp32 result: within half an ulp of bf16.
            assert np.all(np.abs(got - want[k]) <= np.abs(want[k]) * 2.0 ** -8 + 1e-30)


def _row_inputs(rows, n, seed):
    if seed is None:
        return (np.ascontiguousarray(data(n, rows).T).astype(np.float32),
                np.ascontiguousarray(data(n, rows, scale=0.7).T).astype(np.float32))
    rng = np.random.default_rng(seed)
    return rng.standard_normal((rows, n), dtype=np.float32), rng.standard_normal((rows, n), dtype=np.float32)


@pytest.mark.parametrize("which", ["softmax", "layernorm"])
@pytest.mark.parametrize("rows,n,seed", [(6, 8, None), (700, 256, None), (40, 9000, None), (9, 1027, 1),
                                         (3, 16384, 2), (2, 40000, 3), (1, 6, 4), (5, 1, 5), (4096, 1000, 6)])
def test_config2_programs_through_the_floor(target, which, rows, n, seed):
    import tempest_hip as th
    announce("floor config2", which, rows, n)
    x, g = _row_inputs(rows, n, seed)
    prog = th.programs.floor_softmax_columns(rows, n) if which == "softmax" else th.programs.floor_layernorm(rows, n)
    c = th.compile(prog, target, torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda())
    loss, dx = c(torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda())
    f = interpret.softmax_grad if which == "softmax" else interpret.layernorm_grad
    ref_loss, ref_dx = f(x, g)
    assert relative(dx.cpu().numpy(), ref_dx) < TOL
    scale = max(1.0, np.abs(ref_dx).sum() / rows)
    assert abs(loss - ref_loss) <= TOL * scale


@pytest.mark.parametrize("n,m", [(300, 5000), (70000, 8), (64, 64), (3, 100000)])
def test_column_folds_with_lanes_and_parts(target, n, m):
    """Softmax over dims = 2 of an n x m array: items adjacent in memory, the
    folded positions a stride of n apart."""
    from tempest_hip.floor import FloorGroup
    announce("floor columns", n, m)
    rng = np.random.default_rng(n + m)
    x = rng.standard_normal(n * m).astype(np.float32)
    t = rng.standard_normal(n * m).astype(np.float32)
    g = FloorGroup("reduction", (n, m), reduced=(1,))
    g.value("x", "f32", n * m)
    g.value("t", "f32", n * m)
    g.value("y", "f32", n * m)
    g.value("r", "f32", n)
    xx, tt = g.load("x", (1, n)), g.load("t", (1, n))
    e = g.fold("exp", xx)
    y = g.apply("exp", xx - e.logsumexp)
    g.output("y", y, (1, n))
    g.output("r", g.fold("sum", y * tt, phase=2).value, (1, 0), full=False)
    ts = {k: torch.from_numpy(v).cuda() for k, v in (("x", x), ("t", t))}
    ts["y"] = torch.zeros(n * m, device="cuda")
    ts["r"] = torch.zeros(n, device="cuda")
    g.build({k: v.data_ptr() for k, v in ts.items()})()
    torch.cuda.synchronize()
    X, T = x.astype(np.float64).reshape(m, n).T, t.astype(np.float64).reshape(m, n).T
    ey = np.exp(X - X.max(axis=1, keepdims=True))
    Y = ey / ey.sum(axis=1, keepdims=True)
    assert relative(ts["y"].cpu().numpy().reshape(m, n).T, Y) < TOL
    assert relative(ts["r"].cpu().numpy(), (Y * T).sum(axis=1)) < TOL


@pytest.mark.parametrize("count", [1 << 22, 1 << 20, 3 * 7 * 9973])
def test_whole_array_fold_in_parts(target, count):
    """sum(abs2, x) and maximum(x) over one item of millions of positions:
    parts fold into a workspace, the last launch merges them."""
    from tempest_hip.floor import FloorGroup
    announce("floor whole fold", count)
    x = np.random.default_rng(count).standard_normal(count).astype(np.float32)
    g = FloorGroup("reduction", (count,), reduced=(0,))
    g.value("x", "f32", count)
    g.value("out", "f32", 2)
    xx = g.load("x", (1,))
    g.output("out", g.fold("sum", g.apply("abs2", xx)).value, full=False)
    g.output("out", g.fold("max", xx).value, constant=1, full=False)
    ts = {"x": torch.from_numpy(x).cuda(), "out": torch.zeros(2, device="cuda")}
    launch = g.build({k: v.data_ptr() for k, v in ts.items()})
    for _ in range(2):  # the workspace is rewritten each run
        launch()
    torch.cuda.synchronize()
    out = ts["out"].cpu().numpy()
    x64 = x.astype(np.float64)
    assert abs(out[0] - np.sum(x64 * x64)) <= TOL * np.sum(x64 * x64)
    assert out[1] == x.max()


def test_graph_replay_and_repoint(target):
    """A compiled floor program called on moved arrays: the graph's module
    kernel nodes are retargeted, the results follow the new inputs."""
    import tempest_hip as th
    announce("floor graph repoint")
    rows, n = 300, 2048
    prog = th.programs.floor_softmax_columns(rows, n)
    x0, g0 = _row_inputs(rows, n, 11)
    c = th.compile(prog, target, torch.from_numpy(x0).cuda(), torch.from_numpy(g0).cuda())
    for seed in (12, 13, 12):
        x, g = _row_inputs(rows, n, seed)
        xt, gt = torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda()
        loss, dx = c(xt, gt)
        ref_loss, ref_dx = interpret.softmax_grad(x, g)
        assert relative(dx.cpu().numpy(), ref_dx) < TOL
        assert abs(loss - ref_loss) <= TOL * max(1.0, np.abs(ref_dx).sum() / rows)
    ex = c.executable
    for _ in range(3):  # replays with eager work between them
        ex.replay()
        torch.cuda.synchronize()
        assert relative(ex.outputs()[1].cpu().numpy(), ref_dx) < TOL


def test_bf16_inputs_widen(target):
    """A bf16 value read by a reduction: widened exactly, folded in fp32."""
    from tempest_hip.floor import FloorGroup
    announce("floor bf16 inputs")
    n, m = 1000, 37
    x = bf16_round(np.random.default_rng(7).standard_normal(n * m).astype(np.float32))
    g = FloorGroup("reduction", (n, m), reduced=(0,))
    g.value("x", "bf16", n * m)
    g.value("s", "f32", m)
    g.output("s", g.fold("sum", g.load("x", (1, n))).value, (0, 1), full=False)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    s = torch.zeros(m, device="cuda")
    g.build({"x": xt.data_ptr(), "s": s.data_ptr()})()
    torch.cuda.synchronize()
    assert relative(s.cpu().numpy(), x.astype(np.float64).reshape(m, n).sum(axis=1)) < TOL


def test_config2_full_size_through_the_floor(target):
    """32768 x 8192: sampled rows of dx against the oracle, the loss against
    the oracle's per-row losses summed."""
    import tempest_hip as th
    rows, n = 32768, 8192
    gen = torch.Generator(device="cuda").manual_seed(20261201)
    x = torch.randn(rows, n, device="cuda", generator=gen)
    g = torch.randn(rows, n, device="cuda", generator=gen)
    idx = torch.tensor([0, 1, 777, 16384, rows - 1], device="cuda")
    xs, gs = x.index_select(0, idx).cpu().numpy(), g.index_select(0, idx).cpu().numpy()
    for which in ("softmax", "layernorm"):
        announce("floor config2 full", which)
        prog = th.programs.floor_softmax_columns(rows, n) if which == "softmax" else th.programs.floor_layernorm(rows, n)
        c = th.compile(prog, target, x, g)
        loss, dx = c(x, g)
        f = interpret.softmax_grad if which == "softmax" else interpret.layernorm_grad
        _, ref = f(xs, gs)
        assert relative(dx.index_select(0, idx).cpu().numpy(), ref) < TOL
        assert np.isfinite(loss)
        del c, dx
        torch.cuda.empty_cache()


@pytest.mark.parametrize("n,m,axis,reverse", [(300, 2000, 1, False), (1000, 64, 0, True), (1, 100000, 1, False)])
def test_scans_at_size(target, n, m, axis, reverse):
    """Inclusive sums and a linear recurrence along one axis of an n x m
    array, a thread per item (items side by side when the scanned axis is the
    strided one)."""
    from tempest_hip.floor import FloorGroup
    announce("floor scan", n, m, axis, reverse)
    rng = np.random.default_rng(n * 7 + m)
    x = rng.standard_normal(n * m).astype(np.float32)
    a = (0.9 + 0.1 * rng.random(n * m)).astype(np.float32)
    g = FloorGroup("scan", (n, m), reduced=(axis,), reverse=reverse)
    for k in ("x", "a", "c", "h"):
        g.value(k, "f32", n * m)
    xx, aa = g.load("x", (1, n)), g.load("a", (1, n))
    g.output("c", g.fold("sum", xx, scan="inclusive").value, (1, n))
    g.output("h", g.fold("linear", aa, weight=xx, scan="inclusive").value, (1, n))
    ts = {"x": torch.from_numpy(x).cuda(), "a": torch.from_numpy(a).cuda(),
          "c": torch.zeros(n * m, device="cuda"), "h": torch.zeros(n * m, device="cuda")}
    g.build({k: v.data_ptr() for k, v in ts.items()})()
    torch.cuda.synchronize()
    X = x.astype(np.float64).reshape(m, n).T
    A = a.astype(np.float64).reshape(m, n).T
    if reverse:
        X, A = np.flip(X, axis), np.flip(A, axis)
    C = np.cumsum(X, axis=axis)
    H = np.zeros_like(X)
    hh = np.zeros(X.shape[1 - axis])
    for i in range(X.shape[axis]):
        sl = (i, slice(None)) if axis == 0 else (slice(None), i)
        hh = A[sl] * hh + X[sl]
        H[sl] = hh
    if reverse:
        C, H = np.flip(C, axis), np.flip(H, axis)
    got_c = ts["c"].cpu().numpy().reshape(m, n).T
    got_h = ts["h"].cpu().numpy().reshape(m, n).T
    # Sequential fp32 sums of up to 1e5 terms: error grows like the running magnitude.
    assert relative(got_c, C) < (1e-5 if X.shape[axis] <= 2000 else 1e-4)
    assert relative(got_h, H) < TOL


def test_embedding_gather_and_scatter_add_at_size(target):
    """y[:, j] = E[:, t[j]] for 20000 tokens of a 1024 x 30000 table, then the
    gradient dE[:, t[j]] += dy[:, j] (repeated tokens add atomically)."""
    from tempest_hip.floor import FloorGroup
    announce("floor embedding gather / scatter")
    d, vocab, n = 1024, 30000, 20000
    rng = np.random.default_rng(21)
    E = rng.standard_normal(d * vocab).astype(np.float32)
    tok = rng.integers(1, 200, n).astype(np.int32)  # 1-based, heavily repeated
    dy = rng.standard_normal(d * n).astype(np.float32)
    fwd = FloorGroup("pointwise", (d, n), name="E[:, t]")
    fwd.value("E", "f32", d * vocab)
    fwd.value("t", "i32", n)
    fwd.value("y", "f32", d * n)
    fwd.output("y", fwd.load("E", (1, 0), constant=-d, gather=fwd.load("t", (0, 1)), gather_coeff=d), (1, d))
    bwd = FloorGroup("pointwise", (d, n), name="dE[:, t] .+= dy")
    bwd.value("dy", "f32", d * n)
    bwd.value("t", "i32", n)
    bwd.value("dE", "f32", d * vocab)
    bwd.output("dE", bwd.load("dy", (1, d)), (1, 0), constant=-d, gather=bwd.load("t", (0, 1)), gather_coeff=d,
               accumulate=True)
    ts = {"E": torch.from_numpy(E).cuda(), "t": torch.from_numpy(tok).cuda(), "y": torch.zeros(d * n, device="cuda"),
          "dy": torch.from_numpy(dy).cuda(), "dE": torch.zeros(d * vocab, device="cuda")}
    fwd.build({k: ts[k].data_ptr() for k in fwd.values})()
    bwd.build({k: ts[k].data_ptr() for k in bwd.values})()
    torch.cuda.synchronize()
    Em = E.reshape(vocab, d)
    assert np.array_equal(ts["y"].cpu().numpy().reshape(n, d), Em[tok - 1])
    want = np.zeros((vocab, d))
    np.add.at(want, tok - 1, dy.reshape(n, d).astype(np.float64))
    assert relative(ts["dE"].cpu().numpy().reshape(vocab, d), want) < TOL


def test_scatter_add_in_order_is_deterministic(target):
    """TH_FLOOR_ORDERED (what a deterministic target asks of a fold by key):
    dE[:, t[j]] += dy[:, j] with the tokens taken one after another adds in
    the items' order, so two runs agree bit for bit and equal a float32
    accumulation in token order (numpy's add.at in float32), where the
    atomic path's sums may differ in their last bits."""
    from tempest_hip.floor import FloorGroup
    announce("floor scatter add in order")
    d, vocab, n = 64, 300, 2000
    rng = np.random.default_rng(22)
    tok = rng.integers(1, 40, n).astype(np.int32)  # heavily repeated
    dy = rng.standard_normal(d * n).astype(np.float32)
    g = FloorGroup("pointwise", (d, n), name="dE[:, t] .+= dy, in order", ordered=True)
    g.value("dy", "f32", d * n)
    g.value("t", "i32", n)
    g.value("dE", "f32", d * vocab)
    g.output("dE", g.load("dy", (1, d)), (1, 0), constant=-d, gather=g.load("t", (0, 1)), gather_coeff=d,
             accumulate=True)
    dyt, tt = torch.from_numpy(dy).cuda(), torch.from_numpy(tok).cuda()
    runs = []
    for _ in range(2):
        dE = torch.zeros(d * vocab, device="cuda")
        g.build({"dy": dyt.data_ptr(), "t": tt.data_ptr(), "dE": dE.data_ptr()})()
        torch.cuda.synchronize()
        runs.append(dE.cpu().numpy())
    want = np.zeros((vocab, d), dtype=np.float32)
    np.add.at(want, tok - 1, dy.reshape(n, d))
    assert np.array_equal(runs[0], runs[1])
    assert np.array_equal(runs[0].reshape(vocab, d), want)


@pytest.mark.parametrize("n,m,reverse", [(4096, 37, False), (100000, 1, False), (5003, 6, True), (64, 900, False)])
def test_parallel_scans(target, n, m, reverse):
    """Scans along the contiguous axis by a workgroup per item: an inclusive
    sum, and an exclusive linear recurrence whose offset reads the sum at the
    same position (h = a h' + x c, from 0)."""
    from tempest_hip.floor import FloorGroup
    announce("floor parallel scan", n, m, reverse)
    rng = np.random.default_rng(n + m)
    x = rng.standard_normal(n * m).astype(np.float32)
    a = (0.9 + 0.1 * rng.random(n * m)).astype(np.float32)
    g = FloorGroup("scan", (n, m), reduced=(0,), reverse=reverse)
    for k in ("x", "a", "c", "h", "tot"):
        g.value(k, "f32", n * m if k != "tot" else m)
    xx, aa = g.load("x", (1, n)), g.load("a", (1, n))
    c = g.fold("sum", xx, scan="inclusive")
    h = g.fold("linear", aa, weight=xx * c.value, scan="exclusive", phase=2)
    tot = g.fold("max", xx, phase=3)  # a plain fold beside the scans
    g.output("c", c.value, (1, n))
    g.output("h", h.value, (1, n))
    g.output("tot", tot.value, (0, 1), full=False)
    assert "a workgroup per item" in g.source().splitlines()[0]
    ts = {k: torch.from_numpy(v).cuda() for k, v in (("x", x), ("a", a))}
    for k in ("c", "h"):
        ts[k] = torch.zeros(n * m, device="cuda")
    ts["tot"] = torch.zeros(m, device="cuda")
    g.build({k: ts[k].data_ptr() for k in g.values})()
    torch.cuda.synchronize()
    X, A = x.astype(np.float64).reshape(m, n), a.astype(np.float64).reshape(m, n)
    if reverse:
        X, A = X[:, ::-1], A[:, ::-1]
    C = np.cumsum(X, axis=1)
    H = np.zeros_like(X)
    hh = np.zeros(m)
    for i in range(n):  # exclusive: the state before position i
        H[:, i] = hh
        hh = A[:, i] * hh + X[:, i] * C[:, i]
    if reverse:
        C, H = C[:, ::-1], H[:, ::-1]
    tol_c = 1e-5 if n <= 5003 else 1e-4  # fp32 sums of 1e5 terms
    assert relative(ts["c"].cpu().numpy().reshape(m, n), C) < tol_c
    assert relative(ts["h"].cpu().numpy().reshape(m, n), H) < tol_c
    assert np.array_equal(ts["tot"].cpu().numpy(), x.reshape(m, n).max(axis=1))


def test_column_fold_with_a_hoisted_load_and_idle_threads(target):
    """A (2, 100000, 3) fold over axis 1 with a load of x at (i0, 0, i2)
    outside the sweep: 6 items in a 64-item workgroup, so 58 threads have no
    item and must not read past x (they take item 0's positions)."""
    from tempest_hip.floor import FloorGroup
    n0, n1, n2 = 2, 100000, 3
    announce("floor column fold, hoisted load", n0, n1, n2)
    g = FloorGroup("reduction", (n0, n1, n2), reduced=(1,))
    g.value("x", "f32", n0 * n1 * n2)
    g.value("r", "f32", n0 * n2)
    x = g.load("x", (1, n0, n0 * n1))
    x0 = g.load("x", (1, 0, n0 * n1))
    g.output("r", g.fold("sum", x * x0).value, (1, 0, n0), full=False)
    assert g.source().splitlines()[0].startswith("// tempest-hip floor: columns")
    rng = np.random.default_rng(3)
    xs = rng.standard_normal(n0 * n1 * n2).astype(np.float32)
    ts = {"x": torch.from_numpy(xs).cuda(), "r": torch.zeros(n0 * n2, device="cuda")}
    g.build({k: ts[k].data_ptr() for k in g.values})()
    torch.cuda.synchronize()
    X = xs.astype(np.float64).reshape(n2, n1, n0)
    want = (X * X[:, :1, :]).sum(axis=1)  # (n2, n0): r[i0 + n0 * i2]
    assert relative(ts["r"].cpu().numpy().reshape(n2, n0), want) < TOL


@pytest.mark.parametrize("n,m,dtype", [(1000, 3, "f32"), (4099, 2, "bf16"), (64, 5, "f32")])
def test_parallel_scans_of_every_fold(target, n, m, dtype):
    """The workgroup-parallel scan's other folds: a running log-sum-exp (the
    exponential fold, -inf identities in idle lanes), the running mean and
    squared deviations (the square fold), a running product and a running
    minimum, at lengths that leave idle lanes in the last chunk, from fp32 or
    bf16 values."""
    from tempest_hip.floor import FloorGroup
    announce("floor parallel scan folds", n, m, dtype)
    rng = np.random.default_rng(n * 31 + m)
    x = rng.standard_normal(n * m).astype(np.float32)
    p = (0.95 + 0.1 * rng.random(n * m)).astype(np.float32)
    if dtype == "bf16":
        x, p = bf16_round(x), bf16_round(p)
    g = FloorGroup("scan", (n, m), reduced=(0,))
    g.value("x", dtype, n * m)
    g.value("p", dtype, n * m)
    for k in ("lse", "mean", "dev", "prod", "min"):
        g.value(k, "f32", n * m)
    xx, pp = g.load("x", (1, n)), g.load("p", (1, n))
    e = g.fold("exp", xx, scan="inclusive")
    s = g.fold("square", xx, scan="inclusive")
    q = g.fold("prod", pp, scan="inclusive")
    lo = g.fold("min", xx, scan="inclusive")
    g.output("lse", e.logsumexp, (1, n))
    g.output("mean", s.statistic, (1, n))
    g.output("dev", s.sum, (1, n))
    g.output("prod", q.value, (1, n))
    g.output("min", lo.value, (1, n))
    assert "a workgroup per item" in g.source().splitlines()[0]
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    ts = {"x": torch.from_numpy(x).cuda().to(tdt), "p": torch.from_numpy(p).cuda().to(tdt)}
    for k in ("lse", "mean", "dev", "prod", "min"):
        ts[k] = torch.zeros(n * m, device="cuda")
    g.build({k: ts[k].data_ptr() for k in g.values})()
    torch.cuda.synchronize()
    X, Pm = x.astype(np.float64).reshape(m, n), p.astype(np.float64).reshape(m, n)
    cnt = np.arange(1, n + 1)
    mean = np.cumsum(X, axis=1) / cnt
    dev = np.cumsum(X * X, axis=1) - cnt * mean * mean
    got = {k: ts[k].cpu().numpy().astype(np.float64).reshape(m, n) for k in ("lse", "mean", "dev", "prod", "min")}
    assert relative(got["lse"], np.logaddexp.accumulate(X, axis=1)) < TOL
    assert relative(got["mean"], mean) < 1e-4  # a running mean of up to 4099 terms in fp32
    assert relative(got["dev"], dev) < 1e-4
    assert relative(got["prod"], np.cumprod(Pm, axis=1)) < 1e-4
    assert np.array_equal(got["min"], np.minimum.accumulate(X, axis=1))


@pytest.mark.parametrize("shape,axis", [((5000, 37), 0), ((37, 5000), 1), ((300, 700), 0)])
def test_extreme_folds_merge_like_base(target, shape, axis):
    """findmax / findmin folds over rows (lanes merged by shuffles), over
    columns (lanes merged through LDS), on elements full of ties, signed zeros
    and NaNs: the extreme and the first index where it is, as Base finds them."""
    from oracle import floor_groups as FG
    from tempest_hip.floor import FloorGroup
    n, m = shape
    announce("floor extreme folds", shape, axis)
    rng = np.random.default_rng(n + 3 * m)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 3.0, -np.inf], dtype=np.float32)
    x = pool[rng.integers(0, len(pool), n * m)]
    x[rng.integers(0, n * m, 5)] = np.nan
    g = FloorGroup("reduction", shape, reduced=(axis,))
    g.value("x", "f32", n * m)
    items = m if axis == 0 else n
    for k in ("vmax", "imax", "vmin", "imin"):
        g.value(k, "f32", items)
    xx = g.load("x", (1, n))
    pos = g.index((1, 0) if axis == 0 else (0, 1), 1)
    hi = g.fold("argmax", xx, weight=pos)
    lo = g.fold("argmin", xx, weight=pos)
    at = (0, 1) if axis == 0 else (1, 0)
    for k, t in (("vmax", hi.value), ("imax", hi.index), ("vmin", lo.value), ("imin", lo.index)):
        g.output(k, t, at, full=False)
    ts = {"x": torch.from_numpy(x).cuda()}
    for k in ("vmax", "imax", "vmin", "imin"):
        ts[k] = torch.zeros(items, device="cuda")
    g.build({k: ts[k].data_ptr() for k in g.values})()
    torch.cuda.synchronize()
    X = x.astype(np.float64).reshape(m, n).T  # X[i0, i1]
    idx = (np.arange(n)[:, None] + 1.0) * np.ones((1, m)) if axis == 0 else np.ones((n, 1)) * (np.arange(m)[None] + 1.0)
    for kind, v, i in (("argmax", "vmax", "imax"), ("argmin", "vmin", "imin")):
        st = FG.fold_reduce(kind, X, idx, (axis,))
        want_v, want_i = st["value"].ravel(), st["statistic"].ravel()
        got_v, got_i = ts[v].cpu().numpy().astype(np.float64), ts[i].cpu().numpy().astype(np.float64)
        assert np.array_equal(got_i, want_i), kind
        assert np.array_equal(np.isnan(got_v), np.isnan(want_v))
        ok = ~np.isnan(want_v)
        assert np.array_equal(got_v[ok], want_v[ok]) and np.array_equal(np.signbit(got_v[ok]), np.signbit(want_v[ok]))


def test_extreme_fold_split_over_parts(target):
    """findmax over 2^22 elements in one item: the positions split among
    workgroups, the parts' states merged by a second launch."""
    from tempest_hip.floor import FloorGroup
    n = 1 << 22
    announce("floor extreme fold in parts", n)
    rng = np.random.default_rng(12)
    x = rng.integers(0, 1000, n).astype(np.float32)
    g = FloorGroup("reduction", (n,), reduced=(0,))
    g.value("x", "f32", n)
    g.value("r", "f32", 2)
    f = g.fold("argmax", g.load("x", (1,)), weight=g.index((1,), 1))
    g.output("r", f.value, (0,), full=False)
    g.output("r", f.index, (0,), constant=1, full=False)
    assert "parts" in g.source().splitlines()[0] and ", parts 1," not in g.source().splitlines()[0]
    ts = {"x": torch.from_numpy(x).cuda(), "r": torch.zeros(2, device="cuda")}
    g.build({k: ts[k].data_ptr() for k in g.values})()
    torch.cuda.synchronize()
    r = ts["r"].cpu().numpy()
    assert r[0] == x.max() and r[1] == float(np.argmax(x) + 1)  # the first of the equal maxima
