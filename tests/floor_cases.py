"""The reference's fixture programs, planned as generated-floor groups.

Each case is a program of test/fixtures/programs.jl:60-90 (and the row
programs of config 2) written as the groups the floor would run: a list of
FloorGroups run in order over named values, the inputs (the reference tests'
closed-form ``data()``), and a closed form of the result written directly
with numpy, independent of the groups, that pins the oracle's evaluation.

Arrays are column-major as in the reference: an n x m array is stored with
element (i0, i1) at i0 + n * i1 (numpy: ``a.ravel(order="F")``).
"""
from __future__ import annotations

import numpy as np

from oracle.data import data
from tempest_hip.floor import FloorGroup


def F(a):
    return np.asarray(a, dtype=np.float64).ravel(order="F")


class Case:
    def __init__(self, name, groups, inputs, stored, results, closed, dtypes=None):
        self.name = name
        self.groups = groups        # FloorGroups, in order
        self.inputs = inputs        # name -> 1-D float64
        self.stored = stored        # name -> length (intermediates, zero-filled)
        self.results = results      # names checked
        self.closed = closed        # inputs -> {name: expected}
        self.dtypes = dtypes or {}  # name -> "bf16" (default "f32")

    def lengths(self):
        out = {k: len(v) for k, v in self.inputs.items()}
        out.update(self.stored)
        return out


def _full_sum(src: str, n: int, dst: str = "loss", extra: str | None = None) -> FloorGroup:
    """loss = sum(src) (+ extra[0]): the full fold after a row group."""
    g = FloorGroup("reduction", (n,), reduced=(0,), name=f"sum({src})")
    g.value(src, "f32", n)
    if extra:
        g.value(extra, "f32", 1)
    g.value(dst, "f32", 1)
    s = g.fold("sum", g.load(src, (1,))).value
    g.output(dst, s + g.load(extra, (0,)) if extra else s, full=False)
    return g


def _whole(name, shape, build, inputs, closed, dst="loss"):
    """One group folding every axis into a number."""
    g = FloorGroup("reduction", shape, reduced=tuple(range(len(shape))), name=name)
    for k, v in inputs.items():
        g.value(k, "f32", len(v))
    g.value(dst, "f32", 1)
    g.output(dst, build(g), full=False)
    return Case(name, [g], inputs, {dst: 1}, [dst], closed)


def _lin(shape):
    """Column-major coefficients of a dense array of `shape`."""
    c, s = [], 1
    for e in shape:
        c.append(s)
        s *= e
    return c


def dot_product():
    a, b = data(32), data(32, scale=0.3)
    return _whole("dot product", (32,), lambda g: g.fold("sum", g.load("a", (1,)) * g.load("b", (1,))).value,
                  {"a": F(a), "b": F(b)}, lambda v: {"loss": [np.sum(v["a"] * v["b"])]})


def sum_abs2_tanh():
    x = data(8, 6)
    return _whole("sum abs2 tanh", (8, 6),
                  lambda g: g.fold("sum", g.apply("abs2", g.apply("tanh", g.load("x", (1, 8))))).value,
                  {"x": F(x)}, lambda v: {"loss": [np.sum(np.tanh(v["x"]) ** 2)]})


def full_logsumexp():
    x = data(8, 6)

    def closed(v):
        m = v["x"].max()
        return {"loss": [m + np.log(np.sum(np.exp(v["x"] - m)))]}
    return _whole("full logsumexp", (8, 6), lambda g: g.fold("exp", g.load("x", (1, 8))).logsumexp,
                  {"x": F(x)}, closed)


def maximum_and_shifted_sum():
    x = data(8, 6)

    def build(g):
        xx = g.load("x", (1, 8))
        m = g.fold("max", xx).value
        return g.fold("sum", g.apply("exp", xx - m), phase=2).value
    return _whole("maximum and shifted sum", (8, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum(np.exp(v["x"] - v["x"].max()))]})


def minus_mean():
    x = data(8, 6)

    def build(g):
        xx = g.load("x", (1, 8))
        s = g.fold("sum", xx).value
        return g.fold("sum", g.apply("abs2", xx - s / 48.0), phase=2).value
    return _whole("x .- mean", (8, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum((v["x"] - v["x"].mean()) ** 2)]})


def swish():
    x = data(8, 6)
    return _whole("swish", (8, 6), lambda g: g.fold("sum", (lambda t: t / (1.0 + g.apply("exp", -t)))(
        g.load("x", (1, 8)))).value, {"x": F(x)}, lambda v: {"loss": [np.sum(v["x"] / (1 + np.exp(-v["x"])))]})


def powers():
    x = data(8, 6)

    def build(g):
        t = g.load("x", (1, 8))
        return g.fold("sum", t ** 2.0 + t ** 3.0 + g.apply("sqrt", g.apply("abs", t) + 1.0)).value
    return _whole("powers", (8, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum(v["x"] ** 2 + v["x"] ** 3 + np.sqrt(np.abs(v["x"]) + 1))]})


def clamp_and_max():
    x = data(8, 6)

    def build(g):
        t = g.load("x", (1, 8))
        return g.fold("sum", g.apply("clamp", t, -0.5, 0.5) + g.apply("max", t, 0.1)).value
    return _whole("clamp and max", (8, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum(np.clip(v["x"], -0.5, 0.5) + np.maximum(v["x"], 0.1))]})


def strided_view_and_index():
    """sum(abs2, view(x, 2:2:8, :) .+ x[3, 2]): rows 1, 3, 5, 7 (zero-based) and element (2, 1)."""
    x = data(8, 6)

    def build(g):
        v = g.load("x", (2, 8), constant=1)
        s = g.load("x", (0, 0), constant=2 + 8 * 1)
        return g.fold("sum", g.apply("abs2", v + s)).value
    return _whole("strided view and index", (4, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum((v["x"].reshape(8, 6, order="F")[1::2, :] +
                                              v["x"].reshape(8, 6, order="F")[2, 1]) ** 2)]})


def rounded_counted_tested():
    """sum(abs2, x .* round.(3x)) + count(>(0), x) * sum(x) + all(x .< 3) * sum(abs2, x)
    + sum(any(x .> 1; dims = 1) .* x) (programs.jl:63-64; round to Int32 is to
    nearest, ties to even, as Julia's round)."""
    x = data(8, 6)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="whole-array folds")
    g1.value("x", "f32", 48)
    g1.value("part", "f32", 1)
    t = g1.load("x", (1, 8))
    a = g1.fold("sum", g1.apply("abs2", t * g1.apply("round", 3.0 * t))).value
    c = g1.fold("sum", g1.apply(">", t, 0.0)).value
    s = g1.fold("sum", t).value
    al = g1.fold("min", g1.apply("<", t, 3.0)).value
    q = g1.fold("sum", g1.apply("abs2", t)).value
    g1.output("part", a + c * s + al * q, full=False)
    g2 = FloorGroup("reduction", (8, 6), reduced=(0,), name="any per column")
    g2.value("x", "f32", 48)
    g2.value("r", "f32", 6)
    t2 = g2.load("x", (1, 8))
    anyc = g2.fold("max", g2.apply(">", t2, 1.0)).value
    g2.output("r", g2.fold("sum", anyc * t2, phase=2).value, (0, 1), full=False)
    g3 = _full_sum("r", 6, extra="part")

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        r = np.sum(X * np.rint(3 * X) * X * np.rint(3 * X)) + np.sum(X > 0) * X.sum() + \
            float(np.all(X < 3)) * np.sum(X ** 2) + np.sum(np.any(X > 1, axis=0)[None, :] * X)
        return {"loss": [r]}
    return Case("rounded, counted and tested", [g1, g2, g3], {"x": F(x)}, {"part": 1, "r": 6, "loss": 1},
                ["loss"], closed)


def _column_then_sum(name, shape, reduced, build_row, inputs, closed, items):
    g1 = FloorGroup("reduction", shape, reduced=reduced, name=name)
    for k, v in inputs.items():
        g1.value(k, "f32", len(v))
    g1.value("r", "f32", items)
    build_row(g1)
    g2 = _full_sum("r", items)
    return Case(name, [g1, g2], inputs, {"r": items, "loss": 1}, ["r", "loss"], closed)


def column_maxima():
    x, w = data(8, 6), data(1, 6)

    def row(g):
        m = g.fold("max", g.load("x", (1, 8))).value
        g.output("r", m * g.load("w", (0, 1)), (0, 1), full=False)

    def closed(v):
        r = v["x"].reshape(8, 6, order="F").max(axis=0) * v["w"]
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("column maxima", (8, 6), (0,), row, {"x": F(x), "w": F(w)}, closed, 6)


def row_minima():
    x = data(8, 6)

    def row(g):
        g.output("r", g.fold("min", g.load("x", (1, 8))).value, (1, 0), full=False)

    def closed(v):
        r = v["x"].reshape(8, 6, order="F").min(axis=1)
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("row minima", (8, 6), (1,), row, {"x": F(x)}, closed, 8)


def products():
    x = data(5, 3, scale=0.4)

    def row(g):
        g.output("r", g.fold("prod", g.load("x", (1, 5))).value, (0, 1), full=False)

    def closed(v):
        r = v["x"].reshape(5, 3, order="F").prod(axis=0)
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("products", (5, 3), (0,), row, {"x": F(x)}, closed, 3)


def _softmax_closed(x, t, shape, axis):
    X, T = x.reshape(shape, order="F"), t.reshape(shape, order="F")
    e = np.exp(X - X.max(axis=axis, keepdims=True))
    y = e / e.sum(axis=axis, keepdims=True)
    return (y * T).sum(axis=axis)


def softmax_columns(n=8, m=6):
    x, t = data(n, m), data(n, m, scale=0.7)

    def row(g):
        xx, tt = g.load("x", (1, n)), g.load("t", (1, n))
        e = g.fold("exp", xx)
        g.output("r", g.fold("sum", g.apply("exp", xx - e.logsumexp) * tt, phase=2).value, (0, 1), full=False)

    def closed(v):
        r = _softmax_closed(v["x"], v["t"], (n, m), 0)
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum(f"softmax columns {n}x{m}", (n, m), (0,), row, {"x": F(x), "t": F(t)}, closed, m)


def softmax_rows(n=8, m=6):
    """Softmax over dims = 2: the folded axis is the strided one (items adjacent)."""
    x, t = data(n, m), data(n, m, scale=0.7)

    def row(g):
        xx, tt = g.load("x", (1, n)), g.load("t", (1, n))
        e = g.fold("exp", xx)
        g.output("r", g.fold("sum", g.apply("exp", xx - e.logsumexp) * tt, phase=2).value, (1, 0), full=False)

    def closed(v):
        r = _softmax_closed(v["x"], v["t"], (n, m), 1)
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum(f"softmax rows {n}x{m}", (n, m), (1,), row, {"x": F(x), "t": F(t)}, closed, n)


def rank3_softmax():
    """sum(exp.(x .- logsumexp(x; dims = 3)) .* t), x 4 x 3 x 5: the last axis folds."""
    x, t = data(4, 3, 5), data(4, 3, 5, scale=0.2)

    def row(g):
        xx, tt = g.load("x", (1, 4, 12)), g.load("t", (1, 4, 12))
        e = g.fold("exp", xx)
        g.output("r", g.fold("sum", g.apply("exp", xx - e.logsumexp) * tt, phase=2).value, (1, 4, 0), full=False)

    def closed(v):
        r = _softmax_closed(v["x"], v["t"], (4, 3, 5), 2).ravel(order="F")
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("rank 3 softmax", (4, 3, 5), (2,), row, {"x": F(x), "t": F(t)}, closed, 12)


def rmsnorm():
    x, w = data(8, 6), data(8, scale=0.1)

    def row(g):
        xx = g.load("x", (1, 8))
        s = g.fold("sum", g.apply("abs2", xx)).value
        y = xx / g.apply("sqrt", s / 8.0 + 1e-5) * g.load("w", (1, 0))
        g.output("r", g.fold("sum", g.apply("abs2", y), phase=2).value, (0, 1), full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        y = X / np.sqrt((X ** 2).sum(axis=0, keepdims=True) / 8 + 1e-5) * v["w"][:, None]
        r = (y ** 2).sum(axis=0)
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("RMSNorm", (8, 6), (0,), row, {"x": F(x), "w": F(w)}, closed, 6)


def _layernorm_closed(v, n, m):
    X = v["x"].reshape(n, m, order="F")
    mu = X.mean(axis=0, keepdims=True)
    var = ((X - mu) ** 2).mean(axis=0, keepdims=True)
    y = (X - mu) / np.sqrt(var + 1e-5) * v["w"][:, None]
    r = (y ** 2).sum(axis=0)
    return {"r": r, "loss": [r.sum()]}


def layer_norm(n=8, m=6):
    x, w = data(n, m), data(n, scale=0.1)

    def row(g):
        xx = g.load("x", (1, n))
        mu = g.fold("sum", xx).value / float(n)
        var = g.fold("sum", g.apply("abs2", xx - mu), phase=2).value / float(n)
        y = (xx - mu) / g.apply("sqrt", var + 1e-5) * g.load("w", (1, 0))
        g.output("r", g.fold("sum", g.apply("abs2", y), phase=3).value, (0, 1), full=False)
    return _column_then_sum(f"layer norm {n}x{m}", (n, m), (0,), row, {"x": F(x), "w": F(w)},
                            lambda v: _layernorm_closed(v, n, m), m)


def layer_norm_welford(n=8, m=6):
    """The same LayerNorm with mean and variance from one square fold (Chan/Welford)."""
    x, w = data(n, m), data(n, scale=0.1)

    def row(g):
        xx = g.load("x", (1, n))
        f = g.fold("square", xx)
        y = (xx - f.statistic) / g.apply("sqrt", f.sum / float(n) + 1e-5) * g.load("w", (1, 0))
        g.output("r", g.fold("sum", g.apply("abs2", y), phase=2).value, (0, 1), full=False)
    return _column_then_sum(f"layer norm by Welford {n}x{m}", (n, m), (0,), row, {"x": F(x), "w": F(w)},
                            lambda v: _layernorm_closed(v, n, m), m)


def welford_variance():
    """sum(var(x; dims = 1) .* data(1, 6)), var = M2 / n as VARIANCE observes it."""
    x, w = data(8, 6), data(1, 6)

    def row(g):
        f = g.fold("square", g.load("x", (1, 8)))
        g.output("r", f.sum / 8.0 * g.load("w", (0, 1)), (0, 1), full=False)

    def closed(v):
        r = v["x"].reshape(8, 6, order="F").var(axis=0) * v["w"]
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("Welford's variance", (8, 6), (0,), row, {"x": F(x), "w": F(w)}, closed, 6)


def map_over_two_arrays():
    """sum(abs2, map((a, b) -> a * b + a, x, y)): a pointwise group, then the fold."""
    x, y = data(8, 6), data(8, 6, scale=0.4)
    g1 = FloorGroup("pointwise", (8, 6), name="a * b + a")
    for k in ("x", "y", "z"):
        g1.value(k, "f32", 48)
    a, b = g1.load("x", (1, 8)), g1.load("y", (1, 8))
    g1.output("z", a * b + a, (1, 8))
    g2 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="sum abs2")
    g2.value("z", "f32", 48)
    g2.value("loss", "f32", 1)
    g2.output("loss", g2.fold("sum", g2.apply("abs2", g2.load("z", (1, 8)))).value, full=False)

    def closed(v):
        z = v["x"] * v["y"] + v["x"]
        return {"z": z, "loss": [np.sum(z ** 2)]}
    return Case("map over two arrays", [g1, g2], {"x": F(x), "y": F(y)}, {"z": 48, "loss": 1}, ["z", "loss"], closed)


def permutation():
    """permutedims(x, (2, 1, 3)) of a 4 x 3 x 5 array: y (3 x 4 x 5)[j0, j1, j2] = x[j1, j0, j2]."""
    x = data(4, 3, 5)
    g = FloorGroup("pointwise", (3, 4, 5), name="permutedims")
    g.value("x", "f32", 60)
    g.value("y", "f32", 60)
    g.output("y", g.load("x", (4, 1, 12)), (1, 3, 12))
    return Case("permutation", [g], {"x": F(x)}, {"y": 60}, ["y"],
                lambda v: {"y": v["x"].reshape(4, 3, 5, order="F").transpose(1, 0, 2).ravel(order="F")})


def permutation_and_reshape():
    """reshape(permutedims(x, (2, 1, 3)), 3, 20) of a 4 x 3 x 5 array, then
    sum(abs2, y .* w): y[a, b] = x[b mod 4, a, b div 4], an address with a Div
    and a Mod atom of the position b; and the way back, z[(b mod 4) + 4a +
    12 (b div 4)] = y[a, b], the same atoms in a store (z == x)."""
    x, w = data(4, 3, 5), data(3, 20, scale=0.7)
    parts = [("mod", (0, 1), 4, 1), ("div", (0, 1), 4, 12)]
    g1 = FloorGroup("pointwise", (3, 20), name="reshape(permutedims(x, (2, 1, 3)), 3, 20)")
    g1.value("x", "f32", 60)
    g1.value("y", "f32", 60)
    g1.output("y", g1.load("x", (4, 0), parts=parts), (1, 3))
    g2 = FloorGroup("reduction", (3, 20), reduced=(0, 1), name="sum(abs2, y .* w)")
    for v in ("x", "w"):
        g2.value(v, "f32", 60)
    g2.value("loss", "f32", 1)
    g2.output("loss", g2.fold("sum", g2.apply("abs2", g2.load("x", (4, 0), parts=parts) * g2.load("w", (1, 3)))).value,
              full=False)
    g3 = FloorGroup("pointwise", (3, 20), name="the way back")
    g3.value("y", "f32", 60)
    g3.value("z", "f32", 60)
    g3.output("z", g3.load("y", (1, 3)), (4, 0), parts=parts)

    def closed(v):
        y = v["x"].reshape(4, 3, 5, order="F").transpose(1, 0, 2).reshape(3, 20, order="F")
        return {"y": y.ravel(order="F"), "loss": [np.sum((y * v["w"].reshape(3, 20, order="F")) ** 2)],
                "z": v["x"]}
    return Case("permutation and reshape (Div and Mod atoms)", [g1, g2, g3], {"x": F(x), "w": F(w)},
                {"y": 60, "loss": 1, "z": 60}, ["y", "loss", "z"], closed)


def permute_reshape_and_roll():
    """reshape(permutedims(x, (2, 1)), 2, 30) of a 6 x 10 array: y[a, b] =
    x[L mod 10, L div 10] ... read as x[L div 10 + 6 (L mod 10)] with L = a +
    2b, atoms of two positions; and a roll, r[a, b] = x[mod(a + 2b - 7, 60)],
    a Mod atom whose expression goes negative (floor division, remainder in
    0..59)."""
    x = data(6, 10)
    g = FloorGroup("pointwise", (2, 30), name="reshape(permutedims(x, (2, 1)), 2, 30) and a roll")
    g.value("x", "f32", 60)
    g.value("y", "f32", 60)
    g.value("r", "f32", 60)
    g.output("y", g.load("x", (0, 0), parts=[("div", (1, 2), 10, 1), ("mod", (1, 2), 10, 6)]), (1, 2))
    g.output("r", g.load("x", (0, 0), parts=[("mod", (1, 2), 60, 1, -7)]), (1, 2))

    def closed(v):
        y = v["x"].reshape(6, 10, order="F").T.reshape(2, 30, order="F")
        return {"y": y.ravel(order="F"), "r": np.roll(v["x"], 7)}
    return Case("permute, reshape and roll (Div and Mod of two positions)", [g], {"x": F(x)},
                {"y": 60, "r": 60}, ["y", "r"], closed)


def bias_tanh_bf16(n=64, m=40):
    """y = tanh.(x .+ b) with b a column broadcast along the rows, y stored as bfloat16."""
    x, b = data(n, m), data(n, scale=0.3)
    g = FloorGroup("pointwise", (n, m), name="tanh.(x .+ b) to bf16")
    g.value("x", "f32", n * m)
    g.value("b", "f32", n)
    g.value("y", "bf16", n * m)
    g.output("y", g.apply("tanh", g.load("x", (1, n)) + g.load("b", (1, 0))), (1, n))
    return Case("bias and tanh to bf16", [g], {"x": F(x), "b": F(b)}, {"y": n * m}, ["y"],
                lambda v: {"y": np.tanh(v["x"].reshape(n, m, order="F") + v["b"][:, None]).ravel(order="F")},
                dtypes={"y": "bf16"})


def index_scaled(n=12, m=5):
    """y = x .* (i .+ 1), the row's position as a number (Ix)."""
    x = data(n, m)
    g = FloorGroup("pointwise", (n, m), name="x .* position")
    g.value("x", "f32", n * m)
    g.value("y", "f32", n * m)
    g.output("y", g.load("x", (1, n)) * (g.index((1, 0)) + 1.0), (1, n))
    return Case("index scaled", [g], {"x": F(x)}, {"y": n * m}, ["y"],
                lambda v: {"y": (v["x"].reshape(n, m, order="F") * (np.arange(n)[:, None] + 1)).ravel(order="F")})


def kat_sum_abs2():
    """compile(x -> sum(abs2, x), ...)([1, 2, 3, 4]) == 30 (runtime/compile.jl:35-40)."""
    return _whole("sum(abs2, [1, 2, 3, 4])", (4,), lambda g: g.fold("sum", g.apply("abs2", g.load("x", (1,)))).value,
                  {"x": np.array([1.0, 2.0, 3.0, 4.0])}, lambda v: {"loss": [30.0]})


# ---- scan groups (scan_kernel, codegen/scalar.jl:350-398) ----------------------------

def cumulative_sums():
    """sum(cumsum(x; dims = 1) .* data(8, 6; scale = 0.3)) + sum(abs2, cumsum(x[:, 2]))."""
    x, w = data(8, 6), data(8, 6, scale=0.3)
    ga = FloorGroup("scan", (8, 6), reduced=(0,), name="cumsum(x; dims = 1) .* w, summed per column")
    ga.value("x", "f32", 48)
    ga.value("w", "f32", 48)
    ga.value("r", "f32", 6)
    c = ga.fold("sum", ga.load("x", (1, 8)), scan="inclusive")
    ga.output("r", ga.fold("sum", c.value * ga.load("w", (1, 8)), phase=2).value, (0, 1), full=False)
    gb = FloorGroup("scan", (8,), reduced=(0,), name="sum(abs2, cumsum(x[:, 2]))")
    gb.value("x", "f32", 48)
    gb.value("part", "f32", 1)
    c2 = gb.fold("sum", gb.load("x", (1,), constant=8), scan="inclusive")
    gb.output("part", gb.fold("sum", gb.apply("abs2", c2.value), phase=2).value, full=False)
    gc = _full_sum("r", 6, extra="part")

    def closed(v):
        X, W = v["x"].reshape(8, 6, order="F"), v["w"].reshape(8, 6, order="F")
        return {"loss": [np.sum(np.cumsum(X, axis=0) * W) + np.sum(np.cumsum(X[:, 1]) ** 2)]}
    return Case("cumulative sums", [ga, gb, gc], {"x": F(x), "w": F(w)}, {"r": 6, "part": 1, "loss": 1},
                ["loss"], closed)


def cumulative_products_through_a_zero():
    """sum(cumprod(x; dims = 2) .* data(5, 4)), x with a zero at (2, 3)."""
    x = data(5, 4, scale=0.4)
    x[1, 2] = 0.0
    w = data(5, 4)
    g = FloorGroup("scan", (5, 4), reduced=(1,), name="cumprod along rows")
    g.value("x", "f32", 20)
    g.value("w", "f32", 20)
    g.value("r", "f32", 5)
    c = g.fold("prod", g.load("x", (1, 5)), scan="inclusive")
    g.output("r", g.fold("sum", c.value * g.load("w", (1, 5)), phase=2).value, (1, 0), full=False)

    def closed(v):
        X, W = v["x"].reshape(5, 4, order="F"), v["w"].reshape(5, 4, order="F")
        r = np.sum(np.cumprod(X, axis=1) * W, axis=1)
        return {"r": r, "loss": [r.sum()]}
    return Case("cumulative products through a zero", [g, _full_sum("r", 5)], {"x": F(x), "w": F(w)},
                {"r": 5, "loss": 1}, ["r", "loss"], closed)


def running_maxima_and_minima():
    """sum(accumulate(max, x; dims = 1) .* w) + sum of the running minimum in linear order."""
    x, w = data(8, 6, scale=0.7), data(8, 6, scale=0.3)
    ga = FloorGroup("scan", (8, 6), reduced=(0,), name="running maximum down columns")
    ga.value("x", "f32", 48)
    ga.value("w", "f32", 48)
    ga.value("r", "f32", 6)
    m = ga.fold("max", ga.load("x", (1, 8)), scan="inclusive")
    ga.output("r", ga.fold("sum", m.value * ga.load("w", (1, 8)), phase=2).value, (0, 1), full=False)
    gb = FloorGroup("scan", (8, 6), reduced=(0, 1), name="running minimum in linear order")
    gb.value("x", "f32", 48)
    gb.value("part", "f32", 1)
    mn = gb.fold("min", gb.load("x", (1, 8)), scan="inclusive")
    gb.output("part", gb.fold("sum", mn.value, phase=2).value, full=False)

    def closed(v):
        X, W = v["x"].reshape(8, 6, order="F"), v["w"].reshape(8, 6, order="F")
        return {"loss": [np.sum(np.maximum.accumulate(X, axis=0) * W) + np.sum(np.minimum.accumulate(v["x"]))]}
    return Case("running maxima and minima", [ga, gb, _full_sum("r", 6, extra="part")], {"x": F(x), "w": F(w)},
                {"r": 6, "part": 1, "loss": 1}, ["loss"], closed)


def linear_recurrence():
    """sum(abs2, recurrence(a, b)): h = a h' + b from 0 (programs.jl:54-55, 86-88)."""
    a, b = 0.9 + 0.1 * data(30, scale=0.3), data(30, scale=0.7)
    g = FloorGroup("scan", (30,), reduced=(0,), name="h = a h' + b")
    g.value("a", "f32", 30)
    g.value("b", "f32", 30)
    g.value("h", "f32", 30)
    g.value("loss", "f32", 1)
    h = g.fold("linear", g.load("a", (1,)), weight=g.load("b", (1,)), scan="inclusive")
    g.output("h", h.value, (1,))
    g.output("loss", g.fold("sum", g.apply("abs2", h.value), phase=2).value, full=False)

    def closed(v):
        hs, hh = [], 0.0
        for ai, bi in zip(v["a"], v["b"]):
            hh = ai * hh + bi
            hs.append(hh)
        hs = np.array(hs)
        return {"h": hs, "loss": [np.sum(hs ** 2)]}
    return Case("a linear recurrence", [g], {"a": F(a), "b": F(b)}, {"h": 30, "loss": 1}, ["h", "loss"], closed)


def running_average():
    """sum(abs2, accumulate((s, e) -> s / 2 + e, x; dims = 2, init = 1)): h = h'/2 + e
    from 1, i.e. the linear fold's value plus its product (h from 0, plus 1 times
    the product of the halves)."""
    x = data(8, 6)
    g = FloorGroup("scan", (8, 6), reduced=(1,), name="running average along rows")
    g.value("x", "f32", 48)
    g.value("r", "f32", 8)
    h = g.fold("linear", g.lit(0.5), weight=g.load("x", (1, 8)), scan="inclusive")
    g.output("r", g.fold("sum", g.apply("abs2", h.value + h.product), phase=2).value, (1, 0), full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        hh = np.ones(8)
        tot = np.zeros(8)
        for j in range(6):
            hh = hh / 2 + X[:, j]
            tot += hh ** 2
        return {"r": tot, "loss": [tot.sum()]}
    return Case("a running average", [g, _full_sum("r", 8)], {"x": F(x)}, {"r": 8, "loss": 1}, ["r", "loss"], closed)


def reverse_exclusive_sums(n=9, m=5):
    """y[i, j] = sum of x[i', j] over i' > i: an exclusive scan from the last position."""
    x = data(n, m)
    g = FloorGroup("scan", (n, m), reduced=(0,), reverse=True, name="suffix sums, exclusive")
    g.value("x", "f32", n * m)
    g.value("y", "f32", n * m)
    c = g.fold("sum", g.load("x", (1, n)), scan="exclusive")
    g.output("y", c.value, (1, n))

    def closed(v):
        X = v["x"].reshape(n, m, order="F")
        return {"y": (np.cumsum(X[::-1], axis=0)[::-1] - X).ravel(order="F")}
    return Case("reverse exclusive sums", [g], {"x": F(x)}, {"y": n * m}, ["y"], closed)


def running_logsumexp_and_mean(n=12, m=4):
    """Running log-sum-exp (the exponential fold as a scan) and running mean
    (the square fold as a scan) down each column."""
    x = data(n, m) * 3
    g = FloorGroup("scan", (n, m), reduced=(0,), name="running logsumexp and mean")
    g.value("x", "f32", n * m)
    g.value("lse", "f32", n * m)
    g.value("mean", "f32", n * m)
    xx = g.load("x", (1, n))
    g.output("lse", g.fold("exp", xx, scan="inclusive").logsumexp, (1, n))
    g.output("mean", g.fold("square", xx, scan="inclusive").statistic, (1, n))

    def closed(v):
        X = v["x"].reshape(n, m, order="F")
        lse = np.logaddexp.accumulate(X, axis=0)
        mean = np.cumsum(X, axis=0) / np.arange(1, n + 1)[:, None]
        return {"lse": lse.ravel(order="F"), "mean": mean.ravel(order="F")}
    return Case("running logsumexp and mean", [g], {"x": F(x)}, {"lse": n * m, "mean": n * m}, ["lse", "mean"], closed)


# ---- gathers (Indirect atoms) and folds by key -------------------------------------

def _idx(a):
    return np.asarray(a, dtype=np.int64).ravel(order="F")


def gather_by_a_list():
    """sum(abs2, x[:, [3, 1, 3, 6]]): the columns by a list of (1-based) indices."""
    x, i = data(8, 6), _idx([3, 1, 3, 6])
    g = FloorGroup("reduction", (8, 4), reduced=(0, 1), name="x[:, i]")
    g.value("x", "f32", 48)
    g.value("i", "i64", 4)
    g.value("loss", "f32", 1)
    col = g.load("i", (0, 1))
    g.output("loss", g.fold("sum", g.apply("abs2", g.load("x", (1, 0), constant=-8, gather=col, gather_coeff=8))).value,
             full=False)
    return Case("gather by a constant list", [g], {"x": F(x), "i": i}, {"loss": 1}, ["loss"],
                lambda v: {"loss": [np.sum(v["x"].reshape(8, 6, order="F")[:, [2, 0, 2, 5]] ** 2)]},
                dtypes={"i": "i64"})


def gather_by_an_int32_matrix():
    """sum(abs2, x[:, i]), i = Int32[2 5; 6 1; 1 1]: an 8 x 3 x 2 gather."""
    x, i = data(8, 6), np.array([[2, 5], [6, 1], [1, 1]])
    g = FloorGroup("reduction", (8, 3, 2), reduced=(0, 1, 2), name="x[:, i], i a matrix")
    g.value("x", "f32", 48)
    g.value("i", "i32", 6)
    g.value("loss", "f32", 1)
    col = g.load("i", (0, 1, 3))
    g.output("loss", g.fold("sum", g.apply("abs2", g.load("x", (1, 0, 0), constant=-8, gather=col,
                                                          gather_coeff=8))).value, full=False)
    return Case("gather by a traced Int32 matrix", [g], {"x": F(x), "i": _idx(i)}, {"loss": 1}, ["loss"],
                lambda v: {"loss": [np.sum(v["x"].reshape(8, 6, order="F")[:, i.ravel(order="F") - 1] ** 2)]},
                dtypes={"i": "i32"})


def gather_rows_by_an_int64_matrix():
    """sum(abs2, tanh.(x[i, :])), i = [8 1; 2 8]: rows gathered, a 2 x 2 x 6 array."""
    x, i = data(8, 6), np.array([[8, 1], [2, 8]])
    g = FloorGroup("reduction", (2, 2, 6), reduced=(0, 1, 2), name="x[i, :]")
    g.value("x", "f32", 48)
    g.value("i", "i64", 4)
    g.value("loss", "f32", 1)
    row = g.load("i", (1, 2, 0))
    xx = g.load("x", (0, 0, 8), constant=-1, gather=row, gather_coeff=1)
    g.output("loss", g.fold("sum", g.apply("abs2", g.apply("tanh", xx))).value, full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        return {"loss": [np.sum(np.tanh(X[i.ravel(order="F") - 1, :]) ** 2)]}
    return Case("gather rows by a traced Int64 matrix", [g], {"x": F(x), "i": _idx(i)}, {"loss": 1}, ["loss"],
                closed, dtypes={"i": "i64"})


def gather_by_linear_and_scalar_indices():
    """sum(abs2, x[i]) + x[2, t], i = [40, 3, 17], t = 5."""
    x = data(8, 6)
    g = FloorGroup("reduction", (3,), reduced=(0,), name="x[i] and x[2, t]")
    g.value("x", "f32", 48)
    g.value("i", "i64", 3)
    g.value("t", "i64", 1)
    g.value("loss", "f32", 1)
    s = g.fold("sum", g.apply("abs2", g.load("x", (0,), constant=-1, gather=g.load("i", (1,)), gather_coeff=1))).value
    xt = g.load("x", (0,), constant=1 - 8, gather=g.load("t", (0,)), gather_coeff=8)
    g.output("loss", s + xt, full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        return {"loss": [np.sum(v["x"][[39, 2, 16]] ** 2) + X[1, 4]]}
    return Case("gather by linear and scalar indices", [g], {"x": F(x), "i": _idx([40, 3, 17]), "t": _idx([5])},
                {"loss": 1}, ["loss"], closed, dtypes={"i": "i64", "t": "i64"})


def embedding_and_layer_norm():
    """sum(abs2, layernorm(E[:, t] .+ P, w)): E 8 x 10, P 8 x 3, t = Int32[3 1; 10 3; 7 7]."""
    E, P, w = data(8, 10, scale=0.3), data(8, 3, scale=0.2), data(8, scale=0.1)
    t = np.array([[3, 1], [10, 3], [7, 7]])
    g = FloorGroup("reduction", (8, 3, 2), reduced=(0,), name="layernorm(E[:, t] .+ P, w)")
    g.value("E", "f32", 80)
    g.value("P", "f32", 24)
    g.value("w", "f32", 8)
    g.value("t", "i32", 6)
    g.value("r", "f32", 6)
    tok = g.load("t", (0, 1, 3))
    xx = g.load("E", (1, 0, 0), constant=-8, gather=tok, gather_coeff=8) + g.load("P", (1, 8, 0))
    mu = g.fold("sum", xx).value / 8.0
    var = g.fold("sum", g.apply("abs2", xx - mu), phase=2).value / 8.0
    y = (xx - mu) / g.apply("sqrt", var + 1e-5) * g.load("w", (1, 0, 0))
    g.output("r", g.fold("sum", g.apply("abs2", y), phase=3).value, (0, 1, 3), full=False)

    def closed(v):
        Ev, Pv = v["E"].reshape(8, 10, order="F"), v["P"].reshape(8, 3, order="F")
        X = Ev[:, t - 1] + Pv[:, :, None]  # 8 x 3 x 2
        mu_ = X.mean(axis=0, keepdims=True)
        var_ = ((X - mu_) ** 2).mean(axis=0, keepdims=True)
        Y = (X - mu_) / np.sqrt(var_ + 1e-5) * v["w"][:, None, None]
        r = (Y ** 2).sum(axis=0).ravel(order="F")
        return {"r": r, "loss": [r.sum()]}
    return Case("embedding lookup and layer norm", [g, _full_sum("r", 6)],
                {"E": F(E), "P": F(P), "w": F(w), "t": _idx(t)}, {"r": 6, "loss": 1}, ["r", "loss"], closed,
                dtypes={"t": "i32"})


def scatter_add_gradient():
    """The gradient of x[:, i] with i = [3, 1, 3, 6]: dx[:, i] .+= dy, column 3
    twice (a fold by key, accumulate!(::SumFold))."""
    dy, i = data(8, 4, scale=0.5), _idx([3, 1, 3, 6])
    g = FloorGroup("pointwise", (8, 4), name="dx[:, i] .+= dy")
    g.value("dy", "f32", 32)
    g.value("i", "i64", 4)
    g.value("dx", "f32", 48)
    g.output("dx", g.load("dy", (1, 8)), (1, 0), constant=-8, gather=g.load("i", (0, 1)), gather_coeff=8,
             accumulate=True)

    def closed(v):
        dx = np.zeros((8, 6))
        np.add.at(dx.T, [2, 0, 2, 5], v["dy"].reshape(8, 4, order="F").T)
        return {"dx": dx.ravel(order="F")}
    return Case("scatter add (a fold by key)", [g], {"dy": F(dy), "i": i}, {"dx": 48}, ["dx"], closed,
                dtypes={"i": "i64"})


# ---- extremes and where they are (the `Better` fold, program/tracing.jl:735-790) ----

def extremes_and_where_they_are():
    """x -> sum(findmax(x; dims = 1)[1] .* data(1, 6)) + sum(getindex.(argmin(x;
    dims = 2), 2)) + x[argmax(x)] + argmin(abs, x) + sum(last.(extrema(x; dims
    = 2)) .* data(8)), x = data(8, 6) (test/fixtures/programs.jl:144-145).
    The element argmin(abs, x) finds is read by a gather at the index the fold
    stored."""
    x, w, d8 = data(8, 6), data(1, 6), data(8)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0,), name="findmax(x; dims = 1)")
    g1.value("x", "f32", 48)
    g1.value("w", "f32", 6)
    g1.value("r1", "f32", 6)
    fm = g1.fold("argmax", g1.load("x", (1, 8)), weight=g1.index((1, 0), 1))
    g1.output("r1", fm.value * g1.load("w", (0, 1)), (0, 1), full=False)
    g2 = FloorGroup("reduction", (8, 6), reduced=(1,), name="argmin(x; dims = 2), extrema(x; dims = 2)")
    g2.value("x", "f32", 48)
    g2.value("d8", "f32", 8)
    g2.value("r2", "f32", 8)
    xx = g2.load("x", (1, 8))
    am = g2.fold("argmin", xx, weight=g2.index((0, 1), 1))   # the column, 1-based
    mx = g2.fold("max", xx)
    g2.output("r2", am.index + mx.value * g2.load("d8", (1, 0)), (1, 0), full=False)
    g3 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="x[argmax(x)], argmin(abs, x)")
    g3.value("x", "f32", 48)
    g3.value("s", "f32", 3)
    x3 = g3.load("x", (1, 8))
    lin = g3.index((1, 8), 1)
    g3.output("s", g3.fold("argmax", x3, weight=lin).value, (0, 0), full=False)
    g3.output("s", g3.fold("argmin", g3.apply("abs", x3), weight=lin).index, (0, 0), constant=1, full=False)
    g5 = FloorGroup("reduction", (6,), reduced=(0,), name="sum(r1)")
    g5.value("r1", "f32", 6)
    g5.value("s", "f32", 3)
    g5.output("s", g5.fold("sum", g5.load("r1", (1,))).value, (0,), constant=2, full=False)
    g4 = FloorGroup("reduction", (8,), reduced=(0,), name="the sum")
    for k, n in (("x", 48), ("s", 3), ("r2", 8), ("loss", 1)):
        g4.value(k, "f32", n)
    at = g4.load("x", (0,), constant=-1, gather=g4.load("s", (0,), constant=1), gather_coeff=1)
    total = g4.fold("sum", g4.load("r2", (1,))).value + g4.load("s", (0,), constant=2) + g4.load("s", (0,)) + at
    g4.output("loss", total, (0,), full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        r1_ = X.max(axis=0) * v["w"]
        r2_ = (np.argmin(X, axis=1) + 1) + X.max(axis=1) * v["d8"]
        i = int(np.argmin(np.abs(v["x"])))
        s_ = [X.max(), i + 1, r1_.sum()]
        return {"r1": r1_, "r2": r2_, "s": s_, "loss": [r1_.sum() + r2_.sum() + s_[0] + v["x"][i]]}
    return Case("extremes and where they are", [g1, g2, g3, g5, g4], {"x": F(x), "w": F(w), "d8": F(d8)},
                {"r1": 6, "r2": 8, "s": 3, "loss": 1}, ["r1", "r2", "s", "loss"], closed)


def extremes_of_a_vector():
    """v -> v[argmax(v)] * findmin(v)[2] + sum(extrema(v)) + findmax(abs2, v)[1],
    v = data(30) (test/fixtures/programs.jl:146)."""
    v0 = data(30)
    g = FloorGroup("reduction", (30,), reduced=(0,), name="extremes of a vector")
    g.value("v", "f32", 30)
    g.value("loss", "f32", 1)
    v = g.load("v", (1,))
    i = g.index((1,), 1)
    a = g.fold("argmax", v, weight=i).value
    b = g.fold("argmin", v, weight=i).index
    ext = g.fold("min", v).value + g.fold("max", v).value
    c = g.fold("argmax", g.apply("abs2", v), weight=i).value
    g.output("loss", a * b + ext + c, (0,), full=False)

    def closed(val):
        u = val["v"]
        return {"loss": [u[np.argmax(u)] * (np.argmin(u) + 1) + u.min() + u.max() + (u ** 2).max()]}
    return Case("the extremes of a vector", [g], {"v": F(v0)}, {"loss": 1}, ["loss"], closed)


# ---- writes (test/fixtures/programs.jl:119-131): stores at addresses of their own ----

def _copy(src, dst, shape):
    """dst = copy(src): a pointwise group over `shape`."""
    g = FloorGroup("pointwise", shape, name=f"{dst} = copy({src})")
    n = int(np.prod(shape))
    g.value(src, "f32", n)
    g.value(dst, "f32", n)
    g.output(dst, g.load(src, _lin(shape)), _lin(shape))
    return g


def _fill(dst, shape, value):
    g = FloorGroup("pointwise", shape, name=f"{dst} .= {value}")
    g.value(dst, "f32", int(np.prod(shape)))
    g.output(dst, value, _lin(shape))
    return g


def _loss(shape, names, build):
    """loss = sum over `shape` of build(g, loads...), one group."""
    g = FloorGroup("reduction", shape, reduced=tuple(range(len(shape))), name="loss")
    n = int(np.prod(shape))
    for k in names:
        g.value(k, "f32", n)
    g.value("loss", "f32", 1)
    g.output("loss", g.fold("sum", build(g, *[g.load(k, _lin(shape)) for k in names])).value, full=False)
    return g


def write_of_a_slice():
    """y = copy(x); y[2:4, :] = v; sum(abs2, tanh.(y))."""
    x, v = data(8, 6), data(3, 6, scale=0.3)
    w = FloorGroup("pointwise", (3, 6), name="y[2:4, :] = v")
    w.value("v", "f32", 18)
    w.value("y", "f32", 48)
    w.output("y", w.load("v", (1, 3)), (1, 8), constant=1)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        Y[1:4, :] = val["v"].reshape(3, 6, order="F")
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.tanh(Y) ** 2)]}
    return Case("a write of a slice", [_copy("x", "y", (8, 6)), w,
                                       _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("tanh", y)))],
                {"x": F(x), "v": F(v)}, {"y": 48, "loss": 1}, ["y", "loss"], closed)


def padding_by_a_write():
    """y = zeros(10, 8); y[2:9, 2:7] = x; sum(abs2, y .* data(10, 8))."""
    x, d = data(8, 6), data(10, 8)
    w = FloorGroup("pointwise", (8, 6), name="y[2:end-1, 2:end-1] = x")
    w.value("x", "f32", 48)
    w.value("y", "f32", 80)
    w.output("y", w.load("x", (1, 8)), (1, 10), constant=11)

    def closed(val):
        Y = np.zeros((10, 8))
        Y[1:9, 1:7] = val["x"].reshape(8, 6, order="F")
        return {"y": Y.ravel(order="F"), "loss": [np.sum((Y * val["d"].reshape(10, 8, order="F")) ** 2)]}
    return Case("padding by a write", [_fill("y", (10, 8), 0.0), w,
                                       _loss((10, 8), ["y", "d"], lambda g, y, dd: g.apply("abs2", y * dd))],
                {"x": F(x), "d": F(d)}, {"y": 80, "loss": 1}, ["y", "loss"], closed)


def writes_through_views():
    """y = zero(x); view(y, :, 2:3) .= x[:, 1:2] .* 2; y[1, :] .= 1; sum(abs2, y .+ x)."""
    x = data(8, 6)
    w1 = FloorGroup("pointwise", (8, 2), name="view(y, :, 2:3) .= x[:, 1:2] .* 2")
    w1.value("x", "f32", 48)
    w1.value("y", "f32", 48)
    w1.output("y", w1.load("x", (1, 8)) * 2.0, (1, 8), constant=8)
    w2 = FloorGroup("pointwise", (6,), name="y[1, :] .= 1")
    w2.value("y", "f32", 48)
    w2.output("y", 1.0, (8,))

    def closed(val):
        X = val["x"].reshape(8, 6, order="F")
        Y = np.zeros((8, 6))
        Y[:, 1:3] = X[:, 0:2] * 2
        Y[0, :] = 1
        return {"y": Y.ravel(order="F"), "loss": [np.sum((Y + X) ** 2)]}
    return Case("writes through views", [_fill("y", (8, 6), 0.0), w1, w2,
                                         _loss((8, 6), ["y", "x"], lambda g, y, xx: g.apply("abs2", y + xx))],
                {"x": F(x)}, {"y": 48, "loss": 1}, ["y", "loss"], closed)


def strided_and_reversed_writes():
    """y = copy(x); y[1:2:8, end:-2:1] = v; sum(abs2, sin.(y)): rows 1, 3, 5, 7
    and columns 6, 4, 2, an address with a negative coefficient."""
    x, v = data(8, 6), data(4, 3, scale=0.3)
    w = FloorGroup("pointwise", (4, 3), name="y[1:2:8, end:-2:1] = v")
    w.value("v", "f32", 12)
    w.value("y", "f32", 48)
    w.output("y", w.load("v", (1, 4)), (2, -16), constant=40)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        Y[0:8:2, 5::-2] = val["v"].reshape(4, 3, order="F")
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.sin(Y) ** 2)]}
    return Case("strided and reversed writes", [_copy("x", "y", (8, 6)), w,
                                                _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("sin", y)))],
                {"x": F(x), "v": F(v)}, {"y": 48, "loss": 1}, ["y", "loss"], closed)


def write_at_traced_positions():
    """y = copy(x); y[:, i] .= v; y[i[1], 1] = 2 * v[3]; sum(abs2, tanh.(y)),
    i = Int32[4, 1]: stores at gathered addresses, the last landing."""
    x, v, i = data(8, 6), data(8, 2, scale=0.3), _idx([4, 1])
    w1 = FloorGroup("pointwise", (8, 2), name="y[:, i] .= v")
    w1.value("v", "f32", 16)
    w1.value("i", "i32", 2)
    w1.value("y", "f32", 48)
    w1.output("y", w1.load("v", (1, 8)), (1, 0), constant=-8, gather=w1.load("i", (0, 1)), gather_coeff=8)
    w2 = FloorGroup("pointwise", (1,), name="y[i[1], 1] = 2 v[3]")
    w2.value("v", "f32", 16)
    w2.value("i", "i32", 2)
    w2.value("y", "f32", 48)
    w2.output("y", w2.load("v", (0,), constant=2) * 2.0, (0,), constant=-1, gather=w2.load("i", (0,)), gather_coeff=1)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        V = val["v"].reshape(8, 2, order="F")
        Y[:, [3, 0]] = V
        Y[3, 0] = 2 * val["v"][2]
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.tanh(Y) ** 2)]}
    return Case("a write at traced positions", [_copy("x", "y", (8, 6)), w1, w2,
                                                _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("tanh", y)))],
                {"x": F(x), "v": F(v), "i": i}, {"y": 48, "loss": 1}, ["y", "loss"], closed, dtypes={"i": "i32"})


def mean_divided_in_place():
    """r = sum(x; dims = 1); r ./= size(x, 1); sum(abs2, x .- r): a value
    written, then read and written again in place."""
    x = data(8, 6)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0,), name="r = sum(x; dims = 1)")
    g1.value("x", "f32", 48)
    g1.value("r", "f32", 6)
    g1.output("r", g1.fold("sum", g1.load("x", (1, 8))).value, (0, 1), full=False)
    g2 = FloorGroup("pointwise", (6,), name="r ./= 8")
    g2.value("r", "f32", 6)
    g2.output("r", g2.load("r", (1,)) / 8.0, (1,))
    g3 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="sum(abs2, x .- r)")
    g3.value("x", "f32", 48)
    g3.value("r", "f32", 6)
    g3.value("loss", "f32", 1)
    g3.output("loss", g3.fold("sum", g3.apply("abs2", g3.load("x", (1, 8)) - g3.load("r", (0, 1)))).value, full=False)

    def closed(val):
        X = val["x"].reshape(8, 6, order="F")
        r = X.sum(axis=0) / 8
        return {"r": r, "loss": [np.sum((X - r) ** 2)]}
    return Case("a mean divided in place", [g1, g2, g3], {"x": F(x)}, {"r": 6, "loss": 1}, ["r", "loss"], closed)


def permutedims_and_copyto():
    """y = permutedims(x) into a 6 x 8 array; z = copyto!(similar(x, 48), y);
    sum(abs2, z .* data(48))."""
    x, d = data(8, 6), data(48)
    g1 = FloorGroup("pointwise", (8, 6), name="permutedims!(y, x, (2, 1))")
    g1.value("x", "f32", 48)
    g1.value("y", "f32", 48)
    g1.output("y", g1.load("x", (1, 8)), (6, 1))

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").T
        z = Y.ravel(order="F")
        return {"y": z, "z": z, "loss": [np.sum((z * val["d"]) ** 2)]}
    return Case("permutedims! and copyto!", [g1, _copy("y", "z", (48,)),
                                             _loss((48,), ["z", "d"], lambda g, z, dd: g.apply("abs2", z * dd))],
                {"x": F(x), "d": F(d)}, {"y": 48, "z": 48, "loss": 1}, ["y", "z", "loss"], closed)


# ---- recomputed folds and recurrences ----------------------------------------------

def mean_recomputed():
    """x .- mean(x; dims = 1) with the mean recomputed where each element reads
    it (a Recomputed term, codegen/scalar.jl:88-110), then sum(abs2, .)."""
    x = data(8, 6)
    g = FloorGroup("pointwise", (8, 6), name="x .- mean, recomputed")
    g.value("x", "f32", 48)
    g.value("y", "f32", 48)
    mean = g.recompute("sum", g.load("x", (0, 8, 1)), inner=(8,)).value / 8.0
    g.output("y", g.load("x", (1, 8)) - mean, (1, 8))
    g2 = FloorGroup("reduction", (48,), reduced=(0,), name="sum(abs2, y)")
    g2.value("y", "f32", 48)
    g2.value("loss", "f32", 1)
    g2.output("loss", g2.fold("sum", g2.apply("abs2", g2.load("y", (1,)))).value, full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        Y = X - X.mean(axis=0)
        return {"y": Y.ravel(order="F"), "loss": [np.sum(Y ** 2)]}
    return Case("x .- mean, the mean recomputed", [g, g2], {"x": F(x)}, {"y": 48, "loss": 1}, ["y", "loss"], closed)


def recurrence_with_recomputed_sums():
    """h = tanh.(W' * unit(x[:, t]) .+ h) over the columns of x, unit(x) =
    x ./ sqrt(sum(abs2, x) + 1e-6) (test/cuda/folds.jl:85-99): a recurrence
    group stepping along t, its state's start stored at the first step, its
    new state carried one step on, the product and the norm recomputed in
    each step."""
    W, x, h0 = data(256, 64, scale=0.1), data(256, 4, scale=0.3), data(64, scale=0.2)
    g = FloorGroup("recurrence", (64, 4), reduced=(1,), step=1, name="h = tanh(W' unit(x[:, t]) + h)")
    for k, n in (("W", 256 * 64), ("x", 1024), ("h0", 64), ("H", 64 * 5), ("Y", 64 * 4)):
        g.value(k, "f32", n)
    prod = g.recompute("sum", g.load("W", (256, 0, 1)) * g.load("x", (0, 256, 1)), inner=(256,)).value
    norm = g.recompute("sum", g.apply("abs2", g.load("x", (0, 256, 1))), inner=(256,)).value
    h = g.apply("tanh", prod / g.apply("sqrt", norm + 1e-6) + g.load("H", (1, 64)))
    g.output("H", g.load("h0", (1, 0)), (1, 64), when="first")
    g.output("H", h, (1, 64), constant=64, when="carry")
    g.output("Y", h, (1, 64), when="each")

    def closed(v):
        Wm, X = v["W"].reshape(256, 64, order="F"), v["x"].reshape(256, 4, order="F")
        hh, H, Y = v["h0"].copy(), np.zeros((64, 5)), np.zeros((64, 4))
        H[:, 0] = hh
        for t in range(4):
            u = X[:, t] / np.sqrt(np.sum(X[:, t] ** 2) + 1e-6)
            hh = np.tanh(Wm.T @ u + hh)
            Y[:, t] = hh
            if t < 3:
                H[:, t + 1] = hh
        return {"H": H.ravel(order="F"), "Y": Y.ravel(order="F")}
    return Case("a recurrence whose steps recompute sums", [g], {"W": F(W), "x": F(x), "h0": F(h0)},
                {"H": 320, "Y": 256}, ["H", "Y"], closed)


def reverse_recurrence():
    """h = a h' + b stepped from the last position back (a carried state in
    reverse): h at t reads the state t + 1 left."""
    a, b, h0 = 0.9 + 0.1 * data(5, 7, scale=0.3), data(5, 7, scale=0.7), data(5, scale=0.5)
    g = FloorGroup("recurrence", (5, 7), reduced=(1,), step=1, reverse=True, name="h = a h' + b, reversed")
    for k, n in (("a", 35), ("b", 35), ("h0", 5), ("H", 35), ("Y", 35)):
        g.value(k, "f32", n)
    h = g.load("a", (1, 5)) * g.load("H", (1, 5)) + g.load("b", (1, 5))
    g.output("H", g.load("h0", (1, 0)), (1, 5), when="first")
    g.output("H", h, (1, 5), constant=-5, when="carry")
    g.output("Y", h, (1, 5), when="each")

    def closed(v):
        A, B = v["a"].reshape(5, 7, order="F"), v["b"].reshape(5, 7, order="F")
        H, Y, hh = np.zeros((5, 7)), np.zeros((5, 7)), v["h0"].copy()
        H[:, 6] = hh
        for t in range(6, -1, -1):
            hh = A[:, t] * hh + B[:, t]
            Y[:, t] = hh
            if t > 0:
                H[:, t - 1] = hh
        return {"H": H.ravel(order="F"), "Y": Y.ravel(order="F")}
    return Case("a recurrence in reverse", [g], {"a": F(a), "b": F(b), "h0": F(h0)}, {"H": 35, "Y": 35},
                ["H", "Y"], closed)


# ---- more of the fixture programs (test/fixtures/programs.jl:60-146) -----------------

def log_sum_exp_written_out():
    """sum(written_logsumexp(x; dims = 1) .* data(1, 6)), m + log(sum(exp(x - m))) by columns."""
    x, w = data(8, 6), data(1, 6)

    def row(g):
        xx = g.load("x", (1, 8))
        m = g.fold("max", xx).value
        s = g.fold("sum", g.apply("exp", xx - m), phase=2).value
        g.output("r", (m + g.apply("log", s)) * g.load("w", (0, 1)), (0, 1), full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        m = X.max(axis=0)
        r = (m + np.log(np.exp(X - m).sum(axis=0))) * v["w"]
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("log-sum-exp written out", (8, 6), (0,), row, {"x": F(x), "w": F(w)}, closed, 6)


def softmax_by_the_maximum_read():
    """m = maximum(x; dims = 1); e = exp.(x .- m); sum(e ./ sum(e; dims = 1) .* t) + sum(m):
    three phases by columns, the maximum also an output term."""
    x, t = data(8, 6), data(8, 6, scale=0.7)

    def row(g):
        xx, tt = g.load("x", (1, 8)), g.load("t", (1, 8))
        m = g.fold("max", xx).value
        s = g.fold("sum", g.apply("exp", xx - m), phase=2).value
        y = g.fold("sum", g.apply("exp", xx - m) / s * tt, phase=3).value
        g.output("r", y + m, (0, 1), full=False)

    def closed(v):
        X, T = v["x"].reshape(8, 6, order="F"), v["t"].reshape(8, 6, order="F")
        m = X.max(axis=0)
        e = np.exp(X - m)
        r = (e / e.sum(axis=0) * T).sum(axis=0) + m
        return {"r": r, "loss": [r.sum()]}
    return _column_then_sum("softmax by the maximum, the maximum read", (8, 6), (0,), row,
                            {"x": F(x), "t": F(t)}, closed, 6)


def scalar_input():
    """(x, s) -> sum(abs2, x .* s .+ s^2) with s = 0.7, a scalar argument."""
    x = data(8, 6)

    def build(g):
        sv = g.load("s", (0, 0))
        return g.fold("sum", g.apply("abs2", g.load("x", (1, 8)) * sv + sv * sv)).value
    return _whole("scalar input", (8, 6), build, {"x": F(x), "s": np.array([0.7])},
                  lambda v: {"loss": [np.sum((v["x"] * v["s"][0] + v["s"][0] ** 2) ** 2)]})


def _column_sums_squared(name):
    """sum(abs2, y) for y the column sums of x (8 x 6): a column group, then
    the fold of the six sums' squares."""
    x = data(8, 6)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0,), name="column sums")
    g1.value("x", "f32", 48)
    g1.value("r", "f32", 6)
    g1.output("r", g1.fold("sum", g1.load("x", (1, 8))).value, (0, 1), full=False)
    g2 = FloorGroup("reduction", (6,), reduced=(0,), name="sum(abs2, r)")
    g2.value("r", "f32", 6)
    g2.value("loss", "f32", 1)
    g2.output("loss", g2.fold("sum", g2.apply("abs2", g2.load("r", (1,)))).value, full=False)

    def closed(v):
        r = v["x"].reshape(8, 6, order="F").sum(axis=0)
        return {"r": r, "loss": [np.sum(r ** 2)]}
    return Case(name, [g1, g2], {"x": F(x)}, {"r": 6, "loss": 1}, ["r", "loss"], closed)


def vec_and_dropdims():
    """sum(abs2, vec(dropdims(sum(x; dims = 1); dims = 1)))."""
    return _column_sums_squared("vec and dropdims")


def scalar_writes_in_a_loop():
    """y = similar(x, 6); for i in 1:6; y[i] = sum(x[:, i]); end; sum(abs2, y)."""
    return _column_sums_squared("scalar writes in a loop")


def opaque_leaky_with_a_rule():
    """sum(abs2, leaky.(x)), leaky(x) = x > 0 ? x : 0.01 x."""
    x = data(8, 6)

    def build(g):
        t = g.load("x", (1, 8))
        return g.fold("sum", g.apply("abs2", g.apply("ifelse", g.apply(">", t, 0.0), t, t * 0.01))).value
    return _whole("opaque leaky with a rule", (8, 6), build, {"x": F(x)},
                  lambda v: {"loss": [np.sum(np.where(v["x"] > 0, v["x"], 0.01 * v["x"]) ** 2)]})


def norms_and_a_normalized_vector():
    """norm(x) + norm(x, 1) + norm(x, 3) + sum(normalize(u) .* data(8; scale = 0.3)):
    three folds over x, then u's dot and norm."""
    x, u, w = data(8, 6), data(8, scale=0.5), data(8, scale=0.3)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="norms of x")
    g1.value("x", "f32", 48)
    g1.value("nx", "f32", 1)
    t = g1.load("x", (1, 8))
    a = g1.apply("abs", t)
    n2 = g1.fold("sum", g1.apply("abs2", t)).value
    n1 = g1.fold("sum", a).value
    n3 = g1.fold("sum", a * a * a).value
    g1.output("nx", g1.apply("sqrt", n2) + n1 + n3 ** (1.0 / 3.0), full=False)
    g2 = FloorGroup("reduction", (8,), reduced=(0,), name="sum(normalize(u) .* w)")
    for k, n in (("u", 8), ("w", 8), ("nx", 1), ("loss", 1)):
        g2.value(k, "f32", n)
    uu = g2.load("u", (1,))
    dot = g2.fold("sum", uu * g2.load("w", (1,))).value
    nu = g2.fold("sum", g2.apply("abs2", uu)).value
    g2.output("loss", dot / g2.apply("sqrt", nu) + g2.load("nx", (0,)), full=False)

    def closed(v):
        X = v["x"]
        nx = np.sqrt(np.sum(X ** 2)) + np.sum(np.abs(X)) + np.sum(np.abs(X) ** 3) ** (1 / 3)
        return {"nx": [nx], "loss": [nx + np.sum(v["u"] / np.linalg.norm(v["u"]) * v["w"])]}
    return Case("norms and a normalized vector", [g1, g2], {"x": F(x), "u": F(u), "w": F(w)},
                {"nx": 1, "loss": 1}, ["nx", "loss"], closed)


def cartesian_diagonal_and_dot():
    """sum(abs2, diag(x)) + x[CartesianIndex(2, 3)] + dot(x, tanh.(x)), x 6 x 6:
    the diagonal as a load of stride 7, the element at its constant offset."""
    x = data(6, 6)
    g1 = FloorGroup("reduction", (6,), reduced=(0,), name="sum(abs2, diag(x)) + x[2, 3]")
    g1.value("x", "f32", 36)
    g1.value("d", "f32", 1)
    g1.output("d", g1.fold("sum", g1.apply("abs2", g1.load("x", (7,)))).value + g1.load("x", (0,), constant=13),
              full=False)
    g2 = FloorGroup("reduction", (6, 6), reduced=(0, 1), name="dot(x, tanh.(x))")
    for k, n in (("x", 36), ("d", 1), ("loss", 1)):
        g2.value(k, "f32", n)
    t = g2.load("x", (1, 6))
    g2.output("loss", g2.fold("sum", t * g2.apply("tanh", t)).value + g2.load("d", (0, 0)), full=False)

    def closed(v):
        X = v["x"].reshape(6, 6, order="F")
        d = np.sum(np.diag(X) ** 2) + X[1, 2]
        return {"d": [d], "loss": [d + np.sum(X * np.tanh(X))]}
    return Case("Cartesian indices, the diagonal and dot", [g1, g2], {"x": F(x)}, {"d": 1, "loss": 1},
                ["d", "loss"], closed)


def a_scalar_written_into_place():
    """y = copy(x); y[3, 2] = s * 2; sum(abs2, y), s = 0.7."""
    x = data(8, 6)
    w = FloorGroup("pointwise", (1,), name="y[3, 2] = s * 2")
    w.value("s", "f32", 1)
    w.value("y", "f32", 48)
    w.output("y", w.load("s", (0,)) * 2.0, (0,), constant=2 + 8 * 1)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        Y[2, 1] = val["s"][0] * 2
        return {"y": Y.ravel(order="F"), "loss": [np.sum(Y ** 2)]}
    return Case("a scalar written into place", [_copy("x", "y", (8, 6)), w,
                                                _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", y))],
                {"x": F(x), "s": np.array([0.7])}, {"y": 48, "loss": 1}, ["y", "loss"], closed)


def rotation_by_a_constant_permutation():
    """sum(abs2, x .* c .+ x[[3, 4, 1, 2], :] .* s), x 4 x 6, c and s 4 x 1: the
    permutation [3, 4, 1, 2] is i -> (i + 2) mod 4, a load at a rotated row."""
    x, c, sn = data(4, 6), data(4, 1), data(4, 1, scale=0.3)
    g = FloorGroup("reduction", (2, 2, 6), reduced=(0, 1, 2), name="x .* c .+ x[[3, 4, 1, 2], :] .* s")
    for k, n in (("x", 24), ("c", 4), ("s", 4), ("loss", 1)):
        g.value(k, "f32", n)
    # Row i = i0 + 2 i1 (i0, i1 in 0..1); its partner row (i + 2) mod 4 = i0 + 2 (1 - i1).
    xi = g.load("x", (1, 2, 4))
    xp = g.load("x", (1, -2, 4), constant=2)
    y = xi * g.load("c", (1, 2, 0)) + xp * g.load("s", (1, 2, 0))
    g.output("loss", g.fold("sum", g.apply("abs2", y)).value, full=False)

    def closed(v):
        X = v["x"].reshape(4, 6, order="F")
        Y = X * v["c"][:, None] + X[[2, 3, 0, 1], :] * v["s"][:, None]
        return {"loss": [np.sum(Y ** 2)]}
    return Case("rotation by a constant permutation", [g], {"x": F(x), "c": F(c), "s": F(sn)}, {"loss": 1},
                ["loss"], closed)


def concatenations():
    """sum(abs2, vcat(x, v) .* data(11, 6)) + sum(hcat(x, x) .* 2), x 8 x 6, v 3 x 6:
    vcat as two loads of the 11 x 6 domain split by rows, hcat's sum as twice x's."""
    x, v, d = data(8, 6), data(3, 6, scale=0.3), data(11, 6)
    gx = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="x rows of vcat, and hcat(x, x)")
    for k, n in (("x", 48), ("d", 66), ("a", 1)):
        gx.value(k, "f32", n)
    t = gx.load("x", (1, 8))
    gx.output("a", gx.fold("sum", gx.apply("abs2", t * gx.load("d", (1, 11)))).value
              + gx.fold("sum", t * 2.0 + t * 2.0).value, full=False)
    gv = FloorGroup("reduction", (3, 6), reduced=(0, 1), name="v rows of vcat")
    for k, n in (("v", 18), ("d", 66), ("a", 1), ("loss", 1)):
        gv.value(k, "f32", n)
    gv.output("loss", gv.fold("sum", gv.apply("abs2", gv.load("v", (1, 3)) * gv.load("d", (1, 11), constant=8))).value
              + gv.load("a", (0, 0)), full=False)

    def closed(val):
        X, V, D = (val["x"].reshape(8, 6, order="F"), val["v"].reshape(3, 6, order="F"),
                   val["d"].reshape(11, 6, order="F"))
        a = np.sum((X * D[:8]) ** 2) + np.sum(np.hstack([X, X]) * 2)
        return {"a": [a], "loss": [a + np.sum((V * D[8:]) ** 2)]}
    return Case("concatenations", [gx, gv], {"x": F(x), "v": F(v), "d": F(d)}, {"a": 1, "loss": 1},
                ["a", "loss"], closed)


def a_write_at_index_arrays():
    """y = copy(x); y[:, [5, 2, 6]] = v; sum(abs2, tanh.(y)): the index list a
    gather on the written position."""
    x, v, cols = data(8, 6), data(8, 3, scale=0.3), _idx([5, 2, 6])
    w = FloorGroup("pointwise", (8, 3), name="y[:, [5, 2, 6]] = v")
    w.value("v", "f32", 24)
    w.value("cols", "i32", 3)
    w.value("y", "f32", 48)
    w.output("y", w.load("v", (1, 8)), (1, 0), constant=-8, gather=w.load("cols", (0, 1)), gather_coeff=8)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        Y[:, [4, 1, 5]] = val["v"].reshape(8, 3, order="F")
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.tanh(Y) ** 2)]}
    return Case("a write at index arrays", [_copy("x", "y", (8, 6)), w,
                                            _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("tanh", y)))],
                {"x": F(x), "v": F(v), "cols": cols}, {"y": 48, "loss": 1}, ["y", "loss"], closed,
                dtypes={"cols": "i32"})


def gather_by_a_traced_vector():
    """(x, i) -> sum(abs2, x[:, i] .* 2), i = [3, 1, 3, 6] an argument."""
    x, i = data(8, 6), _idx([3, 1, 3, 6])
    g = FloorGroup("reduction", (8, 4), reduced=(0, 1), name="x[:, i] .* 2")
    g.value("x", "f32", 48)
    g.value("i", "i64", 4)
    g.value("loss", "f32", 1)
    col = g.load("i", (0, 1))
    g.output("loss", g.fold("sum", g.apply("abs2", g.load("x", (1, 0), constant=-8, gather=col, gather_coeff=8) * 2.0)).value,
             full=False)
    return Case("gather by a traced vector", [g], {"x": F(x), "i": i}, {"loss": 1}, ["loss"],
                lambda v: {"loss": [np.sum((2 * v["x"].reshape(8, 6, order="F")[:, [2, 0, 2, 5]]) ** 2)]},
                dtypes={"i": "i64"})


def _renamed(make, name):
    case = make()
    case.name = name
    return case


def linear_recurrence_named_with_generic_fold():
    """accumulate(RECURRENCE, tuple.(a, b)): the same combine named with
    GenericFold, which claims it associates; planned as the same scan."""
    return _renamed(linear_recurrence, "a linear recurrence named with GenericFold")


def welford_variance_as_base_spells_it():
    """mapreduce(welford_lift, welford, x; dims = 1) observed s[3] / s[1]:
    Welford's fold as Base spells it, planned as the square fold."""
    return _renamed(welford_variance, "Welford's variance as Base spells it")


def welford_variance_named_with_generic_fold():
    """reduce(VARIANCE, x; dims = 1): the same fold named with GenericFold."""
    return _renamed(welford_variance, "Welford's variance named with GenericFold")


def circular_shifts_rotations_and_repeats():
    """sum(abs2, circshift(x, (1, -2)) .* data(8, 6)) + sum(rotr90(x) .* data(6, 8)) +
    sum(abs2, repeat(x; inner = (1, 2), outer = (2, 1)) .* data(16, 12)), x 8 x 6:
    the shift as two Mod atoms, the rotation as a reversed affine load, the
    repeat as a Mod and a Div atom."""
    x, d1, d2, d3 = data(8, 6), data(8, 6), data(6, 8), data(16, 12)
    g1 = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="circshift(x, (1, -2)) .* d1")
    for k, n in (("x", 48), ("d1", 48), ("a", 1)):
        g1.value(k, "f32", n)
    shifted = g1.load("x", (0, 0), parts=[("mod", (1, 0), 8, 1, -1), ("mod", (0, 1), 6, 8, 2)])
    g1.output("a", g1.fold("sum", g1.apply("abs2", shifted * g1.load("d1", (1, 8)))).value, full=False)
    g2 = FloorGroup("reduction", (6, 8), reduced=(0, 1), name="rotr90(x) .* d2")
    for k, n in (("x", 48), ("d2", 48), ("a", 1), ("b", 1)):
        g2.value(k, "f32", n)
    g2.output("b", g2.fold("sum", g2.load("x", (8, -1), constant=7) * g2.load("d2", (1, 6))).value
              + g2.load("a", (0, 0)), full=False)
    g3 = FloorGroup("reduction", (16, 12), reduced=(0, 1), name="repeat(x; inner = (1, 2), outer = (2, 1)) .* d3")
    for k, n in (("x", 48), ("d3", 192), ("b", 1), ("loss", 1)):
        g3.value(k, "f32", n)
    rep = g3.load("x", (0, 0), parts=[("mod", (1, 0), 8, 1), ("div", (0, 1), 2, 8)])
    g3.output("loss", g3.fold("sum", g3.apply("abs2", rep * g3.load("d3", (1, 16)))).value
              + g3.load("b", (0, 0)), full=False)

    def closed(v):
        X = v["x"].reshape(8, 6, order="F")
        D1, D2, D3 = (v["d1"].reshape(8, 6, order="F"), v["d2"].reshape(6, 8, order="F"),
                      v["d3"].reshape(16, 12, order="F"))
        a = np.sum((np.roll(X, (1, -2), axis=(0, 1)) * D1) ** 2)
        b = a + np.sum(np.rot90(X, -1) * D2)
        return {"a": [a], "b": [b], "loss": [b + np.sum((np.tile(np.repeat(X, 2, axis=1), (2, 1)) * D3) ** 2)]}
    return Case("circular shifts, rotations and repeats", [g1, g2, g3],
                {"x": F(x), "d1": F(d1), "d2": F(d2), "d3": F(d3)}, {"a": 1, "b": 1, "loss": 1},
                ["a", "b", "loss"], closed)


def dropout():
    """(x, s) -> sum(abs2, Ops.dropout(x, s; rate = 0.25) .* 2), s = Int32[7]: the
    keep scale of position i (1-based, column-major) a hash of the seed's
    first element and i (test/fixtures/operations.jl:88-119)."""
    x, s = data(8, 6), _idx([7])

    def build(g):
        pos = g.index((1, 8)) + 1.0
        keep = g.apply("dropout", g.load("s", (0, 0)), pos, 0.25)
        return g.fold("sum", g.apply("abs2", g.load("x", (1, 8)) * keep * 2.0)).value

    def closed(v):
        # The hash restated with numpy's wrapping uint32 arithmetic (the oracle
        # uses Python integers masked to 32 bits).
        i = np.arange(1, 49, dtype=np.uint32)
        with np.errstate(over="ignore"):
            h = (np.uint32(int(v["s"][0])) * np.uint32(0x9E3779B1)) ^ (i * np.uint32(0xC2B2AE35))
            h ^= h >> np.uint32(16)
            h *= np.uint32(0x7FEB352D)
            h ^= h >> np.uint32(15)
            h *= np.uint32(0x846CA68B)
            h ^= h >> np.uint32(16)
        u = (h >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)
        keep = np.where(u >= np.float32(0.25), np.float32(1) / np.float32(0.75), np.float32(0))
        return {"loss": [np.sum((v["x"] * keep * 2) ** 2)]}
    g = FloorGroup("reduction", (8, 6), reduced=(0, 1), name="dropout")
    g.value("x", "f32", 48)
    g.value("s", "i32", 1)
    g.value("loss", "f32", 1)
    g.output("loss", build(g), full=False)
    return Case("dropout", [g], {"x": F(x), "s": s}, {"loss": 1}, ["loss"], closed, dtypes={"s": "i32"})


CASES = [dot_product, sum_abs2_tanh, full_logsumexp, maximum_and_shifted_sum, minus_mean, swish, powers,
         clamp_and_max, strided_view_and_index, rounded_counted_tested, column_maxima, row_minima, products,
         softmax_columns, softmax_rows, rank3_softmax, rmsnorm, layer_norm, layer_norm_welford, welford_variance,
         map_over_two_arrays, permutation, permutation_and_reshape, permute_reshape_and_roll,
         bias_tanh_bf16, index_scaled, kat_sum_abs2,
         cumulative_sums, cumulative_products_through_a_zero, running_maxima_and_minima, linear_recurrence,
         running_average, reverse_exclusive_sums, running_logsumexp_and_mean,
         gather_by_a_list, gather_by_an_int32_matrix, gather_rows_by_an_int64_matrix,
         gather_by_linear_and_scalar_indices, embedding_and_layer_norm, scatter_add_gradient,
         extremes_and_where_they_are, extremes_of_a_vector, mean_recomputed, recurrence_with_recomputed_sums,
         reverse_recurrence, write_of_a_slice, padding_by_a_write, writes_through_views, strided_and_reversed_writes,
         write_at_traced_positions, mean_divided_in_place, permutedims_and_copyto,
         log_sum_exp_written_out, softmax_by_the_maximum_read, scalar_input, vec_and_dropdims,
         scalar_writes_in_a_loop, opaque_leaky_with_a_rule, norms_and_a_normalized_vector,
         cartesian_diagonal_and_dot, a_scalar_written_into_place, rotation_by_a_constant_permutation,
         concatenations, a_write_at_index_arrays, gather_by_a_traced_vector,
         linear_recurrence_named_with_generic_fold, welford_variance_as_base_spells_it,
         welford_variance_named_with_generic_fold, circular_shifts_rotations_and_repeats, dropout]


# ---- writes where several elements land at one position ---------------------------
# REPEATED_WRITES (test/fixtures/programs.jl:148-155): the interpreters and
# the CPU's floor take the colliding writes in order, the last landing; a
# device lands any one of them, so, as in the reference, these are checked on
# the CPU only (the oracle's groups against the closed form).

def a_write_at_repeated_positions():
    """y = copy(x); y[[2, 7, 2], :] .= v; sum(abs2, sin.(y)): rows 2 and 7 of y
    get rows 3 and 2 of v (the later write to row 2 lands)."""
    x, v, rows = data(8, 6), data(3, 6, scale=0.3), _idx([2, 7, 2])
    w = FloorGroup("pointwise", (3, 6), name="y[[2, 7, 2], :] .= v")
    w.value("v", "f32", 18)
    w.value("rows", "i64", 3)
    w.value("y", "f32", 48)
    w.output("y", w.load("v", (1, 3)), (0, 8), constant=-1, gather=w.load("rows", (1, 0)), gather_coeff=1)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        V = val["v"].reshape(3, 6, order="F")
        for k, r in enumerate([1, 6, 1]):
            Y[r, :] = V[k, :]
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.sin(Y) ** 2)]}
    return Case("a write at repeated positions", [_copy("x", "y", (8, 6)), w,
                                                  _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("sin", y)))],
                {"x": F(x), "v": F(v), "rows": rows}, {"y": 48, "loss": 1}, ["y", "loss"], closed,
                dtypes={"rows": "i64"})


def a_write_at_repeated_traced_positions():
    """y = copy(x); y[:, i] .= v; sum(abs2, tanh.(y)), i = Int32[4, 1, 4]:
    column 4 takes v's third column."""
    x, v, i = data(8, 6), data(8, 3, scale=0.3), _idx([4, 1, 4])
    w = FloorGroup("pointwise", (8, 3), name="y[:, i] .= v")
    w.value("v", "f32", 24)
    w.value("i", "i32", 3)
    w.value("y", "f32", 48)
    w.output("y", w.load("v", (1, 8)), (1, 0), constant=-8, gather=w.load("i", (0, 1)), gather_coeff=8)

    def closed(val):
        Y = val["x"].reshape(8, 6, order="F").copy()
        V = val["v"].reshape(8, 3, order="F")
        for k, c in enumerate([3, 0, 3]):
            Y[:, c] = V[:, k]
        return {"y": Y.ravel(order="F"), "loss": [np.sum(np.tanh(Y) ** 2)]}
    return Case("a write at repeated traced positions", [_copy("x", "y", (8, 6)), w,
                                                         _loss((8, 6), ["y"], lambda g, y: g.apply("abs2", g.apply("tanh", y)))],
                {"x": F(x), "v": F(v), "i": i}, {"y": 48, "loss": 1}, ["y", "loss"], closed, dtypes={"i": "i32"})


CPU_ONLY = [a_write_at_repeated_positions, a_write_at_repeated_traced_positions]


def run_oracle(case: Case) -> dict:
    """Every value after the case's groups, by the oracle, in order."""
    from oracle.floor_groups import evaluate
    from oracle.data import bf16_round
    vals = {k: np.array(v, dtype=np.float64) for k, v in case.inputs.items()}
    for k, n in case.stored.items():
        vals[k] = np.zeros(n)
    for k in vals:
        # What the device holds: Float32 inputs, bfloat16 or integers where the case says so.
        dt = case.dtypes.get(k)
        if dt in ("i32", "i64"):
            vals[k] = np.asarray(case.inputs[k], dtype=np.int64)
            continue
        vals[k] = (bf16_round(vals[k].astype(np.float32)) if dt == "bf16"
                   else vals[k].astype(np.float32)).astype(np.float64)
    for g in case.groups:
        out = evaluate(g.spec(), vals)
        vals.update({k: v.astype(np.float64) for k, v in out.items()})
    return vals
