"""The generated floor on the CPU: the oracle's group evaluation pinned by
closed forms and the sequential fold algebra; every fixture group's kernel
written and compiled for gfx950 without a device; the ABI's rejections."""
import numpy as np
import pytest

import floor_cases as FC
from oracle import floor_groups as FG
from oracle import folds as F
from oracle.data import relative

CASES = {c.__name__: c for c in FC.CASES}


def _cast_inputs(case):
    return {k: (np.asarray(v) if case.dtypes.get(k) in ("i32", "i64") else
                np.asarray(v, dtype=np.float32).astype(np.float64)) for k, v in case.inputs.items()}


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_matches_closed_form(name):
    case = CASES[name]()
    vals = FC.run_oracle(case)
    want = case.closed(_cast_inputs(case))
    for k in case.results:
        tol = 1e-2 if case.dtypes.get(k) == "bf16" else 1e-6
        assert relative(vals[k], np.asarray(want[k], dtype=np.float64)) < tol, (name, k)


@pytest.mark.parametrize("make", FC.CPU_ONLY, ids=[c.__name__ for c in FC.CPU_ONLY])
def test_repeated_writes_land_in_order(make):
    """The reference's REPEATED_WRITES, checked on the CPU as it checks them:
    the oracle takes colliding writes in order, the last landing."""
    case = make()
    vals = FC.run_oracle(case)
    want = case.closed(_cast_inputs(case))
    for k in case.results:
        assert relative(vals[k], np.asarray(want[k], dtype=np.float64)) < 1e-6, (case.name, k)


def test_dropout_scale_keeps_its_rate():
    """The dropout hash's keep scale over 20000 positions: 1 / (1 - rate) or 0,
    kept with frequency 1 - rate (a flipped comparison keeps `rate`), the
    same positions for the same seed and different ones for another."""
    pos = np.arange(1, 20001)
    for rate in (0.25, 0.5, 0.9):
        k = FG.dropout_scale(np.full(pos.shape, 7), pos, np.full(pos.shape, rate))
        assert set(np.unique(k)) <= {0.0, float(np.float32(1) / (np.float32(1) - np.float32(rate)))}
        assert abs((k > 0).mean() - (1 - rate)) < 0.015, rate
    a = FG.dropout_scale(np.full(pos.shape, 7), pos, np.full(pos.shape, 0.5))
    b = FG.dropout_scale(np.full(pos.shape, 8), pos, np.full(pos.shape, 0.5))
    assert np.array_equal(a, FG.dropout_scale(np.full(pos.shape, 7), pos, np.full(pos.shape, 0.5)))
    assert 0.4 < ((a > 0) != (b > 0)).mean() < 0.6


def test_kat_sum_of_squares_exact():
    # src/Compiler/runtime/compile.jl:35-40: exactly 30.
    assert FC.run_oracle(FC.kat_sum_abs2())["loss"][0] == 30.0


@pytest.mark.parametrize("seed", range(4))
def test_vectorized_folds_match_sequential_algebra(seed):
    rng = np.random.default_rng(seed)
    y = rng.normal(size=(23, 5)) * 3
    g = rng.normal(size=(23, 5))
    for j in range(5):
        col, w = list(y[:, j]), list(zip(y[:, j], g[:, j]))
        got = {k: FG.fold_reduce(k, y[:, j:j + 1], g[:, j:j + 1] if k == "exp" else None, (0,))
               for k in ("sum", "prod", "max", "min", "exp", "square")}
        assert np.isclose(got["sum"]["value"][0, 0], F.fold(F.SumFold(), col), rtol=1e-13)
        assert np.isclose(got["max"]["value"][0, 0], F.fold(F.MaxFold(), col), rtol=0)
        assert np.isclose(got["min"]["value"][0, 0], -F.fold(F.MaxFold(), [-v for v in col]), rtol=0)
        prod = F.fold(F.GenericFold(init_fn=lambda: (1.0,), combine_fn=lambda a, b: (a[0] * b[0],)), col)
        assert np.isclose(got["prod"]["value"][0, 0], prod, rtol=1e-12)
        weighted = F.Relative(F.Exponential(), F.nth_sum(0))
        assert np.isclose(got["exp"]["sum"][0, 0], F.fold(weighted, w), rtol=1e-12)
        assert np.isclose(got["exp"]["statistic"][0, 0], F.fold(F.Relative(F.Exponential(), F.statistic), w))
        plain = FG.fold_reduce("exp", y[:, j:j + 1], None, (0,))
        assert np.isclose(plain["logsumexp"][0, 0], F.fold(F.LOGSUMEXP, col), rtol=1e-13)
        sq_mean = F.fold(F.Relative(F.Square(), F.statistic), col)
        sq_m2 = F.fold(F.Relative(F.Square(), F.nth_sum(0)), col)
        assert np.isclose(got["square"]["statistic"][0, 0], sq_mean, rtol=1e-12)
        assert np.isclose(got["square"]["sum"][0, 0], sq_m2, rtol=1e-12)


def test_planted_missing_rebase_is_caught(monkeypatch):
    """An exponential fold that forgets to shift by its maximum must fail the
    closed form of a softmax with large entries."""
    real = FG.fold_reduce

    def planted(kind, y, g, axes):
        if kind != "exp":
            return real(kind, y, g, axes)
        w = 1.0 if g is None else g
        s = (w * np.exp(y)).sum(axis=axes, keepdims=True)      # no rebase
        m = y.max(axis=axes, keepdims=True)
        return {"statistic": m, "sum": s, "logsumexp": m + np.log(s)}
    monkeypatch.setattr(FG, "fold_reduce", planted)
    case = FC.softmax_columns()
    case.inputs["x"] = case.inputs["x"] * 30.0
    vals = FC.run_oracle(case)
    want = case.closed(_cast_inputs(case))
    assert relative(vals["loss"], np.asarray(want["loss"])) > 1e-3


@pytest.mark.parametrize("name", list(CASES))
def test_kernels_compile_without_a_device(name):
    case = CASES[name]()
    for g in case.groups:
        src = g.source()
        assert src.startswith("// tempest-hip floor:") and "extern \"C\" __global__" in src
        g.compile()  # hiprtc for gfx950, into the code-object cache


@pytest.mark.parametrize("rows,n", [(32768, 8192), (700, 256), (2, 40000), (9, 1027)])
def test_config2_floor_programs_compile(rows, n):
    import tempest_hip as th
    for prog in (th.programs.floor_softmax_columns(rows, n), th.programs.floor_layernorm(rows, n)):
        for grp in prog.groups:
            grp.build.__self__.compile()


def test_plans_take_each_mapping():
    """Rows (resident, streamed, split), columns (lanes and parts), pointwise."""
    from tempest_hip.floor import FloorGroup

    def head(extents, reduced, unit_axis):
        g = FloorGroup("reduction", extents, reduced=reduced)
        n = int(np.prod(extents))
        g.value("x", "f32", n)
        g.value("r", "f32", n)
        coeffs = [1, extents[0]] if unit_axis == 0 else [1, extents[0]]
        x = g.load("x", coeffs)
        g.output("r", g.fold("sum", x).value, [0 if k in reduced else c for k, c in enumerate(coeffs)], full=False)
        return g.source().splitlines()[0]
    assert "rows" in head((8192, 64), (0,), 0) and "resident" in head((8192, 64), (0,), 0)
    assert "streamed" in head((100000, 64), (0,), 0)
    assert "parts" in head((1 << 22, 1), (0,), 0) and ", parts 1," not in head((1 << 22, 1), (0,), 0)
    col = head((300, 5000), (1,), 0)
    assert col.startswith("// tempest-hip floor: columns") and ", lanes 4," in col and ", parts 1," not in col
    assert ", lanes 1, parts 1," in head((300000, 8), (1,), 0)


@pytest.mark.parametrize("break_it,message", [
    ("load_outside", "outside its value"),
    ("later_stat", "own or a later phase"),
    ("pointwise_fold", "only a reduction group folds"),
    ("write_outside", "writes outside"),
    ("zero_divisor", "positive divisor"),
    ("part_outside", "outside its value"),
    ("part_store_outside", "writes outside"),
])
def test_abi_rejects(break_it, message):
    from tempest_hip import HIPError
    from tempest_hip.floor import FloorGroup
    g = FloorGroup("reduction", (8, 6), reduced=(0,))
    g.value("x", "f32", 48)
    g.value("r", "f32", 6)
    x = g.load("x", (1, 8))
    try:
        if break_it == "load_outside":
            bad = g.load("x", (1, 9))
            g.output("r", g.fold("sum", bad).value, (0, 1), full=False)
        elif break_it == "later_stat":
            f2 = g.fold("sum", x, phase=2)
            g.output("r", g.fold("sum", x * f2.value, phase=2).value, (0, 1), full=False)
        elif break_it == "pointwise_fold":
            FloorGroup("pointwise", (8,)).fold("sum", 1.0)
        elif break_it == "zero_divisor":
            g.output("r", g.fold("sum", g.load("x", (1, 0), parts=[("div", (0, 1), 0, 8)])).value, (0, 1), full=False)
        elif break_it == "part_outside":  # i1 div 2 reaches 2: 7 + 9 * 2 + 24 = 49 > 47
            g.output("r", g.fold("sum", g.load("x", (1, 0), 24, parts=[("div", (0, 1), 2, 9)])).value, (0, 1),
                     full=False)
        elif break_it == "part_store_outside":  # i1 mod 4 reaches 3: 3 * 2 = 6 > 5
            g.output("r", g.fold("sum", x).value, (0, 0), full=False, parts=[("mod", (0, 1), 4, 2)])
        else:
            g.output("r", g.fold("sum", x).value, (0, 2), full=False)
        g.source()
    except (HIPError, ValueError) as e:
        assert message in str(e)
    else:
        raise AssertionError("accepted")


def test_scans_along_the_contiguous_axis_take_a_workgroup_per_item():
    """A scan whose loads run along its positions plans a parallel scan (four
    positions a lane going forward, one in reverse); a strided one, a thread
    per item.  Each plan's kernel compiles."""
    from tempest_hip.floor import FloorGroup

    def group(n, m, axis, reverse=False):
        g = FloorGroup("scan", (n, m), reduced=(axis,), reverse=reverse)
        for k in ("x", "a", "c", "h"):
            g.value(k, "f32", n * m)
        x, a = g.load("x", (1, n)), g.load("a", (1, n))
        c = g.fold("sum", x, scan="inclusive")
        h = g.fold("linear", a, weight=x * c.value, scan="exclusive", phase=2)
        g.output("c", c.value, (1, n))
        g.output("h", h.value, (1, n))
        return g
    fwd, rev, col = group(4096, 3, 0), group(1000, 5, 0, reverse=True), group(300, 2000, 1)
    assert "a workgroup per item, width 4" in fwd.source().splitlines()[0]
    assert "a workgroup per item, width 1, reversed" in rev.source().splitlines()[0]
    assert "a thread per item" in col.source().splitlines()[0]
    for g in (fwd, rev, col):
        g.compile()


def _part_address_range(extents, coeffs, constant, parts):
    """The least and greatest address over the domain, by enumeration."""
    at = np.meshgrid(*[np.arange(e) for e in extents], indexing="ij")
    a = constant + sum(c * at[k] for k, c in enumerate(coeffs))
    for kind, inner, dv, cf, *c0 in parts:
        e = (c0[0] if c0 else 0) + sum(c * at[k] for k, c in enumerate(inner))
        a = a + cf * (np.floor_divide(e, dv) if kind == "div" else np.mod(e, dv))
    return int(np.min(a)), int(np.max(a))


def _accepts(extents, coeffs, constant, parts, length):
    from tempest_hip import HIPError
    from tempest_hip.floor import FloorGroup
    g = FloorGroup("pointwise", extents)
    g.value("x", "f32", length)
    g.value("y", "f32", int(np.prod(extents)))
    g.output("y", g.load("x", coeffs, constant, parts=parts), [1, extents[0]][:len(extents)])
    try:
        g.source()
    except HIPError as e:
        assert "outside its value" in str(e)
        return False
    return True


@pytest.mark.parametrize("parts,constant", [
    ([("mod", (1,), 20, 1, 10)], 0),        # 10..13, no wrap
    ([("mod", (1,), 20, 1, -8)], 0),        # -8..-5 mod 20 = 12..15
    ([("div", (1,), 4, -3, -5)], 0),        # fld(-5..-2, 4) = -2..-1, times -3: 3..6
    ([("div", (1, 4), 3, 2), ("mod", (1, 4), 3, 1)], 1),
])
def test_div_mod_bounds_are_exact_where_the_steps_are_unit(parts, constant):
    """An address of div/mod atoms is accepted exactly when its enumerated
    range lies in the value: at the smallest length that holds it, and not one
    element shorter."""
    extents = (4, 3)
    lo, hi = _part_address_range(extents, (0, 0), constant, parts)
    assert lo >= 0
    assert _accepts(extents, (0, 0), constant, parts, hi + 1)
    assert not _accepts(extents, (0, 0), constant, parts, hi)


def test_div_mod_bounds_are_sound_on_random_atoms():
    """Whatever the atoms, an accepted address never leaves its value."""
    rng = np.random.default_rng(11)
    for _ in range(300):
        extents = (int(rng.integers(1, 6)), int(rng.integers(1, 6)))
        parts = []
        for _ in range(int(rng.integers(1, 3))):
            parts.append((["div", "mod"][rng.integers(2)], tuple(int(v) for v in rng.integers(-4, 5, 2)),
                          int(rng.integers(1, 9)), int(rng.integers(-3, 4)), int(rng.integers(-10, 10))))
        coeffs = tuple(int(v) for v in rng.integers(0, 3, 2))
        lo, hi = _part_address_range(extents, coeffs, 0, parts)
        constant = max(0, -lo)
        length = int(rng.integers(max(1, hi + constant - 2), hi + constant + 3))
        if _accepts(extents, coeffs, constant, parts, length):
            assert lo + constant >= 0 and hi + constant < length, (extents, coeffs, constant, parts, length)


def test_column_reduction_hoists_loads_of_live_items_only():
    """A reduction over axis 1 of a (2, 100000, 3) array, plus a load of x at
    (i0, 0, i2) hoisted out of the sweep: 6 items in workgroups of 64, so 58
    threads have no item.  They must take item 0's positions, or the hoisted
    load reads up to 24 MB past the value."""
    from tempest_hip.floor import FloorGroup
    n0, n1, n2 = 2, 100000, 3
    g = FloorGroup("reduction", (n0, n1, n2), reduced=(1,))
    g.value("x", "f32", n0 * n1 * n2)
    g.value("r", "f32", n0 * n2)
    x = g.load("x", (1, n0, n0 * n1))
    x0 = g.load("x", (1, 0, n0 * n1))
    g.output("r", g.fold("sum", x * x0).value, (1, 0, n0), full=False)
    src = g.source()
    head = src.splitlines()[0]
    assert head.startswith("// tempest-hip floor: columns"), head
    assert "(live ? item : 0L)" in src
    g.compile()


@pytest.mark.parametrize("extents,length", [((1000, 0), 1), ((0, 7), 7)])
def test_once_outputs_of_an_empty_fold_are_checked(extents, length):
    """sum over an empty axis still writes every item's result, at the folded
    position zero: a (1000, 0) reduction over axis 1 writing r[i0] into a
    one-element value is refused (the kernel would write 1000 elements).  An
    empty kept axis writes nothing and is accepted."""
    from tempest_hip import HIPError
    from tempest_hip.floor import FloorGroup
    g = FloorGroup("reduction", extents, reduced=(1,))
    g.value("x", "f32", 0)
    g.value("r", "f32", length)
    g.output("r", g.fold("sum", g.load("x", (1, extents[0]))).value, (1, 0), full=False)
    if extents[0] == 0:
        g.source()
        return
    with pytest.raises(HIPError, match="writes outside"):
        g.source()


def test_once_output_loads_are_checked_at_folded_zero():
    """A once output that reads x at the folded position zero, over an empty
    folded axis: the load runs once per item, so x must hold it."""
    from tempest_hip import HIPError
    from tempest_hip.floor import FloorGroup
    g = FloorGroup("reduction", (16, 0), reduced=(1,))
    g.value("x", "f32", 8)
    g.value("r", "f32", 16)
    s = g.fold("sum", g.load("x", (1, 16)))
    g.output("r", s.value + g.load("x", (1, 16)), (1, 0), full=False)
    with pytest.raises(HIPError, match="folded positions at zero"):
        g.source()


def _base_extreme(y, idx, largest):
    """findmax / findmin by brute force over Base's orders: isless (NaN the
    largest, -0.0 before 0.0) for findmax, isgreater (NaN the smallest) for
    findmin, the first index among equals."""
    import math

    def key(j):
        x = float(y[j])
        nan = x != x
        pos = (not nan) and math.copysign(1.0, x) > 0
        return (nan, 0.0 if nan else x, pos, -idx[j]) if largest else (not nan, 0.0 if nan else x, pos, idx[j])
    j = (max if largest else min)(range(len(y)), key=key)
    return y[j], idx[j]


@pytest.mark.parametrize("largest", [True, False])
def test_extreme_folds_follow_base_order(largest):
    """The oracle's extreme folds (sequential, and combined in any grouping)
    against brute force over Base's orders, on elements full of ties, signed
    zeros, infinities and NaNs."""
    from oracle import floor_groups as FG
    rng = np.random.default_rng(7 + largest)
    pool = np.array([0.0, -0.0, 1.0, -1.0, 2.5, np.inf, -np.inf, np.nan])
    kind = "argmax" if largest else "argmin"
    for trial in range(200):
        n = int(rng.integers(1, 12))
        y = pool[rng.integers(0, len(pool) - (0 if trial % 3 == 0 else 1), n)]
        idx = rng.permutation(n).astype(np.float64) + 1
        st = FG.fold_reduce(kind, y[:, None], idx[:, None], (0,))
        want_y, want_i = _base_extreme(y, idx, largest)
        assert st["statistic"][0, 0] == want_i, (y, idx)
        assert (np.isnan(want_y) and np.isnan(st["value"][0, 0])) or (
            st["value"][0, 0] == want_y and np.signbit(st["value"][0, 0]) == np.signbit(want_y))
        # Any grouping: a random split into two halves, combined.
        cut = int(rng.integers(0, n + 1))
        a = FG.fold_reduce(kind, y[:cut, None], idx[:cut, None], (0,)) if cut else None
        b = FG.fold_reduce(kind, y[cut:, None], idx[cut:, None], (0,)) if cut < n else None
        parts = [p for p in (a, b) if p is not None]
        st2 = (parts[0]["value"], parts[0]["statistic"])
        for p in parts[1:]:
            st2 = FG.better(largest, st2, (p["value"], p["statistic"]))
        assert st2[1][0, 0] == want_i


def test_a_planted_tie_break_mistake_is_caught(monkeypatch):
    """The extreme fold without its index tie-break keeps the later of equal
    elements: the brute-force order catches it."""
    from oracle import floor_groups as FG
    def no_tie_break(largest, a, b):
        t = FG.lesser(a[0], b[0]) if largest else FG.greater(a[0], b[0])
        t = t | (a[0] == b[0])
        return np.where(t, b[0], a[0]), np.where(t, b[1], a[1])
    monkeypatch.setattr(FG, "better", no_tie_break)
    y, idx = np.array([1.0, 3.0, 3.0]), np.array([1.0, 2.0, 3.0])
    st = FG.fold_reduce("argmax", y[:, None], idx[:, None], (0,))
    assert st["statistic"][0, 0] != _base_extreme(y, idx, True)[1]
