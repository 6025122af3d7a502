"""The oracle's fold algebra against what fixes it: the reference's doctest,
two-pass formulas in float64, and partition invariance."""
import math
import random

import numpy as np
import pytest

from oracle import folds as F


def test_generic_fold_recurrence_doctest():
    # src/Compiler/IR/folds.jl:279-288: accumulate of the linear recurrence.
    rec = F.GenericFold(init_fn=lambda: (1.0, 0.0), lift_fn=lambda e: e,
                        combine_fn=lambda a, b: (b[0] * a[0], b[0] * a[1] + b[1]), observe_fn=lambda s: s[-1])
    assert F.accumulate(rec, [(0.5, 1.0)] * 3) == [1.0, 1.5, 1.75]


def test_sum_of_squares_doctest():
    # src/Compiler/runtime/compile.jl:35-40: sum(abs2, [1,2,3,4]) == 30.
    assert F.fold(F.SumFold(), [x * x for x in [1.0, 2.0, 3.0, 4.0]]) == 30.0


def test_lse_shift_special_values():
    assert F.lse_shift(-math.inf) == 0.0 and F.lse_shift(math.inf) == 0.0 and F.lse_shift(2.5) == 2.5
    # An all -Inf column's exponential sum is zero, its logsumexp -Inf.
    assert F.fold(F.LOGSUMEXP, [-math.inf, -math.inf]) == -math.inf


@pytest.mark.parametrize("seed", range(5))
def test_online_exponential_fold_matches_two_pass(seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=37) * 4
    g = rng.normal(size=37)
    two_pass = float(np.log(np.exp(x - x.max()).sum()) + x.max())
    assert math.isclose(F.fold(F.LOGSUMEXP, list(x)), two_pass, rel_tol=1e-13)
    # Sum of g weighted by exp(x - max), observed against the max.
    weighted = F.Relative(F.Exponential(), F.nth_sum(0))
    w = np.exp(x - x.max())
    assert math.isclose(F.fold(weighted, list(zip(x, g))), float((g * w).sum()), rel_tol=1e-12)


@pytest.mark.parametrize("seed", range(5))
def test_square_law_matches_two_pass_variance(seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=53) * 3 + 7
    m2 = F.Relative(F.Square(), F.nth_sum(0))
    assert math.isclose(F.fold(m2, list(x)), float(((x - x.mean()) ** 2).sum()), rel_tol=1e-12)
    assert math.isclose(F.fold(F.Relative(F.Square(), F.statistic), list(x)), float(x.mean()), rel_tol=1e-13)


@pytest.mark.parametrize("law", ["exp", "square"])
def test_relative_folds_are_partition_invariant(law):
    # Any grouping of the elements, combined, equals the sequential fold:
    # what a device's tree of lanes relies on (folds.jl:1-9).
    rng = random.Random(7)
    f = F.Relative(F.Exponential(), F.nth_sum(0)) if law == "exp" else F.Relative(F.Square(), F.nth_sum(0))
    xs = [rng.gauss(0, 3) for _ in range(100)]
    seq = F.fold(f, xs)
    tree = F.fold_tree(f, xs)
    assert math.isclose(seq, tree, rel_tol=1e-12)
    # A random split into two parts, combined.
    k = 41
    a, b = F.init_state = None, None
    sa = f.init()
    for x in xs[:k]:
        sa = f.combine(sa, f.lift(x))
    sb = f.init()
    for x in xs[k:]:
        sb = f.combine(sb, f.lift(x))
    assert math.isclose(f.observe(f.combine(sa, sb)), seq, rel_tol=1e-12)


def test_a_dropped_rebase_term_is_caught():
    # A plausible slip -- combining exponential sums without moving them to
    # the common maximum -- must change the result the tests compare.
    class Broken(F.Exponential):
        def rebase(self, a, s, m):
            return a
    xs = [0.0, 5.0, -2.0]
    good = F.fold(F.Relative(F.Exponential(), F.nth_sum(0)), xs)
    bad = F.fold(F.Relative(Broken(), F.nth_sum(0)), xs)
    assert not math.isclose(good, bad, rel_tol=1e-3)
