"""TEST INFRASTRUCTURE ONLY: the reference's fold algebra, restated.

Follows src/Compiler/IR/folds.jl: a fold lifts each element to a state
(``lift``), merges states earlier-first (``combine``) and maps the last state
to its result (``observe``); ``init`` is the identity state.

Pinned by (tests/test_oracle_folds.py): the GenericFold doctest
``[1.0, 1.5, 1.75]`` (folds.jl:279-288); the online exponential fold against
two-pass log-sum-exp and softmax-weighted sums in float64; Chan/Welford
combination against two-pass variance; partition invariance of every
relative fold (any split of the elements, combined, equals the whole);
``lse_shift`` on all -Inf and +Inf inputs.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Sequence


def lse_shift(m: float) -> float:
    """folds.jl:194: shift by the maximum when finite, by zero otherwise."""
    return m if math.isfinite(m) else 0.0


class SumFold:  # folds.jl:66-71
    def init(self):
        return (0.0,)

    def lift(self, x):
        return (x,)

    def combine(self, a, b):
        return (a[0] + b[0],)

    def observe(self, s):
        return s[0]


class MaxFold:  # folds.jl:73-81
    def init(self):
        return (-math.inf,)

    def lift(self, x):
        return (x,)

    def combine(self, a, b):
        return (max(a[0], b[0]),)

    def observe(self, s):
        return s[0]


class Exponential:
    """``exp(y - m)`` against the maximum (folds.jl:126-133, 160-176, 193)."""

    def statistic_init(self):
        return (-math.inf,)

    def statistic_lift(self, y):
        return (y,)

    def statistic_combine(self, a, b):
        return (max(a[0], b[0]),)

    def statistic_of(self, s):
        return s[0]

    def split(self, s):
        return s[:1], s[1:]

    def element_sums(self, y, gs):
        return tuple(gs)

    def rebase(self, a, s, m):
        return a * math.exp(s[0] - lse_shift(m))


class Square:
    """``(y - m)^2`` against the mean, Chan's combination (folds.jl:135-192)."""

    def statistic_init(self):
        return (0.0, 0.0)

    def statistic_lift(self, y):
        return (1.0, y)

    def statistic_combine(self, a, b):
        return (a[0] + b[0], a[1] + b[1])

    def statistic_of(self, s):
        return s[1] / s[0]

    def split(self, s):
        return s[:2], s[2:]

    def element_sums(self, y, gs):
        return tuple(0.0 for _ in gs)

    def rebase(self, a, s, m):
        if s[0] == 0:
            return a
        return a + s[0] * (s[1] / s[0] - m) ** 2


@dataclass
class Relative:
    """A sum relative to a statistic of its own elements, in one pass
    (folds.jl:99-222).  An element is ``(y, g...)`` or a number ``y`` = ``(y, 1)``."""

    law: object
    observe_fn: Callable
    sums: int = 1

    def init(self):
        return tuple(self.law.statistic_init()) + tuple(0.0 for _ in range(self.sums))

    def lift(self, e):
        if not isinstance(e, tuple):
            e = (e, 1.0)
        return tuple(self.law.statistic_lift(e[0])) + tuple(self.law.element_sums(e[0], e[1:]))

    def combine(self, a, b):
        sa, xs = self.law.split(a)
        sb, ys = self.law.split(b)
        s = self.law.statistic_combine(sa, sb)
        m = self.law.statistic_of(s)
        return tuple(s) + tuple(self.law.rebase(x, sa, m) + self.law.rebase(y, sb, m) for x, y in zip(xs, ys))

    def observe(self, s):
        return self.observe_fn(self.law, s)


def statistic(law, s):
    return law.statistic_of(law.split(s)[0])


def nth_sum(i: int):
    return lambda law, s: law.split(s)[1][i]


def logsumexp_observe(law, s):
    """LOGSUMEXP = statistic + log(sum 1) (folds.jl:263)."""
    return statistic(law, s) + math.log(law.split(s)[1][0]) if law.split(s)[1][0] > 0 else -math.inf


LOGSUMEXP = Relative(Exponential(), logsumexp_observe)


@dataclass
class GenericFold:
    """folds.jl:265-303."""

    init_fn: Callable
    combine_fn: Callable
    lift_fn: Callable = lambda x: (x,)
    observe_fn: Callable = lambda s: s[0]

    def init(self):
        return self.init_fn()

    def lift(self, x):
        return self.lift_fn(x)

    def combine(self, a, b):
        return self.combine_fn(a, b)

    def observe(self, s):
        return self.observe_fn(s)


def fold(f, xs: Sequence):
    """A left fold in order from ``init``: the CPU floor's order."""
    s = f.init()
    for x in xs:
        s = f.combine(s, f.lift(x))
    return f.observe(s)


def fold_tree(f, xs: Sequence):
    """The same fold combined as a balanced tree: what a device's lanes do."""
    states = [f.lift(x) for x in xs] or [f.init()]
    while len(states) > 1:
        nxt = [f.combine(states[i], states[i + 1]) for i in range(0, len(states) - 1, 2)]
        if len(states) % 2:
            nxt.append(states[-1])
        states = nxt
    return f.observe(states[0])


def accumulate(f, xs: Sequence, exclusive: bool = False, reverse: bool = False):
    """A scan in sequence (in_sequence, folds.jl:363-386)."""
    order = range(len(xs) - 1, -1, -1) if reverse else range(len(xs))
    out = [None] * len(xs)
    s = f.init()
    for i in order:
        if exclusive:
            out[i] = f.observe(s)
        s = f.combine(s, f.lift(xs[i]))
        if not exclusive:
            out[i] = f.observe(s)
    return out
