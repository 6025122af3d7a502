"""Op class (a), generated: the floor for any pointwise or reduction group.

The reference's floor realizes any group one item at a time from the group's
terms (src/Compiler/codegen/scalar.jl:1-250): ``Load`` (an element of a value
at an affine position), ``Lit``, ``Ix`` (a position as a number), ``Stat``
(a fold's result) and ``Apply`` (a function of terms); a reduction group
folds some of its axes, in phases, and writes outputs at every position
(``full``) or once per item.  ``FloorGroup`` states such a group and hands it
to ``th_build_floor`` (include/tempest_hip.h), which writes a gfx950 kernel
for it, compiles it at run time and caches the code object on disk.

Axes are the reference's column-major ones (axis 0 fastest); positions are
zero-based, so an affine index of a dense n x m value at (i0, i1) is
``i0 + n * i1``.

    g = FloorGroup("reduction", (n, m), reduced=(0,))
    x = g.value("x", "f32", n * m)
    ...
    e = g.fold("exp", g.load("x", (1, n)))          # Relative{Exponential}
    g.output("lse", e.logsumexp, (0, 1), full=False)
    launch = g.build({"x": ptr_x, "lse": ptr_lse})
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

from . import _lib
from ._lib import Affine, FloorDesc, FloorValue, FoldStruct, OutputStruct, TermStruct, call  # noqa: F401
from .launch import Launch
from .runtime import Group

RANK = _lib.FLOOR_RANK

GROUP = {"pointwise": 0, "reduction": 1, "scan": 2, "recurrence": 3}
TERM = {"load": 0, "lit": 1, "index": 2, "stat": 3, "apply": 4, "recompute": 5}
STEP = {"each": 0, "first": 1, "last": 2, "carry": 3}  # a recurrence output's rule
FN = {name: k for k, name in enumerate([
    "+", "-", "*", "/", "neg", "abs", "abs2", "sqrt", "exp", "log", "tanh", "sin", "cos", "log1p", "expm1", "^",
    "max", "min", "<", "<=", ">", ">=", "==", "!=", "ifelse", "round", "floor", "ceil", "sign", "clamp", "fma",
    "inv", "bfloat16", "dropout"])}
ARITY = {name: (2 if name in ("+", "-", "*", "/", "^", "max", "min", "<", "<=", ">", ">=", "==", "!=") else
                3 if name in ("ifelse", "clamp", "fma", "dropout") else 1) for name in FN}
FOLD = {"sum": 0, "prod": 1, "max": 2, "min": 3, "exp": 4, "square": 5, "linear": 6, "argmax": 7, "argmin": 8}
SCAN = {None: 0, "inclusive": 1, "exclusive": 2}
OBSERVE = {"value": 0, "statistic": 1, "sum": 2, "logsumexp": 3}
DTYPE = {"f32": 0, "bf16": 1, "i32": 2, "i64": 3}


class Term:
    """A term of a FloorGroup; arithmetic on terms (and numbers) applies."""

    __slots__ = ("group", "index")

    def __init__(self, group: "FloorGroup", index: int):
        self.group = group
        self.index = index

    def _f(self, fn, *others):
        return self.group.apply(fn, self, *others)

    def __add__(self, o): return self._f("+", o)
    def __radd__(self, o): return self.group.apply("+", o, self)
    def __sub__(self, o): return self._f("-", o)
    def __rsub__(self, o): return self.group.apply("-", o, self)
    def __mul__(self, o): return self._f("*", o)
    def __rmul__(self, o): return self.group.apply("*", o, self)
    def __truediv__(self, o): return self._f("/", o)
    def __rtruediv__(self, o): return self.group.apply("/", o, self)
    def __neg__(self): return self._f("neg")
    def __pow__(self, o): return self._f("^", o)


@dataclass
class Fold:
    group: "FloorGroup"
    number: int
    kind: str
    recomputed: bool = False  # computed where it is read (phase 0), over axes of its own

    def _stat(self, observe: str) -> Term:
        return self.group._term("recompute" if self.recomputed else "stat", ref=self.number,
                                observe=OBSERVE[observe])

    @property
    def value(self) -> Term:
        """A plain fold's result (sum, prod, max, min)."""
        return self._stat("value")

    @property
    def statistic(self) -> Term:
        """The exponential fold's maximum; the square fold's mean."""
        return self._stat("statistic")

    @property
    def sum(self) -> Term:
        """The exponential fold's weighted sum of exp(y - lse_shift(m)); the
        square fold's sum of squared deviations."""
        return self._stat("sum")

    @property
    def logsumexp(self) -> Term:
        return self._stat("logsumexp")

    @property
    def product(self) -> Term:
        """The linear fold's product of its factors a."""
        return self._stat("statistic")

    @property
    def index(self) -> Term:
        """An extreme fold's index (its weight where the extreme is)."""
        return self._stat("statistic")


PART = {"div": 1, "mod": 2}


def _affine(coeffs: Sequence[int] | None, constant: int, rank: int, gather=None, gather_coeff: int = 1,
            parts=()) -> tuple:
    """(constant, coefficients, gather term, gather coefficient, div/mod parts).
    A part is ("div" | "mod", inner coefficients, divisor, coefficient[, inner
    constant]): coefficient * fld or mod(inner constant + sum inner[k] i_k,
    divisor), the Div and Mod atoms; at most two."""
    c = list(coeffs or ())
    if len(c) > RANK:  # beyond the domain's rank: a recomputed fold's own axes
        raise ValueError(f"{len(c)} coefficients: at most {RANK} positions")
    if len(parts) > 2:
        raise ValueError("at most two div / mod atoms an address")
    g = -1 if gather is None else gather.index
    ps = []
    for part in parts:
        kind, inner, dv, cf = part[:4]
        inner = list(inner)
        if len(inner) > rank:
            raise ValueError(f"{len(inner)} inner coefficients for a rank-{rank} domain")
        ps.append((PART[kind], tuple(int(x) for x in inner) + (0,) * (RANK - len(inner)), int(dv), int(cf),
                   int(part[4]) if len(part) > 4 else 0))
    ps = tuple(ps)
    return (int(constant), tuple(int(x) for x in c) + (0,) * (RANK - len(c)), g, int(gather_coeff), ps)


def _fill(dst, aff) -> None:
    c0, cs, gt, gc, ps = aff
    dst.constant, dst.gather, dst.gather_coeff = c0, gt, gc
    dst.coeff[:] = list(cs)
    for j, (kind, inner, dv, cf, c) in enumerate(ps):
        q = dst.part[j]
        q.kind, q.divisor, q.coeff, q.constant = kind, dv, cf, c
        q.inner[:] = list(inner)


@dataclass
class FloorGroup:
    """A pointwise or reduction group of the floor (scalar.jl:186-250)."""

    kind: str
    extents: tuple
    reduced: tuple = ()                             # folded axes (a scan group: scanned)
    name: str = "floor group"
    reverse: bool = False                           # a scan or recurrence group from its last position
    step: int = -1                                  # a recurrence group's step axis (one of `reduced`)
    ordered: bool = False                           # a pointwise group's items one after another (TH_FLOOR_ORDERED)
    values: dict = field(default_factory=dict)      # name -> (dtype, length), in value order
    terms: list = field(default_factory=list)       # (op, fn, args, ref, observe, lit, affine)
    folds: list = field(default_factory=list)       # (kind, phase, body, weight, scan, inner extents)
    outputs: list = field(default_factory=list)     # (value, term, full, affine)

    def __post_init__(self):
        if self.kind not in GROUP:
            raise ValueError(f"unknown group kind {self.kind!r}")
        self.extents = tuple(int(e) for e in self.extents)
        if not 1 <= len(self.extents) <= RANK:
            raise ValueError("a group's domain has 1 to 4 axes")
        self.reduced = tuple(int(k) for k in self.reduced)

    # -- building the group -------------------------------------------------------

    def value(self, name: str, dtype: str, length: int) -> str:
        """A value the group reads or writes: f32 or bf16, or i32 / i64 indices (read only)."""
        if dtype not in DTYPE:
            raise ValueError(f"values are f32, bf16, i32 or i64, not {dtype!r}")
        self.values[name] = (dtype, int(length))
        return name

    def _term(self, op: str, fn: int = 0, args=(), ref: int = 0, observe: int = 0, lit: float = 0.0,
              affine=(0, (0,) * RANK, -1, 0, ())) -> Term:
        self.terms.append((TERM[op], fn, tuple(args) + (0,) * (3 - len(args)), ref, observe, float(lit), affine))
        return Term(self, len(self.terms) - 1)

    def _as_term(self, x) -> Term:
        if isinstance(x, Term):
            if x.group is not self:
                raise ValueError("a term of another group")
            return x
        return self.lit(float(x))

    def load(self, name: str, coeffs: Sequence[int] | None = None, constant: int = 0, gather: Term | None = None,
             gather_coeff: int = 1, parts=()) -> Term:
        """Element ``constant + sum(coeffs[k] * i_k) (+ gather_coeff * gather)
        (+ each part: coefficient * fld|mod(inner affine, divisor))`` of value
        ``name``; ``gather`` is a load of integers (an Indirect atom)."""
        ref = list(self.values).index(name)
        return self._term("load", ref=ref,
                          affine=_affine(coeffs, constant, len(self.extents), gather, gather_coeff, parts))

    def lit(self, x: float) -> Term:
        return self._term("lit", lit=x)

    def index(self, coeffs: Sequence[int], constant: int = 0, parts=()) -> Term:
        """The number ``constant + sum(coeffs[k] * i_k)`` (+ div / mod parts) (Ix)."""
        return self._term("index", affine=_affine(coeffs, constant, len(self.extents), parts=parts))

    def apply(self, fn: str, *args) -> Term:
        if fn not in FN:
            raise ValueError(f"unknown function {fn!r}")
        if len(args) != ARITY[fn]:
            raise ValueError(f"{fn} takes {ARITY[fn]} arguments")
        ts = [self._as_term(a) for a in args]
        return self._term("apply", fn=FN[fn], args=[t.index for t in ts])

    def fold(self, kind: str, body, weight=None, phase: int = 1, scan: str | None = None) -> Fold:
        """A fold of ``body`` over the group's folded axes.  ``weight``: the
        exponential fold's weight, the linear fold's offset b (h = body h' + b).
        In a scan group, ``scan`` = "inclusive" or "exclusive" makes its result
        the running one at each position; folds take their elements in
        (phase, order of definition) order."""
        if self.kind == "pointwise":
            raise ValueError("only a reduction group folds")
        if kind not in FOLD:
            raise ValueError(f"unknown fold {kind!r}")
        if scan not in SCAN or (scan and self.kind != "scan"):
            raise ValueError("only a scan group's folds scan (inclusive or exclusive)")
        b = self._as_term(body).index
        w = -1 if weight is None else self._as_term(weight).index
        self.folds.append((FOLD[kind], int(phase), b, w, SCAN[scan], ()))
        return Fold(self, len(self.folds) - 1, kind)

    def recompute(self, kind: str, body, inner: Sequence[int], weight=None) -> Fold:
        """A fold computed where it is read (the reference's Recomputed term):
        its body over the group's positions and axes of its own, of extents
        ``inner``, numbered after the group's (coefficient rank, rank + 1, ...
        of the addresses its body reaches)."""
        if kind not in FOLD:
            raise ValueError(f"unknown fold {kind!r}")
        b = self._as_term(body).index
        w = -1 if weight is None else self._as_term(weight).index
        self.folds.append((FOLD[kind], 0, b, w, 0, tuple(int(e) for e in inner)))
        return Fold(self, len(self.folds) - 1, kind, recomputed=True)

    def output(self, name: str, term, coeffs: Sequence[int] | None = None, constant: int = 0,
               full: bool = True, gather: Term | None = None, gather_coeff: int = 1,
               accumulate: bool = False, parts=(), when: str | None = None) -> None:
        """Write ``term`` at the address (every position, or once per item);
        ``accumulate`` adds it instead, atomically (a fold by key).  In a
        recurrence group, ``when`` is the step rule: "each", "first" (a state
        where it starts), "last", or "carry" (every step but the last, the
        address one step on)."""
        v = list(self.values).index(name)
        rule = STEP[when or "each"] if self.kind == "recurrence" else int(bool(full))
        self.outputs.append((v, self._as_term(term).index, rule,
                             _affine(coeffs, constant, len(self.extents), gather, gather_coeff, parts),
                             int(bool(accumulate))))

    # -- the ABI ---------------------------------------------------------------------

    def _desc(self, ptrs: Sequence[int]):
        nv, nt, nf, no = len(self.values), len(self.terms), len(self.folds), len(self.outputs)
        values = (FloorValue * nv)()
        for k, ((dt, n), p) in enumerate(zip(self.values.values(), ptrs)):
            values[k].dtype, values[k].length, values[k].ptr = DTYPE[dt], n, p
        terms = (TermStruct * max(nt, 1))()
        for k, (op, fn, args, ref, obs, lit, aff) in enumerate(self.terms):
            t = terms[k]
            t.op, t.fn, t.ref, t.observe, t.lit = op, fn, ref, obs, lit
            t.args[:] = list(args)
            _fill(t.index, aff)
        folds = (FoldStruct * max(nf, 1))()
        for k, (kind, phase, body, weight, scan, inner) in enumerate(self.folds):
            folds[k].kind, folds[k].phase, folds[k].body, folds[k].weight = kind, phase, body, weight
            folds[k].scan, folds[k].n_inner = scan, len(inner)
            folds[k].inner[:] = list(inner) + [0] * (RANK - len(inner))
        outs = (OutputStruct * max(no, 1))()
        for k, (v, term, full, aff, acc) in enumerate(self.outputs):
            outs[k].value, outs[k].term, outs[k].full, outs[k].accumulate = v, term, full, acc
            _fill(outs[k].index, aff)
        d = FloorDesc()
        d.kind, d.rank = GROUP[self.kind], len(self.extents)
        d.extents[:] = list(self.extents) + [1] * (RANK - len(self.extents))
        d.reduced = sum(1 << k for k in self.reduced)
        d.n_values, d.n_terms, d.n_folds, d.n_outputs = nv, nt, nf, no
        d.flags = ((1 if self.reverse else 0) | ((self.step << 8) if self.kind == "recurrence" else 0) |
                   ((1 << 16) if self.ordered else 0))
        d.values, d.terms, d.folds, d.outputs = values, terms, folds, outs
        return d, (values, terms, folds, outs)

    def _stand_in(self) -> list[int]:
        # Addresses for a build without a device: 256-byte aligned, as device
        # allocations are, so the source is the one a device build writes.
        return [(k + 1) << 20 for k in range(len(self.values))]

    def source(self, ptrs: Sequence[int] | None = None) -> str:
        """The generated HIP source (needs no device)."""
        d, keep = self._desc(ptrs or self._stand_in())
        need = _lib.c_size()
        call("th_floor_source", ctypes.byref(d), None, 0, ctypes.byref(need))
        buf = ctypes.create_string_buffer(need.value)
        call("th_floor_source", ctypes.byref(d), buf, need.value, ctypes.byref(need))
        return buf.value.decode()

    def compile(self, ptrs: Sequence[int] | None = None) -> None:
        """Compile into the code-object cache (needs no device)."""
        d, keep = self._desc(ptrs or self._stand_in())
        call("th_floor_compile", ctypes.byref(d))

    def build(self, ptrs: dict[str, int]) -> Launch:
        """The group's launch over the values at ``ptrs`` (name -> device address)."""
        order = list(self.values)
        missing = [n for n in order if n not in ptrs]
        if missing:
            raise ValueError(f"{self.name}: no address for {missing}")
        d, keep = self._desc([int(ptrs[n]) for n in order])
        out = ctypes.c_void_p()
        call("th_build_floor", ctypes.byref(d), ctypes.byref(out))
        return Launch(out, tuple(order))

    def as_group(self) -> Group:
        """The group as a kernel of a Program (runtime.Group)."""
        order = tuple(self.values)
        writes = tuple(dict.fromkeys(order[o[0]] for o in self.outputs))
        reads = tuple(dict.fromkeys(order[self.terms[t][3]] for t in range(len(self.terms))
                                    if self.terms[t][0] == TERM["load"]))
        return Group(self.name, order, reads, writes, self.build)

    def spec(self) -> dict:
        """A plain description of the group (for checkers)."""
        inv_fn = {v: k for k, v in FN.items()}
        inv_fold = {v: k for k, v in FOLD.items()}
        inv_obs = {v: k for k, v in OBSERVE.items()}
        inv_term = {v: k for k, v in TERM.items()}
        inv_scan = {v: k for k, v in SCAN.items()}
        return {
            "kind": self.kind, "extents": self.extents, "reduced": self.reduced, "reverse": self.reverse,
            "values": dict(self.values),
            "terms": [{"op": inv_term[op], "fn": inv_fn.get(fn) if op == TERM["apply"] else None,
                       "args": list(args[:ARITY[inv_fn[fn]]]) if op == TERM["apply"] else [],
                       "ref": ref, "observe": inv_obs[obs], "lit": lit, "constant": aff[0], "coeffs": list(aff[1]),
                       "gather": aff[2], "gather_coeff": aff[3], "parts": list(aff[4])}
                      for op, fn, args, ref, obs, lit, aff in self.terms],
            "folds": [{"kind": inv_fold[k], "phase": p, "body": b, "weight": w, "scan": inv_scan[sc], "inner": inner}
                      for k, p, b, w, sc, inner in self.folds],
            "step": self.step,
            "outputs": [{"value": list(self.values)[v], "term": t, "full": int(f), "constant": aff[0],
                         "coeffs": list(aff[1]), "gather": aff[2], "gather_coeff": aff[3], "parts": list(aff[4]),
                         "accumulate": bool(acc)}
                        for v, t, f, aff, acc in self.outputs],
        }
