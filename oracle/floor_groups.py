"""TEST INFRASTRUCTURE ONLY: the Float64 meaning of a floor group.

A group (tempest_hip.floor.FloorGroup.spec()) is evaluated as the reference's
plan-free interpreter evaluates the program it came from
(src/Compiler/program/interpret.jl): every term over the whole domain at
once, in Float64, each fold over the group's folded axes by the fold algebra
of src/Compiler/IR/folds.jl (a sum, product, maximum or minimum; the
exponential fold's maximum m and sum of weight * exp(y - lse_shift(m)),
folds.jl:126-133,160-176,193-194; the square fold's mean and sum of squared
deviations, folds.jl:135-192; the linear recurrence h = a h' + b, the
`chain` of test/fixtures/programs.jl:54-55), phase after phase, then the outputs: a full
output at every position of the domain, the others once per item with the
folded positions at zero (scalar.jl:232-248).  A scan group steps its
scanned positions in order (reversed if asked), every item at once: at each
position the folds take their elements in (phase, definition) order, a
scan's result read before (exclusive) or after (inclusive) its element, then
the full outputs (scan_kernel, scalar.jl:350-398; in_sequence, folds.jl:
372-386).  Written values are rounded once to their type (Float32, or
bfloat16 to nearest, ties to even).

Parity pinned by (tests/test_oracle_floor.py): each fold kind against the
sequential restatement in ``oracle.folds`` on the same elements (lift, then
combine earlier-first); each of the reference's fixture programs expressed as
groups against a closed form written independently with numpy
(test/fixtures/programs.jl:60-90 and the row programs); the reference's
doctest sum(abs2, [1, 2, 3, 4]) == 30 (runtime/compile.jl:35-40); a planted
mistake (the exponential fold without its rebase) is caught.
"""
from __future__ import annotations

import numpy as np

from .data import bf16_round

_UNARY = {
    "neg": np.negative, "abs": np.abs, "abs2": np.square, "sqrt": np.sqrt, "exp": np.exp, "log": np.log,
    "tanh": np.tanh, "sin": np.sin, "cos": np.cos, "log1p": np.log1p, "expm1": np.expm1,
    "round": np.rint, "floor": np.floor, "ceil": np.ceil, "sign": np.sign, "inv": lambda x: 1.0 / x,
    "bfloat16": lambda x: bf16_round(np.asarray(x, dtype=np.float32)).astype(np.float64),
}
_BINARY = {
    "+": np.add, "-": np.subtract, "*": np.multiply, "/": np.divide, "^": np.power,
    "max": np.fmax, "min": np.fmin,
    "<": lambda a, b: (a < b) * 1.0, "<=": lambda a, b: (a <= b) * 1.0, ">": lambda a, b: (a > b) * 1.0,
    ">=": lambda a, b: (a >= b) * 1.0, "==": lambda a, b: (a == b) * 1.0, "!=": lambda a, b: (a != b) * 1.0,
}


def _ternary(fn, a, b, c):
    if fn == "ifelse":
        return np.where(a != 0, b, c)
    if fn == "clamp":
        return np.where(a > c, c, np.where(a < b, b, a))
    if fn == "fma":
        return a * b + c
    if fn == "dropout":
        return dropout_scale(a, b, c)
    raise ValueError(fn)


def dropout_scale(key, pos, rate):
    """The dropout fixture's keep scale (test/fixtures/operations.jl:88-103,
    stream 0): Int32 products of the key and the 1-based position with the
    fixture's constants, wrapping, xor-folded; logical shifts; the top 24
    bits as a Float32 fraction u; 1 / (1 - rate) in Float32 when u >= rate.
    Computed in Python integers masked to 32 bits."""
    key, pos, rate = np.broadcast_arrays(np.asarray(key), np.asarray(pos), np.asarray(rate))
    out = np.empty(key.shape)
    m = 0xFFFFFFFF
    for idx in np.ndindex(key.shape):
        h = ((int(key[idx]) * -1640531535) & m) ^ ((int(pos[idx]) * -1028477387) & m)
        h ^= h >> 16
        h = (h * 2146121005) & m
        h ^= h >> 15
        h = (h * -2073254261) & m
        h ^= h >> 16
        u = np.float32(h >> 8) * np.float32(2.0 ** -24)
        r = np.float32(rate[idx])
        out[idx] = np.float32(1) / (np.float32(1) - r) if u >= r else 0.0
    return out


def fold_reduce(kind: str, y: np.ndarray, g, axes: tuple):
    """A fold's state over ``axes`` of ``y`` (keepdims), as a dict of observations."""
    if kind == "sum":
        return {"value": y.sum(axis=axes, keepdims=True)}
    if kind == "prod":
        return {"value": y.prod(axis=axes, keepdims=True)}
    if kind == "max":
        return {"value": y.max(axis=axes, keepdims=True, initial=-np.inf)}
    if kind == "min":
        return {"value": y.min(axis=axes, keepdims=True, initial=np.inf)}
    if kind == "exp":
        m = y.max(axis=axes, keepdims=True, initial=-np.inf)
        sh = np.where(np.isfinite(m), m, 0.0)
        w = 1.0 if g is None else g
        s = (w * np.exp(y - sh)).sum(axis=axes, keepdims=True)
        with np.errstate(divide="ignore", invalid="ignore"):
            return {"statistic": m, "sum": s, "logsumexp": sh + np.log(s)}
    if kind == "linear":
        # In order over the folded positions, first axis fastest: h = a h + b.
        yy = np.moveaxis(y, axes, tuple(range(len(axes))))
        gg = np.moveaxis(np.broadcast_to(g, y.shape), axes, tuple(range(len(axes))))
        cnt = int(np.prod(yy.shape[:len(axes)]))
        ya = yy.reshape((cnt,) + yy.shape[len(axes):], order="F")
        ga = gg.reshape((cnt,) + gg.shape[len(axes):], order="F")
        p, h = np.ones(ya.shape[1:]), np.zeros(ya.shape[1:])
        for i in range(cnt):
            p, h = p * ya[i], ya[i] * h + ga[i]
        shape = tuple(1 if k in axes else y.shape[k] for k in range(y.ndim))
        return {"value": h.reshape(shape), "statistic": p.reshape(shape)}
    if kind in ("argmax", "argmin"):
        # In order over the folded positions, first axis fastest, by the
        # extreme's combine (each pair of elements ordered alike whatever the order).
        yy = np.moveaxis(y, axes, tuple(range(len(axes))))
        gg = np.moveaxis(np.broadcast_to(g, y.shape), axes, tuple(range(len(axes))))
        cnt = int(np.prod(yy.shape[:len(axes)]))
        ya = yy.reshape((cnt,) + yy.shape[len(axes):], order="F")
        ga = gg.reshape((cnt,) + gg.shape[len(axes):], order="F")
        st = tuple(np.full(ya.shape[1:], v) for v in _INIT[kind])
        for i in range(cnt):
            st = _step(kind, st, ya[i], ga[i])
        shape = tuple(1 if k in axes else y.shape[k] for k in range(y.ndim))
        return {"value": st[0].reshape(shape), "statistic": st[1].reshape(shape)}
    if kind == "square":
        n = np.prod([y.shape[a] for a in axes]) if y.size else 0
        with np.errstate(invalid="ignore"):
            mean = y.sum(axis=axes, keepdims=True) / n
        return {"statistic": mean, "sum": ((y - mean) ** 2).sum(axis=axes, keepdims=True)}
    raise ValueError(kind)


def evaluate(spec: dict, arrays: dict[str, np.ndarray], rounded: bool = True) -> dict[str, np.ndarray]:
    """The group's written values, given every value's contents (1-D);
    rounded to the values' types, or Float64 with ``rounded=False``."""
    arrays = dict(arrays)
    ext = tuple(spec["extents"])
    rank = len(ext)
    idx = np.indices(ext, dtype=np.int64)  # idx[k]: position along axis k
    reduced = tuple(spec["reduced"])
    vals = list(spec["values"])
    out = {o["value"]: np.array(arrays[o["value"]], dtype=np.float64, copy=True) for o in spec["outputs"]}

    def addr(t, at, memo=None, length=None):
        a = np.full(np.shape(at[0]), t["constant"], dtype=np.int64)
        for k in range(len(at)):  # past the domain's rank: a recomputed fold's own axes
            if t["coeffs"][k]:
                a = a + t["coeffs"][k] * at[k]
        for kind, inner, dv, cf, c in t.get("parts", ()):  # Div (1) and Mod (2) atoms: floor division
            e = c + sum(inner[k] * at[k] for k in range(rank) if inner[k])
            a = a + cf * (np.floor_divide(e, dv) if kind == 1 else np.mod(e, dv))
        if t.get("gather", -1) >= 0:
            # An Indirect atom: the integer a load reads, held inside the value.
            a = a + t["gather_coeff"] * np.asarray(term(t["gather"], at, memo), dtype=np.int64)
            a = np.clip(a, 0, length - 1)
        return a

    stats: dict[int, dict] = {}

    def term(i, at, memo):
        if i in memo:
            return memo[i]
        t = spec["terms"][i]
        op = t["op"]
        if op == "load":
            src = np.asarray(arrays[vals[t["ref"]]])
            r = (src if src.dtype.kind == "i" else src.astype(np.float64))[addr(t, at, memo, len(src))]
        elif op == "lit":
            r = np.float64(t["lit"])
        elif op == "index":
            r = addr(t, at, memo).astype(np.float64)
        elif op == "stat":
            r = stats[t["ref"]][t["observe"]]
        elif op == "recompute":
            # The fold over its own axes, appended after the positions' shape
            # (Recomputed, codegen/scalar.jl:88-110).
            f = spec["folds"][t["ref"]]
            inner = tuple(f["inner"])
            shape = np.broadcast_shapes(*[np.shape(a) for a in at])
            grids = np.indices(inner, dtype=np.int64)
            ext_at = [np.broadcast_to(np.reshape(a, np.shape(a) + (1,) * len(inner)), shape + inner) for a in at]
            ext_at += [np.broadcast_to(grids[q].reshape((1,) * len(shape) + inner), shape + inner)
                       for q in range(len(inner))]
            inner_memo: dict = {}
            y = np.broadcast_to(term(f["body"], ext_at, inner_memo), shape + inner).astype(np.float64)
            g = None if f["weight"] < 0 else np.broadcast_to(term(f["weight"], ext_at, inner_memo), shape + inner)
            st = fold_reduce(f["kind"], y, g, tuple(range(len(shape), len(shape) + len(inner))))
            r = st[t["observe"]].reshape(shape)
        else:
            a = [term(j, at, memo) for j in t["args"]]
            fn = t["fn"]
            with np.errstate(all="ignore"):
                r = _UNARY[fn](a[0]) if len(a) == 1 else _BINARY[fn](*a) if len(a) == 2 else _ternary(fn, *a)
        memo[i] = r
        return r

    full_at = [idx[k] for k in range(rank)]
    if spec["kind"] == "recurrence":
        return _recurrence(spec, arrays, out, addr, term, rounded)
    if spec["kind"] == "scan":
        return _scan(spec, arrays, out, idx, addr, term, stats, rounded)
    if spec["kind"] == "reduction":
        for phase in sorted({f["phase"] for f in spec["folds"]}):
            memo: dict = {}
            for k, f in enumerate(spec["folds"]):
                if f["phase"] != phase:
                    continue
                y = np.broadcast_to(term(f["body"], full_at, memo), ext).astype(np.float64)
                g = None if f["weight"] < 0 else np.broadcast_to(term(f["weight"], full_at, memo), ext)
                stats[k] = fold_reduce(f["kind"], y, g, reduced)
    # Once outputs: the folded positions at zero, the kept ones everywhere.
    once_at = [idx[k][tuple(slice(0, 1) if j in reduced else slice(None) for j in range(rank))]
               for k in range(rank)]
    memo_full: dict = {}
    memo_once: dict = {}
    for o in spec["outputs"]:
        at = full_at if o["full"] else once_at
        memo = memo_full if o["full"] else memo_once
        v = np.broadcast_to(term(o["term"], at, memo), at[0].shape).astype(np.float64)
        dst = out[o["value"]]
        where = addr(o, at, memo, len(dst)).ravel()
        if o.get("accumulate"):
            np.add.at(dst, where, v.ravel())  # a fold by key: repeated positions add
        else:
            dst[where] = v.ravel()
    if not rounded:
        return out
    result = {}
    for n, a in out.items():
        dt = spec["values"][n][0]
        result[n] = bf16_round(a.astype(np.float32)) if dt == "bf16" else a.astype(np.float32)
    return result



def _recurrence(spec, arrays, out, addr, term, rounded):
    """A recurrence group (recurrence_kernel, codegen/scalar.jl:402-440): its
    steps in order, at each its outputs in order over the other reduced axes
    their addresses mention, the loads reading what was stored so far."""
    ext = tuple(spec["extents"])
    rank = len(ext)
    step, reverse = spec["step"], spec.get("reverse", False)
    E = ext[step]
    # Loads read the written values as they are written.
    for n, a in out.items():
        arrays[n] = a
    for s_ in range(E):
        pos = E - 1 - s_ if reverse else s_
        for o in spec["outputs"]:
            rule = o["full"]
            if (rule == 1 and s_ != 0) or (rule == 2 and s_ != E - 1) or (rule == 3 and s_ == E - 1):
                continue
            ranges = []
            for k in range(rank):
                mentioned = o["coeffs"][k] != 0 or any(q[1][k] for q in o.get("parts", ()) if q[3])
                if k == step:
                    ranges.append([pos])
                elif k not in spec["reduced"] or mentioned:
                    ranges.append(range(ext[k]))
                else:
                    ranges.append([0])
            at = list(np.meshgrid(*[np.asarray(r, dtype=np.int64) for r in ranges], indexing="ij"))
            memo: dict = {}
            v = np.broadcast_to(term(o["term"], at, memo), at[0].shape).astype(np.float64)
            dst = out[o["value"]]
            dst[addr(o, at, memo, len(dst)).ravel()] = v.ravel()
    if not rounded:
        return out
    return {n: (bf16_round(a.astype(np.float32)) if spec["values"][n][0] == "bf16" else a.astype(np.float32))
            for n, a in out.items()}


def _observe(kind, st):
    if kind in ("sum", "prod", "max", "min"):
        return {"value": st[0]}
    if kind == "exp":
        m, s = st
        sh = np.where(np.isfinite(m), m, 0.0)
        with np.errstate(divide="ignore", invalid="ignore"):
            return {"statistic": m, "sum": s, "logsumexp": sh + np.log(s)}
    if kind == "square":
        n, mean, q = st
        return {"statistic": np.where(n > 0, mean, np.nan), "sum": q}
    if kind in ("argmax", "argmin"):
        return {"value": st[0], "statistic": st[1]}
    return {"value": st[1], "statistic": st[0]}  # linear: (product, h)


def lesser(x, y):
    """Base's isless in comparisons alone (program/tracing.jl:788-792): NaN
    the largest, -0.0 before 0.0."""
    with np.errstate(divide="ignore"):
        return np.where(np.isnan(x), False, np.isnan(y) | (x < y) | ((x == y) & (1.0 / x < 1.0 / y)))


def greater(x, y):
    """Base's isgreater, the order findmin keeps: NaN the smallest."""
    with np.errstate(divide="ignore"):
        return np.where(np.isnan(x), False, np.isnan(y) | (y < x) | ((x == y) & (1.0 / y < 1.0 / x)))


def better(largest, a, b):
    """Of two (element, index) states the one an extreme keeps, the earlier of
    equals (`Better`, program/tracing.jl:779-784)."""
    precedes, follows = (lesser(a[0], b[0]), lesser(b[0], a[0])) if largest else (greater(a[0], b[0]), greater(b[0], a[0]))
    t = precedes | (~follows & (b[1] < a[1]))
    return np.where(t, b[0], a[0]), np.where(t, b[1], a[1])


def _step(kind, st, y, g):
    if kind in ("argmax", "argmin"):
        return better(kind == "argmax", st, (y, g))
    if kind == "sum":
        return (st[0] + y,)
    if kind == "prod":
        return (st[0] * y,)
    if kind == "max":
        return (np.maximum(st[0], y),)
    if kind == "min":
        return (np.minimum(st[0], y),)
    if kind == "exp":  # combine with lift(y, g), the oracle.folds rebase
        m, s = st
        n = np.maximum(m, y)
        sh = np.where(np.isfinite(n), n, 0.0)
        with np.errstate(invalid="ignore"):
            return (n, s * np.exp(m - sh) + g * np.exp(y - sh))
    if kind == "square":  # Welford
        n, mean, q = st
        n1 = n + 1
        e = y - mean
        mean1 = mean + e / n1
        return (n1, mean1, q + e * (y - mean1))
    p, h = st  # linear
    return (p * y, y * h + g)


_INIT = {"sum": (0.0,), "prod": (1.0,), "max": (-np.inf,), "min": (np.inf,), "exp": (-np.inf, 0.0),
         "square": (0.0, 0.0, 0.0), "linear": (1.0, 0.0), "argmax": (-np.inf, np.inf), "argmin": (np.inf, np.inf)}


def _scan(spec, arrays, out, idx, addr, term, stats, rounded):
    ext = tuple(spec["extents"])
    rank = len(ext)
    swept = tuple(spec["reduced"])
    kept_shape = tuple(1 if k in swept else ext[k] for k in range(rank))
    order = sorted(range(len(spec["folds"])), key=lambda f: spec["folds"][f]["phase"])
    states = {f: tuple(np.full(kept_shape, v) for v in _INIT[spec["folds"][f]["kind"]]) for f in order}
    positions = list(np.ndindex(*[ext[k] for k in swept][::-1]))  # last axis slowest
    positions = [tuple(reversed(p)) for p in positions]            # first swept axis fastest
    if spec.get("reverse"):
        positions = positions[::-1]
    for pos in positions:
        sl = [slice(None)] * rank
        for k, c in zip(swept, pos):
            sl[k] = slice(c, c + 1)
        at = [idx[k][tuple(sl)] for k in range(rank)]
        memo: dict = {}
        for f in order:
            fd = spec["folds"][f]
            if fd["scan"] == "exclusive":
                stats[f] = _observe(fd["kind"], states[f])
                memo.clear()
            y = np.broadcast_to(term(fd["body"], at, memo), kept_shape)
            g = None if fd["weight"] < 0 else np.broadcast_to(term(fd["weight"], at, memo), kept_shape)
            states[f] = _step(fd["kind"], states[f], y, 1.0 if g is None else g)
            if fd["scan"] == "inclusive":
                stats[f] = _observe(fd["kind"], states[f])
                memo.clear()
        for o in spec["outputs"]:
            if o["full"]:
                v = np.broadcast_to(term(o["term"], at, memo), kept_shape)
                out[o["value"]][addr(o, at, memo, len(out[o["value"]])).ravel()] = v.ravel()
    for f in order:
        if spec["folds"][f]["scan"] is None:
            stats[f] = _observe(spec["folds"][f]["kind"], states[f])
    once_at = [idx[k][tuple(slice(0, 1) if j in swept else slice(None) for j in range(rank))] for k in range(rank)]
    memo = {}
    for o in spec["outputs"]:
        if not o["full"]:
            v = np.broadcast_to(term(o["term"], once_at, memo), once_at[0].shape)
            out[o["value"]][addr(o, once_at, memo, len(out[o["value"]])).ravel()] = v.ravel()
    if not rounded:
        return out
    return {n: (bf16_round(a.astype(np.float32)) if spec["values"][n][0] == "bf16" else a.astype(np.float32))
            for n, a in out.items()}
