"""Julia method signatures read as text, and the dispatch questions a binding
raises about them: which method a call reaches, and whether two methods of one
function are ambiguous or one hides the other.

No Julia toolchain exists where this backend is built, so the binding
(tempest.jl_amd/julia/HIPExt.jl) is checked by this model of Julia's rules:

- a method is `name(args...) [where {...}]`, defined at the top level of a
  file (long form `function name(...)` or short form `name(...) = ...`);
- types are nominal with parameters: `A{P...} <: B{Q...}` as the files (and a
  table of Base's array and range types) declare them, parameters invariant
  but for `Tuple`'s, `<:X` and `where` variables bindable (one binding per
  variable across a method's arguments), `Union{...}` a set, aliases
  (`const A{T} = ...`) expanded;
- method `m` is more specific than `n` when every argument type of `m` is a
  subtype of `n`'s and they differ; two methods whose argument types all
  intersect are ambiguous when neither is more specific.

It is a model, not Julia: keyword arguments, `Vararg` bounds and diagonal
rules are simplified.  What it answers is what the tests need: the methods
the binding adds against the reference's methods of the same functions.
"""
from __future__ import annotations

import pathlib
import re
from dataclasses import dataclass, field

# ---- types ---------------------------------------------------------------------------------


@dataclass(frozen=True)
class Name:
    name: str
    params: tuple = ()


@dataclass(frozen=True)
class Union_:
    members: tuple


@dataclass(frozen=True)
class Var:
    name: str
    upper: object = None  # None: Any


@dataclass(frozen=True)
class Lit:
    value: str


ANY = Name("Any")


def _strip_module(n: str) -> str:
    return n.split(".")[-1]


class _Tokens:
    def __init__(self, text: str):
        self.toks = re.findall(r"<:|::|\.\.\.|[A-Za-z_][\w.!]*|-?\d+|[{}(),:=]|\S", text)
        self.i = 0

    def peek(self):
        return self.toks[self.i] if self.i < len(self.toks) else None

    def take(self, want=None):
        t = self.peek()
        if want is not None and t != want:
            raise ValueError(f"expected {want!r}, got {t!r} in {' '.join(self.toks)}")
        self.i += 1
        return t


def parse_type(text: str, vars_: dict | None = None):
    """A type expression: names with parameters, Union, `<:X` parameters,
    literals; names in `vars_` are the method's `where` variables."""
    t = _Tokens(text)
    out = _type(t, vars_ or {})
    return out


def _type(t: _Tokens, vars_: dict):
    tok = t.peek()
    if tok == "<:":
        t.take()
        return Var("_", _type(t, vars_))
    if tok is None:
        return ANY
    if re.fullmatch(r"-?\d+", tok) or tok in ("true", "false"):
        t.take()
        return Lit(tok)
    if tok == ":":  # a Symbol literal parameter, e.g. Val{:fields}
        t.take()
        return Lit(":" + t.take())
    name = _strip_module(t.take())
    params = []
    if t.peek() == "{":
        t.take()
        while t.peek() not in ("}", None):
            before = t.i
            params.append(_type(t, vars_))
            if t.peek() == ",":
                t.take()
            elif t.i == before:  # a token no type starts with: skip it
                t.take()
        if t.peek() == "}":
            t.take()
    if name in vars_ and not params:
        return vars_[name]
    if name == "Union":
        return Union_(tuple(params))
    if name == "Any":
        return ANY
    return Name(name, tuple(params))


# Base's types a binding meets, as Julia declares them (supertype with
# parameters), and its aliases.
BASE_DECLS = """
abstract type Number end
abstract type Real <: Number end
abstract type AbstractFloat <: Real end
abstract type Integer <: Real end
abstract type Signed <: Integer end
abstract type Unsigned <: Integer end
struct Bool <: Integer end
struct Int32 <: Signed end
struct Int64 <: Signed end
struct UInt8 <: Unsigned end
struct UInt32 <: Unsigned end
struct UInt64 <: Unsigned end
struct Float16 <: AbstractFloat end
struct Float32 <: AbstractFloat end
struct Float64 <: AbstractFloat end
struct BFloat16 <: AbstractFloat end
struct Symbol end
struct Nothing end
struct String end
struct DataType end
struct Function end
struct Ptr{T} end
struct Tuple end
struct NamedTuple end
struct Type{T} end
struct Val{x} end
abstract type AbstractArray{T,N} end
abstract type DenseArray{T,N} <: AbstractArray{T,N} end
struct Array{T,N} <: DenseArray{T,N} end
struct SubArray{T,N,P,I,L} <: AbstractArray{T,N} end
struct ReinterpretArray{T,N,S,A,R} <: AbstractArray{T,N} end
struct ReshapedArray{T,N,P,MI} <: AbstractArray{T,N} end
abstract type AbstractRange{T} <: AbstractArray{T,1} end
abstract type OrdinalRange{T,S} <: AbstractRange{T} end
abstract type AbstractUnitRange{T} <: OrdinalRange{T,T} end
struct UnitRange{T} <: AbstractUnitRange{T} end
"""
BASE_ALIASES = {
    "Vector": (["T"], "Array{T,1}"), "Matrix": (["T"], "Array{T,2}"),
    "DenseVector": (["T"], "DenseArray{T,1}"), "AbstractVector": (["T"], "AbstractArray{T,1}"),
    "AbstractMatrix": (["T"], "AbstractArray{T,2}"), "Int": ([], "Int64"), "Cint": ([], "Int32"),
    "Cvoid": ([], "Nothing"), "Cdouble": ([], "Float64"), "Csize_t": ([], "UInt64"), "Dims": ([], "Tuple"),
    "StridedArray": ([], "AbstractArray"), "AbstractString": ([], "String"),
}


@dataclass
class Decl:
    name: str
    vars: list
    super: object  # a Name over `vars`, or ANY


class Types:
    """The declared types and aliases of some Julia files, on Base's."""

    def __init__(self):
        self.decls: dict[str, Decl] = {}
        self.aliases: dict[str, tuple[list, str]] = dict(BASE_ALIASES)
        self.add_text(BASE_DECLS)

    def add_text(self, text: str) -> None:
        for m in re.finditer(r"^(?:mutable\s+)?(?:struct|abstract\s+type)\s+(\w+)(\{[^}]*\})?(?:\s*<:\s*([^\n#]+?))?\s*(?:end)?\s*$",
                             text, flags=re.M):
            name, params, sup = m.group(1), m.group(2), m.group(3)
            vs = [re.split(r"\s*<:\s*", p.strip())[0] for p in params[1:-1].split(",")] if params else []
            env = {v: Var(v) for v in vs}
            self.decls.setdefault(name, Decl(name, vs, parse_type(sup, env) if sup else ANY))
        for m in re.finditer(r"^const\s+(\w+)(\{[^}]*\})?\s*=\s*((?:Union|[A-Z][\w.]*)\{.*|[A-Z][\w.]*)\s*$", text, flags=re.M):
            vs = [p.strip() for p in m.group(2)[1:-1].split(",")] if m.group(2) else []
            self.aliases.setdefault(m.group(1), (vs, m.group(3)))

    # Aliases expanded, repeatedly.
    def resolve(self, t):
        if isinstance(t, Union_):
            return Union_(tuple(self.resolve(x) for x in t.members))
        if isinstance(t, Var):
            return Var(t.name, None if t.upper is None else self.resolve(t.upper))
        if isinstance(t, Name):
            if t.name in self.aliases and t.name not in self.decls:
                vs, body = self.aliases[t.name]
                # A parameter the use leaves out is free: an anonymous variable,
                # never bound to another argument's.
                env = {v: (self.resolve(t.params[i]) if i < len(t.params) else Var("_")) for i, v in enumerate(vs)}
                return self.resolve(parse_type(body, env))
            return Name(t.name, tuple(self.resolve(p) for p in t.params))
        return t

    def supertype(self, t: Name):
        d = self.decls.get(t.name)
        if d is None or d.super == ANY or t.name == "Any":
            return None
        env = {v: (t.params[i] if i < len(t.params) else Var(v)) for i, v in enumerate(d.vars)}
        return self.resolve(_subst(d.super, env))

    # -- relations --
    def sub(self, a, b, env=None) -> bool:
        """a <: b, binding b's variables in `env` (a dict, shared across a call's arguments)."""
        env = {} if env is None else env
        a, b = self.resolve(a), self.resolve(b)
        if b == ANY:
            return True
        if isinstance(a, Union_):
            return all(self.sub(x, b, env) for x in a.members)
        if isinstance(b, Union_):
            for x in b.members:
                trial = dict(env)
                if self.sub(a, x, trial):
                    env.update(trial)
                    return True
            return False
        if isinstance(b, Var):
            if b.upper is not None and not self.sub(a, b.upper, env):
                return False
            if b.name == "_":
                return True
            if b.name in env:
                return self.same(env[b.name], a)
            env[b.name] = a
            return True
        if isinstance(a, Var):
            return self.sub(ANY if a.upper is None else a.upper, b, env)
        if isinstance(a, Lit) or isinstance(b, Lit):
            return a == b
        if a == ANY:
            return False
        while a is not None:
            if a.name == b.name:
                return self._params(a, b, env)
            a = self.supertype(a)
        return False

    def _params(self, a: Name, b: Name, env) -> bool:
        for i, bp in enumerate(b.params):
            if i >= len(a.params):
                ap = Var("_")
            else:
                ap = a.params[i]
            if isinstance(bp, Var):
                if not self.sub(ap, bp, env):
                    return False
            elif isinstance(ap, Var):
                # An unbound parameter of `a` (a UnionAll) is not inside a fixed one.
                return False
            elif a.name == "Tuple":
                if not self.sub(ap, bp, env):
                    return False
            elif not (self.same(ap, bp)):
                return False
        return True

    def same(self, a, b) -> bool:
        return self.sub(a, b, {}) and self.sub(b, a, {})

    def disjoint(self, a, b) -> bool:
        """No value has both types (nominal single inheritance: two types
        intersect only if one is a subtype of the other, or through unions
        and variables)."""
        a, b = self.resolve(a), self.resolve(b)
        if a == ANY or b == ANY:
            return False
        if isinstance(a, Union_):
            return all(self.disjoint(x, b) for x in a.members)
        if isinstance(b, Union_):
            return all(self.disjoint(a, x) for x in b.members)
        if isinstance(a, Var):
            return a.upper is not None and self.disjoint(a.upper, b)
        if isinstance(b, Var):
            return b.upper is not None and self.disjoint(a, b.upper)
        if isinstance(a, Lit) or isinstance(b, Lit):
            return a != b
        return not (self._loose_sub(a, b) or self._loose_sub(b, a))

    def _loose_sub(self, a: Name, b: Name) -> bool:
        """a's name reaches b's name going up, parameters intersecting."""
        while a is not None:
            if a.name == b.name:
                return all(not self.disjoint(x, y) for x, y in zip(a.params, b.params))
            a = self.supertype(a)
        return False


def show(t) -> str:
    """A type as Julia writes it."""
    if isinstance(t, Name):
        return t.name + ("{" + ", ".join(map(show, t.params)) + "}" if t.params else "")
    if isinstance(t, Union_):
        return "Union{" + ", ".join(map(show, t.members)) + "}"
    if isinstance(t, Var):
        return ("<:" + show(t.upper)) if t.upper is not None else t.name
    return t.value


def _subst(t, env):
    if isinstance(t, Var) and t.name in env:
        return env[t.name]
    if isinstance(t, Name):
        return Name(t.name, tuple(_subst(p, env) for p in t.params))
    if isinstance(t, Union_):
        return Union_(tuple(_subst(p, env) for p in t.members))
    if isinstance(t, Var):
        return Var(t.name, None if t.upper is None else _subst(t.upper, env))
    return t


# ---- methods -------------------------------------------------------------------------------


@dataclass
class Method:
    name: str           # the function, module prefix stripped
    qualified: str      # as written (e.g. Base.copyto!, Tempest.Compiler.capture)
    args: list          # argument types
    vararg: bool
    file: str
    line: int
    text: str = field(repr=False, default="")

    def where(self) -> str:
        return f"{self.file}:{self.line}: {self.text.strip()[:140]}"


def _split_top(s: str, seps=",") -> list[str]:
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "({[":
            depth += 1
        elif ch in ")}]":
            depth -= 1
        if ch in seps and depth == 0:
            out.append(cur)
            cur = ""
            if ch == ";":
                out.append(";")
        else:
            cur += ch
    out.append(cur)
    return out


def _balanced(text: str, start: int) -> int:
    """The index after the bracket that closes the one at `start`."""
    depth = 0
    for i in range(start, len(text)):
        if text[i] in "({[":
            depth += 1
        elif text[i] in ")}]":
            depth -= 1
            if depth == 0:
                return i + 1
    raise ValueError("unbalanced")


_HEAD = re.compile(r"^(function\s+)?((?:[A-Za-z_]\w*\.)*[A-Za-z_][\w!]*)\s*(\{[^}]*\})?\(", re.M)


def methods(text: str, file: str = "") -> list[Method]:
    """Every method defined at the top level (column 0) of a Julia file."""
    out = []
    for m in _HEAD.finditer(text):
        qual = m.group(2)
        if qual in ("function", "struct", "if", "for", "while", "begin", "let", "module", "macro", "return",
                    "using", "import", "export", "public", "include", "const", "Base.@kwdef"):
            continue
        open_ = m.end() - 1
        try:
            close = _balanced(text, open_)
        except ValueError:
            continue
        rest = text[close:close + 400]
        long_form = m.group(1) is not None
        where = ""
        wm = re.match(r"\s*(?:::\s*[\w.{}, ]+?\s*)?where\s*(\{[^}]*\}|\w+(?:\s*<:\s*[\w.{}]+)?)", rest)
        if wm:
            where = wm.group(1).strip("{}")
            after = rest[wm.end():]
        else:
            after = rest
        if not long_form:
            # Short form: `name(args) [where ...] = body` (not `==`).
            if not re.match(r"\s*(?:::\s*[\w.{}, ]+?)?\s*=(?!=)", after):
                continue
        vars_ = {}
        for w in (_split_top(where) if where else []):
            w = w.strip()
            if not w:
                continue
            parts = re.split(r"\s*<:\s*", w, maxsplit=1)
            vars_[parts[0]] = Var(parts[0], parse_type(parts[1], vars_) if len(parts) > 1 else None)
        inner = text[open_ + 1:close - 1]
        args, vararg = [], False
        for a in _split_top(inner, ",;"):
            if a == ";":
                break
            a = a.strip()
            if not a:
                continue
            a = re.sub(r"^@nospecialize\((.*)\)$", r"\1", a)
            a = re.split(r"(?<![=!<>])=(?!=)", a, maxsplit=1)[0].strip()  # default value
            if a.endswith("..."):
                vararg = True
                a = a[:-3]
            if "::" in a:
                t = a.split("::", 1)[1].strip()
                args.append(parse_type(t, vars_))
            else:
                args.append(ANY)
        line = text.count("\n", 0, m.start()) + 1
        out.append(Method(_strip_module(qual), qual, args, vararg, file, line, text[m.start():close]))
    return out


# ---- dispatch ------------------------------------------------------------------------------


def _arity_pairs(m: Method, n: Method):
    """The argument types of m and n aligned, or None if no call fits both."""
    a, b = list(m.args), list(n.args)
    if len(a) == len(b):
        return a, b
    if m.vararg and len(a) - 1 <= len(b):
        a = a[:-1] + [a[-1]] * (len(b) - len(a) + 1) if a else [ANY] * len(b)
        return a, b
    if n.vararg and len(b) - 1 <= len(a):
        b = b[:-1] + [b[-1]] * (len(a) - len(b) + 1) if b else [ANY] * len(a)
        return a, b
    return None


def more_specific(types: Types, m: Method, n: Method) -> bool:
    """m's argument types are all subtypes of n's, and not all the same."""
    pair = _arity_pairs(m, n)
    if pair is None:
        return False
    a, b = pair
    env: dict = {}
    if not all(types.sub(x, y, env) for x, y in zip(a, b)):
        return False
    return not all(types.sub(y, x, {}) for x, y in zip(a, b)) or (n.vararg and not m.vararg)


def intersect(types: Types, m: Method, n: Method) -> bool:
    pair = _arity_pairs(m, n)
    if pair is None:
        return False
    return not any(types.disjoint(x, y) for x, y in zip(*pair))


def conflict(types: Types, ours: Method, theirs: Method) -> str | None:
    """Why `ours` fails beside `theirs`, or None: ambiguous, hidden by theirs,
    or the same signature (an overwrite)."""
    if not intersect(types, ours, theirs):
        return None
    if more_specific(types, ours, theirs):
        return None
    if more_specific(types, theirs, ours):
        return "hidden: the reference's method is more specific where both apply"
    pair = _arity_pairs(ours, theirs)
    if pair and all(types.same(x, y) for x, y in zip(*pair)):
        return "the same signature: an overwrite of the reference's method"
    return "ambiguous: neither method is more specific where both apply"


def applies(types: Types, m: Method, call: list) -> bool:
    args = list(m.args)
    if m.vararg:
        if len(call) < len(args) - 1:
            return False
        args = args[:-1] + [args[-1]] * (len(call) - len(args) + 1)
    if len(args) != len(call):
        return False
    env: dict = {}
    return all(types.sub(c, a, env) for c, a in zip(call, args))


def load_types(*texts: str) -> Types:
    t = Types()
    for x in texts:
        t.add_text(x)
    return t


def julia_files(root: pathlib.Path) -> list[pathlib.Path]:
    return sorted(root.rglob("*.jl"))
