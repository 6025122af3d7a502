"""The Julia extension (tempest.jl_amd/julia/HIPExt.jl) against the C ABI, on
the CPU: no Julia runs here, so the binding is checked as text.  Every
`ccall((:th_..., LIB), R, (T...), ...)` names an entry point the header
declares, with the header's argument count and C types; every struct mirror
has the field names, offsets and size gcc gives the header's struct; the
group kinds the floor refuses throw rather than build a wrong kernel."""
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
JL = (ROOT / "tempest.jl_amd" / "julia" / "HIPExt.jl").read_text()
HEADER = (ROOT / "include" / "tempest_hip.h").read_text()


def _split_top(s: str) -> list[str]:
    """Split at commas outside braces and parentheses."""
    out, depth, cur = [], 0, ""
    for ch in s:
        if ch in "({":
            depth += 1
        elif ch in ")}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def _ccalls() -> list[tuple[str, str, list[str]]]:
    """(symbol, return type, argument types) of every ccall into LIB."""
    calls = []
    for m in re.finditer(r"ccall\(\(:(th_\w+),\s*LIB\),\s*", JL):
        rest = JL[m.end():]
        ret = re.match(r"[\w{}]+", rest).group(0)
        rest = rest[len(ret):].lstrip()
        assert rest.startswith(","), m.group(1)
        rest = rest[1:].lstrip()
        assert rest.startswith("("), m.group(1)
        depth, i = 0, 0
        for i, ch in enumerate(rest):
            depth += ch == "("
            depth -= ch == ")"
            if depth == 0:
                break
        calls.append((m.group(1), ret, _split_top(rest[1:i])))
    return calls


def _prototypes() -> dict[str, tuple[str, list[str]]]:
    """name -> (return type, parameter types) from the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    protos = {}
    for m in re.finditer(r"(int|const char\s*\*)\s+(th_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p.strip() for p in m.group(3).split(",") if p.strip() and p.strip() != "void"]
        types = []
        for p in params:
            p = " ".join(p.split())
            name = re.search(r"(\w+)$", p).group(1)
            types.append(p[: -len(name)].strip())
        protos[m.group(2)] = (m.group(1).replace(" ", ""), types)
    return protos


SCALAR = {"Cint": {"int"}, "Int32": {"int32_t", "int"}, "Int64": {"int64_t"}, "UInt64": {"uint64_t"},
          "Csize_t": {"size_t"}, "Float32": {"float"}, "Cdouble": {"double"}, "UInt32": {"uint32_t"}}


def _matches(jl: str, c: str) -> bool:
    c = re.sub(r"\bconst\b", "", c).replace(" ", "")
    if jl in SCALAR:
        return c in SCALAR[jl]
    if jl == "Cstring":
        return c == "char*"
    if jl.startswith("Ptr{"):
        inner = jl[4:-1]
        if not c.endswith("*"):
            return False
        if inner.startswith("Ptr{"):
            return c.endswith("**")
        return not c.endswith("**") or inner == "Cvoid"
    return False


def test_every_ccall_matches_the_header():
    protos = _prototypes()
    calls = _ccalls()
    assert len(calls) > 30
    for name, ret, args in calls:
        assert name in protos, f"{name} is not declared in include/tempest_hip.h"
        cret, cargs = protos[name]
        assert (ret, cret) in {("Cint", "int"), ("Cstring", "constchar*")}, (name, ret, cret)
        assert len(args) == len(cargs), (name, args, cargs)
        for a, c in zip(args, cargs):
            assert _matches(a, c), (name, a, c)


def test_the_binding_reaches_every_builder_and_the_pool():
    """The libraries and the target call every builder, the pool and the
    grouped products (the claims the reference's libraries make)."""
    used = {n for n, _, _ in _ccalls()}
    for name in ("th_build_gemm", "th_build_gemm_grouped", "th_build_attention_fwd", "th_build_attention_bwd",
                 "th_build_softmax_grad", "th_build_layernorm_grad", "th_build_softmax_fwd", "th_build_layernorm_fwd",
                 "th_build_deltanet", "th_build_deltanet_fwd", "th_build_floor", "th_pool_create", "th_pool_alloc",
                 "th_pool_free", "th_pool_destroy", "th_graph_capture", "th_graph_replay", "th_graph_retarget",
                 "th_time_launch", "th_device_rates", "th_launch_repoint"):
        assert name in used, name


# ---- struct mirrors ----------------------------------------------------------------------

JL_SIZES = {"Int32": 4, "UInt32": 4, "Cint": 4, "Float32": 4, "Int64": 8, "UInt64": 8, "Cdouble": 8, "Float64": 8}
MIRRORS = {"Rates": "th_rates", "CWork": "th_work", "GemmDesc": "th_gemm_desc", "AttentionDesc": "th_attention_desc",
           "DeltaNetDesc": "th_deltanet_desc", "FloorValue": "th_floor_value", "CPart": "th_part",
           "CAffine": "th_affine", "CTerm": "th_term", "CFold": "th_fold", "COutput": "th_output",
           "FloorDesc": "th_floor_desc"}


def _jl_structs() -> dict[str, list[tuple[str, str]]]:
    out = {}
    for m in re.finditer(r"^struct (\w+)(.*?)\bend\b", JL, flags=re.S | re.M):
        body = m.group(2)
        fields = []
        for part in re.split(r"[;\n]", body):
            part = part.strip()
            f = re.match(r"(\w+)::(.+)$", part)
            if f:
                fields.append((f.group(1), f.group(2).strip()))
        out[m.group(1)] = fields
    return out


def _layout(structs, name) -> tuple[int, int, dict[str, int]]:
    """(size, alignment, field offsets) of a Julia isbits struct: C's rules."""
    off, align, offsets = 0, 1, {}
    for field, t in structs[name]:
        s, a = _type_size(structs, t)
        off = (off + a - 1) // a * a
        offsets[field] = off
        off += s
        align = max(align, a)
    return (off + align - 1) // align * align, align, offsets


def _type_size(structs, t: str) -> tuple[int, int]:
    if t in JL_SIZES:
        return JL_SIZES[t], JL_SIZES[t]
    if t.startswith("Ptr{"):
        return 8, 8
    m = re.match(r"NTuple\{(\d+),\s*(.+)\}$", t)
    if m:
        s, a = _type_size(structs, m.group(2))
        return int(m.group(1)) * s, a
    if t in structs:
        s, a, _ = _layout(structs, t)
        return s, a
    raise AssertionError(f"unknown field type {t}")


def test_struct_mirrors_match_gcc_layout(tmp_path):
    structs = _jl_structs()
    missing = [s for s in MIRRORS if s not in structs]
    assert not missing, missing
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{ROOT}/include/tempest_hip.h"', "int main(void) {"]
    for jl, c in MIRRORS.items():
        lines.append(f'  printf("{jl} %zu\\n", sizeof({c}));')
        for field, _ in structs[jl]:
            lines.append(f'  printf("{jl}.{field} %zu\\n", offsetof({c}, {field}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    # A field the C struct lacks fails here, at compile time.
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines() if l)
    for jl in MIRRORS:
        size, _, offsets = _layout(structs, jl)
        assert int(got[jl]) == size, (jl, size, got[jl])
        for field, off in offsets.items():
            assert int(got[f"{jl}.{field}"]) == off, (jl, field, off, got[f"{jl}.{field}"])


def test_struct_mirrors_cover_every_c_field():
    """A mirror names every member of its C struct, in order."""
    structs = _jl_structs()
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    for jl, c in MIRRORS.items():
        m = re.search(r"typedef struct " + c + r" \{(.*?)\} " + c + ";", text, flags=re.S)
        assert m, c
        c_fields = []
        for decl in m.group(1).split(";"):
            decl = " ".join(decl.split())
            if not decl:
                continue
            names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
            for n in names.split(","):
                c_fields.append(re.sub(r"[\s*]|\[.*\]", "", n))
        assert [f for f, _ in structs[jl]] == c_fields, (jl, c_fields)


# ---- the floor's group kinds -------------------------------------------------------------

def test_floor_kinds_are_dispatched_by_name():
    """Pointwise, reduction, scan and recurrence groups map to their kinds;
    anything else (a crossing) throws instead of building a wrong kernel."""
    m = re.search(r"function floor_kind\(kind\)(.*?)\nend", JL, flags=re.S)
    assert m
    body = m.group(1)
    for kind, code in (("PointwiseKind", "GROUP_POINTWISE"), ("ReductionKind", "GROUP_REDUCTION"),
                       ("ScanKind", "GROUP_SCAN"), ("RecurrenceKind", "GROUP_RECURRENCE")):
        assert f"kind isa C_.{kind} && return {code}" in body
    assert "throw(ArgumentError" in body.strip().splitlines()[-1]
    header_codes = re.search(r"enum \{ TH_GROUP_POINTWISE = 0, TH_GROUP_REDUCTION = 1, TH_GROUP_SCAN = 2, "
                             r"TH_GROUP_RECURRENCE = 3 \};", HEADER)
    assert header_codes and "Int32(0), Int32(1), Int32(2), Int32(3)" in JL


@pytest.mark.parametrize("fn,code", [("exp", 8), ("tanh", 10), ("inv", 31), ("ifelse", 24)])
def test_floor_function_codes_match_the_header(fn, code):
    """FLOOR_FN's numbers are the header's TH_FN_* order."""
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    enum = re.search(r"enum \{\s*(TH_FN_ADD = 0.*?)TH_FN_COUNT", text, flags=re.S).group(1)
    names = [n.strip().split("=")[0].strip() for n in enum.split(",") if n.strip()]
    assert names.index("TH_FN_" + fn.upper()) == code
    assert re.search(rf"\b{fn} => {code}\b", JL)
