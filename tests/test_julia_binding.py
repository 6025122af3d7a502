"""The Julia extension (tempest.jl_amd/julia/HIPExt.jl) against the C ABI and
against Tempest's runtime, on the CPU: no Julia runs here, so the binding is
checked as text.  Every `ccall((:th_..., LIB), R, (T...), ...)` names an entry
point the header declares, with the header's argument count and C types;
every struct mirror has the field names, offsets and size gcc gives the
header's struct; the group kinds the floor refuses throw rather than build a
wrong kernel.  Read through a model of Julia's dispatch (tests/julia_sig.py),
every method the binding adds to one of Tempest's functions is neither
ambiguous with nor hidden by the reference's methods of it; the Target
protocol functions CUDATarget specialises are defined for HIPTarget or left to
a default named here with the reason; the calls the runtime makes on a slot's
storage, a `Copy` step and a result reach the binding's methods; a capture
records every kind of step and a retarget patches the moved steps by position.
Each of those checks is shown to catch a defect planted in a copy of the text."""
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


# ---- dispatch: the binding's methods against the reference's -----------------------------
#
# The binding extends the reference's functions; in Julia a method that is
# ambiguous with, or less specific than, a method of the reference never runs
# (a MethodError, or the reference's method instead).  These checks read both
# as text through tests/julia_sig.py's model of Julia's dispatch.

import julia_sig as js  # noqa: E402

REF = pathlib.Path("/root/reference")
needs_ref = pytest.mark.skipif(not (REF / "src").is_dir(), reason="the reference's sources are not on this machine")


def _ref_texts() -> dict[str, str]:
    if not hasattr(_ref_texts, "cache"):
        _ref_texts.cache = {str(p.relative_to(REF)): p.read_text() for p in js.julia_files(REF / "src")}
    return _ref_texts.cache


def _imported(text: str) -> set[str]:
    """The functions the binding extends: those it imports from Tempest."""
    names = set()
    for m in re.finditer(r"^import\s+Tempest\.Compiler(?:\.Implement)?:\s*(.*?)(?=\n\S)", text, flags=re.S | re.M):
        names |= {x.strip() for x in m.group(1).replace("\n", " ").split(",") if x.strip()}
    return names


def _types(text: str) -> js.Types:
    return js.load_types(text, *_ref_texts().values(), (REF / "ext" / "CUDAExt.jl").read_text())


def ambiguity_problems(text: str) -> list[str]:
    """Every method the binding adds to a reference function, against every
    reference method of it: no ambiguity, not hidden; and the binding's own
    methods of one function (its Base extensions too) pairwise."""
    types = _types(text)
    ours = js.methods(text, "HIPExt.jl")
    theirs = [m for f, t in _ref_texts().items() for m in js.methods(t, f)]
    extended = _imported(text)
    problems = []
    for o in ours:
        if o.name not in extended:
            continue
        for t in theirs:
            if t.name == o.name and (why := js.conflict(types, o, t)):
                problems.append(f"{o.where()}\n  vs {t.where()}\n  {why}")
    by_name: dict[str, list] = {}
    for o in ours:
        if o.name in extended or o.qualified.startswith("Base."):
            by_name.setdefault(o.qualified, []).append(o)
    for ms in by_name.values():
        for i, a in enumerate(ms):
            for b in ms[i + 1:]:
                if js.intersect(types, a, b) and not (js.more_specific(types, a, b) or js.more_specific(types, b, a)):
                    problems.append(f"{a.where()}\n  vs {b.where()}\n  ambiguous with each other")
    return problems


@needs_ref
def test_methods_extending_tempest_are_unambiguous():
    problems = ambiguity_problems(JL)
    assert not problems, "\n".join(problems)


# ---- the Target protocol: what CUDATarget specialises, HIPTarget defines or relies on ---

# Functions of the protocol that HIPTarget leaves to the reference's default,
# each with why the default is right for one MI355X driven by one stream.
DEFAULTS = {
    "taken": "HIP buffers are the library's own: no package orders their uses by stream, as CUDA.jl does "
             "CuArrays' (ext/CUDAExt.jl:50-68)",
    "stream": "one device, one stream: the default pair (device, device) names it",
    "event": "one stream: steps run in the order they are launched, so nothing waits for an event",
    "record!": "one stream: no event is recorded",
    "wait!": "one stream: no event is waited for",
    "on_stream": "one stream on one device: the default enters the device (on_device)",
    "lane": "plans_across_devices is false (its default): no crossings, no lanes",
    "link": "plans_across_devices is false: no crossings leave the device",
    "task_state": "the library's device and stream are the process's (th_init): a new task finds them as they are",
    "floor_split": "the cover's estimate of the floor splits nothing; the library's floor chooses its split itself",
    "merge_lanes": "called only by generated Julia kernels, which this target does not compile (build_floor is its own)",
    "accumulate!": "called only by generated Julia kernels, which this target does not compile (build_floor is its own)",
    "at_home": "one device: the target is at home on it",
    "plans_across_devices": "one device: false, the default",
}
# Functions with no default that HIPTarget never reaches, and why.
UNREACHED = {
    "crossing": "plans_across_devices(::HIPTarget) is false: no value crosses devices",
    "time_crossing": "plans_across_devices(::HIPTarget) is false: no crossing is timed",
    "floor_launch": "build_floor(::HIPTarget, ::Plan, ::Group, buffers) replaces the generic floor that calls it",
}


def _cuda_specialised() -> set[str]:
    """Functions of Tempest.Compiler that the CUDA target specialises: methods
    typed with CUDATarget in the reference's sources, and every method
    ext/CUDAExt.jl adds to a Tempest.Compiler function."""
    names = set()
    for f, t in _ref_texts().items():
        for m in js.methods(t, f):
            if "CUDATarget" in m.text.split("=")[0] and m.name not in ("CUDATarget", "show"):
                names.add(m.name)
    for m in js.methods((REF / "ext" / "CUDAExt.jl").read_text(), "ext/CUDAExt.jl"):
        if m.qualified.startswith("Tempest.Compiler."):
            names.add(m.name)
    return names


def protocol_problems(text: str) -> list[str]:
    types = _types(text)
    ours = js.methods(text, "HIPExt.jl")
    theirs = [m for f, t in _ref_texts().items() for m in js.methods(t, f)]
    extended = _imported(text)
    problems = []
    for name in sorted(_cuda_specialised()):
        if name in ("repoint!", "repoints"):  # launch types, checked with the libraries below
            continue
        mine = [m for m in ours if m.name == name and any(
            isinstance(a, js.Name) and a.name in ("HIPTarget", "HIPDense", "HIPBuffer") for a in map(types.resolve, m.args))
            or (m.name == name and any("HIP" in repr(types.resolve(a)) for a in m.args))]
        if mine:
            if name not in extended:
                problems.append(f"{name}: defined for HIPTarget but not imported from Tempest (a new function, not a method of Tempest's)")
            continue
        if name in DEFAULTS:
            # The default must apply with a HIPTarget where CUDA's takes its target.
            generic = [m for m in theirs if m.name == name and not any(
                isinstance(a, js.Name) and a.name in ("CPUTarget", "CUDATarget") for a in m.args)
                and not any(isinstance(a, js.Union_) for a in m.args)]
            if not generic:
                problems.append(f"{name}: relied on as a default, but the reference has no generic method")
            continue
        if name in UNREACHED:
            continue
        problems.append(f"{name}: CUDATarget specialises it; HIPTarget neither defines it nor records the default relied on")
    return problems


@needs_ref
def test_target_protocol_covers_what_cuda_specialises():
    problems = protocol_problems(JL)
    assert not problems, "\n".join(problems)


@needs_ref
def test_relied_defaults_hold():
    """What the relied-on defaults assume: the target does not plan across
    devices, and the floor is this target's own."""
    ours = js.methods(JL, "HIPExt.jl")
    assert not any(m.name == "plans_across_devices" for m in ours)
    assert re.search(r"^plans_across_devices\(::Target\) = false$", _ref_texts()["src/Compiler/runtime/target.jl"], re.M)
    floor = [m for m in ours if m.name == "build_floor"]
    assert floor and all(isinstance(a, js.Name) for a in floor[0].args[:3])
    assert [a.name for a in floor[0].args[:3]] == ["HIPTarget", "Plan", "Group"]


# ---- the Implement interface: what the reference's own libraries define ------------------

LIBRARIES = ("HIPProducts", "HIPEpilogues", "HIPAttention", "HIPRows", "HIPDeltaNet")
LIBRARY_DEFAULTS = {
    ("resources", "*"): "launches take their workspaces from the target's pool (HIPLaunch), not per executable",
    ("in_place", "HIPEpilogues"): "writes no output over an input",
    ("in_place", "HIPAttention"): "writes no output over an input",
    ("in_place", "HIPRows"): "writes no output over an input",
    ("in_place", "HIPDeltaNet"): "writes no output over an input",
    ("estimate", "HIPRows"): "memory-bound: the default prices the group's bytes (Implement.jl:127)",
    ("estimate", "HIPAttention"): None,
}


def _reference_library_functions() -> set[str]:
    """The Implement functions the reference's own libraries specialise:
    those cuBLASExt and cuDNNExt import to extend, and package_of
    (Implement/packages.jl:42-44)."""
    names = {"package_of"}
    for f in ("ext/cuBLASExt.jl", "ext/cuDNNExt.jl"):
        t = (REF / f).read_text()
        m = re.search(r"^import Tempest\.Compiler\.Implement:\s*(.*)$", t, flags=re.M)
        names |= {x.strip() for x in m.group(1).split(",")}
    return names


def library_problems(text: str) -> list[str]:
    types = _types(text)
    ours = js.methods(text, "HIPExt.jl")
    problems = []
    for name in sorted(_reference_library_functions() - {"repoints", "repoint!"}):
        for lib in LIBRARIES:
            call0 = js.Name("Type", (js.Name(lib),)) if name == "loaded" else js.Name(lib)
            have = [m for m in ours if m.name == name and m.args and types.sub(call0, m.args[0], {})]
            if have:
                continue
            if (name, lib) in LIBRARY_DEFAULTS or (name, "*") in LIBRARY_DEFAULTS:
                continue
            problems.append(f"{name}: the reference's libraries define it; {lib} neither does nor records the default relied on")
    # Launches: every run the binding builds repoints, by program value, onto any storage.
    for launch in ("HIPLaunch", "HIPFloorRun"):
        for name, call in (("repoints", [js.Name(launch)]),
                           ("repoint!", [js.Name(launch), js.Name("Int64"), SLOT])):
            if not any(m.name == name and js.applies(types, m, call) for m in ours):
                problems.append(f"{name}({launch}, ...): no method takes a slot's storage")
    return problems


@needs_ref
def test_libraries_cover_the_implement_interface():
    problems = library_problems(JL)
    assert not problems, "\n".join(problems)


# ---- storage: the calls Tempest's runtime makes on what `allocate` returns ---------------

U8, F32, I64 = js.Name("UInt8"), js.Name("Float32"), js.Name("Int64")


def _buf(t):
    return js.Name("HIPBuffer", (t,))


# A slot's value: reinterpret(T, view(slot, 1:n*sizeof(T))) (runtime.jl:605).
SUB = js.Name("SubArray", (U8, js.Lit("1"), _buf(U8), js.Name("Tuple", (js.Name("UnitRange", (I64,)),)), js.Lit("true")))
SLOT = js.Name("ReinterpretArray", (F32, js.Lit("1"), U8, SUB, js.Lit("false")))
# A result: reshape(storage, dims) (runtime.jl:524), a matrix or a number.
RESULT2 = js.Name("ReshapedArray", (F32, js.Lit("2"), SLOT, js.Name("Tuple")))
RESULT0 = js.Name("ReshapedArray", (F32, js.Lit("0"), _buf(F32), js.Name("Tuple")))

# (function, argument types, the reference's call it stands for)
STORAGE_CALLS = [
    ("pointer", [SLOT], "Base.pointer(s::Strided) = pointer(s.buffer)"),
    ("pointer", [_buf(F32)], "Base.pointer(s::Strided) = pointer(s.buffer)"),
    ("pointer", [RESULT2], "address_of(x) = x isa StridedArray ? reinterpret(UInt, pointer(x))"),
    ("copyto!", [SLOT, I64, SLOT, I64, I64], "(c::Copy)() = (copyto!(c.to, 1, c.from, c.offset + 1, length(c.to)); nothing)"),
    ("copyto!", [_buf(F32), I64, SLOT, I64, I64], "(c::Copy)() = (copyto!(c.to, 1, c.from, c.offset + 1, length(c.to)); nothing)"),
    ("copyto!", [js.Name("Array", (F32, js.Lit("0"))), RESULT0], "on_each_device(i -> scalar[ks[i]] && (arrays[i] = Array(ex.results[ks[i]])[])"),
    ("copyto!", [RESULT2, RESULT2], "arrays[i] = copy(ex.results[ks[i]])"),
    ("similar", [_buf(F32), js.Name("Type", (F32,)), js.Name("Tuple", (I64, I64))], "arrays[i] = copy(ex.results[ks[i]])"),
    ("upload!", [js.Name("HIPTarget"), _buf(F32), js.Name("Array", (F32, js.Lit("1")))], "upload!(ex.target, own, vec(x))"),
    ("download!", [js.Name("HIPTarget"), js.Name("Array", (F32, js.Lit("1"))), SLOT],
     "download!(ex.target, vec(x), ex.arguments[a])"),
    ("size", [_buf(U8)], "reinterpret(T, view(slot, 1:(n * sizeof(T))))"),
    ("getindex", [_buf(F32), I64], "Array(ex.results[ks[i]])[]"),
]


def storage_problems(text: str) -> list[str]:
    types = js.load_types(text)
    ours = js.methods(text, "HIPExt.jl")
    problems = []
    if not types.sub(_buf(U8), js.Name("DenseArray", (U8, js.Lit("1")))):
        problems.append("HIPBuffer is not a dense vector: view, reinterpret and pointer of a slot's value do not apply")
    for name, call, site in STORAGE_CALLS:
        if not any(m.name == name and js.applies(types, m, call) for m in ours):
            problems.append(f"{name}({', '.join(map(js.show, call))}) reaches no method of the binding; the runtime calls it: {site}")
    return problems


def test_runtime_calls_on_slot_storage_reach_the_binding():
    problems = storage_problems(JL)
    assert not problems, "\n".join(problems)


@needs_ref
def test_storage_calls_are_the_reference_s():
    """The calls above are the reference's own, where it makes them."""
    text = "\n".join(_ref_texts().values())
    for _, _, site in STORAGE_CALLS:
        assert site in text, site


# ---- graphs: what a captured run holds, and how it is retargeted -------------------------

def capture_problems(text: str) -> list[str]:
    """capture records every kind of run a step holds (launches, the floor's
    runs, the runtime's Copy steps, runtime.jl:47-64,502-504) or replays the
    runs themselves; retarget! takes the moved steps as positions
    (runtime.jl:1127) and patches exactly their launches."""
    types = js.load_types(text)
    ours = js.methods(text, "HIPExt.jl")
    problems = []
    cap = [m for m in ours if m.name == "capture"]
    if not cap or "recorded" not in cap[0].text + text[text.find(cap[0].text):text.find(cap[0].text) + 900]:
        problems.append("capture does not map the steps' runs through `recorded`")
    for run in ("HIPLaunch", "HIPFloorRun", "Copy"):
        # A method of its own: the fallback would leave the whole run unrecorded.
        if not any(m.name == "recorded" and m.args and m.args[0] != js.ANY and js.applies(types, m, [js.Name(run)])
                   for m in ours):
            problems.append(f"capture cannot record a step whose run is a {run}")
    if not any(m.name == "recorded" and js.applies(types, m, [js.Name("Stepped")]) for m in ours):
        problems.append("capture has no fallback for runs it cannot record")
    ret = [m for m in ours if m.name == "retarget!" and m.args[1:2] and isinstance(m.args[1], js.Name)
           and m.args[1].name == "HIPGraph"]
    if not ret:
        problems.append("no retarget! for a HIPGraph")
    else:
        start = text.find(ret[0].text)
        body = text[start:text.find("\nend", start)]
        if re.search(r"\b(s|step)\.step\b", body) or ".step.run" in body:
            problems.append("retarget! reads the moved steps as Scheduled steps; the runtime passes their positions")
        if "g.first[" not in body:
            problems.append("retarget! does not patch the moved steps' own launches")
    return problems


def test_capture_records_every_run_and_retargets_by_position():
    problems = capture_problems(JL)
    assert not problems, "\n".join(problems)


@needs_ref
def test_retarget_positions_are_the_reference_s():
    runtime = _ref_texts()["src/Compiler/runtime/runtime.jl"]
    assert "retarget!(ex.target, segment.graph, [last(r.at[j]) for j in at], [m[3] for m in mine], repoint)" in runtime
    assert "copies = Copy[Copy(buffers[a], buffers[r], a => r) for (r, a) in s.staged]" in runtime


# ---- each check catches the defect it is for --------------------------------------------
#
# A defect planted in a copy of the binding's text (never in the file) must
# fail the check written for it.

def _plant(old: str, new: str) -> str:
    assert old in JL, old
    return JL.replace(old, new, 1)


@needs_ref
def test_checks_catch_planted_defects():
    # An untyped plan and group: ambiguous with runtime.jl:1323.
    planted = _plant("function build_floor(target::HIPTarget, p::C.Plan, g::C.Group, buffers)",
                     "function build_floor(target::HIPTarget, p, g, buffers)")
    assert any("build_floor" in p and "ambiguous" in p for p in ambiguity_problems(planted))
    # No implementations(::HIPTarget): the cover would offer no group to any library.
    planted = _plant("implementations(t::HIPTarget) = t.implementations\n", "")
    assert any(p.startswith("implementations:") for p in protocol_problems(planted))
    # A buffer that is not an array: slot_view, pointer and copyto! fail.
    planted = _plant("mutable struct HIPBuffer{T} <: DenseVector{T}", "mutable struct HIPBuffer{T}")
    assert any("dense vector" in p for p in storage_problems(planted))
    planted = _plant("function repoint!(l::HIPLaunch, value, buffer)", "function repoint!(l::HIPLaunch, value, buffer::HIPBuffer)")
    assert any("repoint!(HIPLaunch" in p for p in library_problems(planted))
    # A capture that knows launches alone: Copy steps unrecorded.
    planted = _plant("recorded(run::C.Copy) =", "recorded_copy(run::C.Copy) =")
    assert any("Copy" in p for p in capture_problems(planted))
    # retarget! reading its steps as Scheduled steps.
    planted = _plant("        run = g.runs[s]\n", "        run = s.step.run\n")
    assert any("positions" in p for p in capture_problems(planted))
    # No package_of: the rates file's `HIP` lines would be looked up as `HIPExt`.
    planted = _plant("package_of(::HIPLibrary) = :HIP\n", "")
    assert any(p.startswith("package_of:") for p in library_problems(planted))


def test_gemm_flags_match_the_header():
    """The product flags the binding sets are the header's TH_GEMM_* values,
    and HIPTarget's precision reaches the descriptor (bf16x3 for Float32
    factors with a Float32 result only)."""
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    want = {n: int(v) for n, v in re.findall(r"#define TH_GEMM_(\w+) (\d+)", text)}
    got = re.search(r"const GEMM_F32_FACTORS, GEMM_F16_FACTORS, GEMM_ACCUMULATE, GEMM_BF16X3 = "
                    r"Int32\((\d+)\), Int32\((\d+)\), Int32\((\d+)\), Int32\((\d+)\)", JL)
    assert got, "GEMM flag constants"
    assert [int(x) for x in got.groups()] == [want["F32_FACTORS"], want["F16_FACTORS"], want["ACCUMULATE"],
                                               want["BF16X3"]]
    assert "x3 = precision === :bf16x3 && T === Float32 && R === Float32 ? GEMM_BF16X3 : Int32(0)" in JL
    assert JL.count("gemm_desc(b; precision = t.precision)") == 2
    assert "precision in (:full, :bf16x3) ||" in JL
