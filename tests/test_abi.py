"""The C ABI on the CPU: the library loads, exports every entry point the
header declares, the ctypes table matches the header, and the host logic
(slot planning) behaves as the reference's planner."""
import ctypes
import pathlib
import re

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _declared() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:int|const char\*)\s+(th_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert "th_init" in names and "th_graph_capture" in names and len(names) > 20


def test_library_exports_every_declared_symbol():
    import tempest_hip._lib as L
    lib = L.load()
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    import tempest_hip._lib as L
    declared = _declared() - {"th_last_error"}
    assert declared == set(L.SIGNATURES), (declared ^ set(L.SIGNATURES))


def test_entry_points_refuse_before_init():
    # No GPU is touched: th_init was never called, so every call that needs a
    # device reports TH_E_STATE with a message.
    import tempest_hip._lib as L
    lib = L.load()
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible; the state check runs on the CPU only")
    out = ctypes.c_void_p()
    assert lib.th_alloc(16, ctypes.byref(out)) == -2
    assert b"th_init" in lib.th_last_error()
    assert lib.th_launch_run(None) == -2


def test_slot_planner_reuses_free_slots():
    from tempest_hip.runtime import Group, Program, Value, storage
    f32 = torch.float32
    vals = {n: Value(n, f32, (s,), "stored") for n, s in [("a", 100), ("b", 50), ("c", 80), ("d", 200)]}
    vals["x"] = Value("x", f32, (10,), "input")
    noop = lambda a: None  # noqa: E731
    groups = [
        Group("k0", (), ("x",), ("a",), noop),       # a lives 0..1
        Group("k1", (), ("a",), ("b",), noop),       # b lives 1..2
        Group("k2", (), ("b",), ("c",), noop),       # c lives 2..3: a's slot is free (smallest that fits)
        Group("k3", (), ("c",), ("d",), noop),       # d: b's slot is free, grown to fit (the largest free)
    ]
    s = storage(Program("p", vals, groups, ["x"], []))
    assert s.slots["a"] == 0 and s.slots["b"] == 1
    assert s.slots["c"] == 0  # a (400 bytes) is free at k2 and fits c (320)
    assert s.slots["d"] == 1 and s.sizes[1] == 800  # b's slot grown
    assert len(s.sizes) == 2
    # Lifetimes never overlap within a slot.
    by_slot = {}
    for v, sl in s.slots.items():
        by_slot.setdefault(sl, []).append(s.lifetimes[v])
    for spans in by_slot.values():
        spans.sort()
        for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
            assert a1 < b0


def test_floor_structures_match_the_header(tmp_path):
    """sizeof and member offsets of the generated floor's structures, as gcc
    lays out include/tempest_hip.h, against the ctypes mirror."""
    import subprocess
    import tempest_hip._lib as L
    members = {"th_part": (L.Part, ["kind", "divisor", "coeff", "constant", "inner"]),
               "th_affine": (L.Affine, ["constant", "coeff", "gather", "gather_coeff", "part"]),
               "th_floor_value": (L.FloorValue, ["dtype", "length", "ptr"]),
               "th_term": (L.TermStruct, ["op", "fn", "args", "ref", "observe", "lit", "index"]),
               "th_fold": (L.FoldStruct, ["kind", "phase", "body", "weight", "scan"]),
               "th_output": (L.OutputStruct, ["value", "term", "full", "accumulate", "index"]),
               "th_floor_desc": (L.FloorDesc, ["kind", "rank", "extents", "reduced", "n_values", "n_terms",
                                               "n_folds", "n_outputs", "flags", "values", "terms", "folds",
                                               "outputs"])}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{ROOT}/include/tempest_hip.h"', 'int main(void) {']
    for s, (_, ms) in members.items():
        lines.append(f'  printf("{s} %zu\\n", sizeof({s}));')
        for m in ms:
            lines.append(f'  printf("{s}.{m} %zu\\n", offsetof({s}, {m}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n") if l)
    for s, (cls, ms) in members.items():
        assert int(got[s]) == ctypes.sizeof(cls), s
        for m in ms:
            assert int(got[f"{s}.{m}"]) == getattr(cls, m).offset, (s, m)
