"""The floor's code-object store on the CPU (hiprtc needs no device): keyed
by the generated source, which names the toolchain; bounded, removing the
entries used least recently; off at capacity 0 (the store of
src/Compiler/runtime/cache.jl:1-60, bounded as :43-45)."""
import ctypes
import re
import time

import pytest

from tempest_hip import _lib
from tempest_hip.floor import FloorGroup


def _group(c: float) -> FloorGroup:
    """A small pointwise group whose source differs with `c`."""
    g = FloorGroup("pointwise", (64,))
    g.value("x", "f32", 64)
    g.value("y", "f32", 64)
    g.output("y", g.apply("exp", g.load("x", [1]) * c), [1])
    return g


def _counts() -> tuple[int, int]:
    loaded, compiled = ctypes.c_int64(), ctypes.c_int64()
    _lib.call("th_floor_cache_counts", ctypes.byref(loaded), ctypes.byref(compiled))
    return loaded.value, compiled.value


def _entries(d):
    return sorted(p.name for p in d.glob("floor-*.hsaco"))


@pytest.fixture
def store(tmp_path, monkeypatch):
    monkeypatch.setenv("TEMPEST_HIP_CACHE", str(tmp_path))
    monkeypatch.delenv("TEMPEST_HIP_CACHE_CAPACITY", raising=False)
    return tmp_path


def test_the_source_names_the_toolchain():
    head = _group(1.0).source().splitlines()[1]
    assert re.fullmatch(r"// toolchain: hiprtc \d+\.\d+, HIP runtime \d+, store schema \d+", head), head


def test_a_second_compile_loads(store):
    g = _group(1.5)
    l0, c0 = _counts()
    g.compile()
    assert _counts() == (l0, c0 + 1)
    names = _entries(store)
    assert len(names) == 1
    key = re.search(r"th_floor_([0-9a-f]{16})_0", g.source()).group(1)
    assert names == [f"floor-{key}.hsaco"]  # named by the key the kernels carry
    g.compile()
    assert _counts() == (l0 + 1, c0 + 1)


def test_capacity_zero_keeps_nothing(store, monkeypatch):
    monkeypatch.setenv("TEMPEST_HIP_CACHE_CAPACITY", "0")
    l0, c0 = _counts()
    g = _group(2.5)
    g.compile()
    g.compile()
    assert _counts() == (l0, c0 + 2)
    assert _entries(store) == []


def test_the_store_removes_what_was_used_least_recently(store, monkeypatch):
    groups = {"a": _group(3.0), "b": _group(4.0), "c": _group(5.0)}
    sizes = {}
    for k, g in groups.items():
        before = set(_entries(store))
        g.compile()
        (new,) = set(_entries(store)) - before
        sizes[k] = (store / new).stat().st_size
    for p in store.glob("floor-*.hsaco"):
        p.unlink()
    # Room for a and b, or a and c, not all three.
    cap = max(sizes["a"] + sizes["b"], sizes["a"] + sizes["c"])
    assert cap < sum(sizes.values())
    monkeypatch.setenv("TEMPEST_HIP_CACHE_CAPACITY", str(cap))
    name = {}
    for k in "ab":
        before = set(_entries(store))
        groups[k].compile()
        (name[k],) = set(_entries(store)) - before
        time.sleep(0.02)
    l0, _ = _counts()
    groups["a"].compile()  # a load: a is now used more recently than b
    assert _counts()[0] == l0 + 1
    time.sleep(0.02)
    groups["c"].compile()
    left = set(_entries(store))
    assert name["a"] in left and name["b"] not in left and len(left) == 2
    assert sum((store / n).stat().st_size for n in left) <= cap


def test_capacity_takes_a_suffix(store, monkeypatch):
    monkeypatch.setenv("TEMPEST_HIP_CACHE_CAPACITY", "1K")
    g = _group(6.0)
    g.compile()  # larger than 1 KiB: the entry just written stays, alone
    assert len(_entries(store)) == 1
    _group(7.0).compile()
    assert len(_entries(store)) == 1


def test_concurrent_builds_share_the_store(store):
    """Claims and builds run side by side on threads (runtime.jl:649-680): the
    generator and the store are safe to call from several threads at once;
    each distinct group is compiled once per key and every thread sees the
    same source."""
    from concurrent.futures import ThreadPoolExecutor
    groups = [_group(10.0 + (i % 4)) for i in range(16)]
    l0, c0 = _counts()

    def work(g):
        src = g.source()
        g.compile()
        return src

    with ThreadPoolExecutor(max_workers=8) as ex:
        sources = list(ex.map(work, groups))
    for i, src in enumerate(sources):
        assert src == sources[i % 4]
    assert len(_entries(store)) == 4
    loaded, compiled = _counts()
    assert compiled - c0 == 4 and loaded - l0 == 12
