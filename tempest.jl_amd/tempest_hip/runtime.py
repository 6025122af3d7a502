"""The executable: slots, binding and pointing, execute!/capture!/replay!.

Mirrors src/Compiler/runtime/runtime.jl and runtime/compile.jl for programs
whose plan is given (the front end that traces and plans them is Julia's and
stays there; ``programs.py`` states each plan it would form):

- ``storage``     the slot pool of plan/storage.jl:236-319 for one stream:
                  values take, in kernel order, the smallest free slot that
                  fits, else the largest free slot grown, else a new one.
- ``prepare``     runtime.jl:194-200, 337-539: slots in one arena
                  (th_arena_create), own buffers for results, one launch per
                  group built on the values' addresses.
- ``bind`` / ``point``  runtime.jl:719-830: copy inputs into own buffers, or
                  take the caller's arrays as storage by reference and
                  repoint the launches that read them where they moved.
- ``execute``, ``capture``, ``replay``  runtime.jl:1158-1214.
- ``compile`` / ``Compiled``  compile.jl:48-62, 310-349: signature check,
                  point, replay, and results returned as copies (numbers
                  read to the host).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Callable, Sequence

import torch

from ._lib import call
from .launch import Launch
from .target import Direct, Graph, HIPTarget, Move

_ELEMENT = {torch.float32: 4, torch.bfloat16: 2, torch.float16: 2, torch.float64: 8, torch.int32: 4,
            torch.int64: 8, torch.uint8: 1}


@dataclass
class Value:
    """A value of a plan: its element type, its Julia dimensions (column-major,
    first fastest) and its role: an ``input``, a ``result`` (own buffer,
    returned) or ``stored`` (kept between kernels, in a slot)."""

    name: str
    dtype: torch.dtype
    dims: tuple
    role: str

    @property
    def count(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    @property
    def nbytes(self) -> int:
        return self.count * _ELEMENT[self.dtype]

    @property
    def scalar(self) -> bool:
        return self.dims == ()


@dataclass
class Group:
    """A kernel of the plan: the claim that runs it builds one launch from the
    addresses of the values it names, in its launch's value order."""

    name: str
    values: tuple[str, ...]
    reads: tuple[str, ...]
    writes: tuple[str, ...]
    build: Callable[[dict[str, int]], Launch]


@dataclass
class Program:
    name: str
    values: dict[str, Value]
    groups: list[Group]
    inputs: list[str]
    outputs: list[str]


@dataclass
class Storage:
    """plan/storage.jl:37-46: lifetimes (first and last kernel), slots, sizes."""

    lifetimes: dict[str, tuple[int, int]]
    slots: dict[str, int]
    sizes: list[int]


def storage(program: Program) -> Storage:
    """Slots for the stored values, one stream (plan/storage.jl:64-80, 236-319)."""
    first: dict[str, int] = {}
    last: dict[str, int] = {}
    for k, g in enumerate(program.groups):
        for v in g.writes:
            first.setdefault(v, k)
            last[v] = max(last.get(v, k), k)
        for v in g.reads:
            first.setdefault(v, k)
            last[v] = max(last.get(v, k), k)
    stored = [v for v in program.values.values() if v.role == "stored"]
    sizes: list[int] = []
    until: list[int] = []  # per slot: the last kernel using what it holds
    slots: dict[str, int] = {}
    for v in sorted(stored, key=lambda v: (first.get(v.name, 0), v.name)):
        k = first.get(v.name, 0)
        free = [s for s in range(len(sizes)) if until[s] < k]
        fits = [s for s in free if sizes[s] >= v.nbytes]
        if fits:
            s = min(fits, key=lambda s: (sizes[s], s))
        elif free:
            s = max(free, key=lambda s: (sizes[s], -s))
        else:
            sizes.append(0)
            until.append(-1)
            s = len(sizes) - 1
        sizes[s] = max(sizes[s], v.nbytes)
        until[s] = last.get(v.name, k)
        slots[v.name] = s
    return Storage({v: (first[v], last[v]) for v in first}, slots, sizes)


class Arena:
    """The slots in one device slab (th_arena_create)."""

    def __init__(self, sizes: Sequence[int], align: int = 256):
        arr = (ctypes.c_uint64 * max(1, len(sizes)))(*sizes)
        self._h = ctypes.c_void_p()
        call("th_arena_create", arr, len(sizes), align, ctypes.byref(self._h))
        self.addresses = []
        for i in range(len(sizes)):
            p = ctypes.c_void_p()
            call("th_arena_slot", self._h, i, ctypes.byref(p))
            self.addresses.append(p.value)
        b = ctypes.c_uint64()
        call("th_arena_bytes", self._h, ctypes.byref(b))
        self.bytes = b.value

    def destroy(self) -> None:
        if self._h is not None:
            call("th_arena_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Pool:
    """A reserved range of device addresses that hands out blocks (th_pool_*):
    the slots of executables allocated one at a time, as ``planned`` allocates
    each (src/Compiler/runtime/runtime.jl:415), all inside one range."""

    def __init__(self, reserve: int = 64 << 30):
        self._h = ctypes.c_void_p()
        self._closed = False
        call("th_pool_create", ctypes.c_uint64(reserve), ctypes.byref(self._h))

    def alloc(self, nbytes: int, align: int = 256) -> int:
        p = ctypes.c_void_p()
        call("th_pool_alloc", self._h, ctypes.c_uint64(nbytes), ctypes.c_uint64(align), ctypes.byref(p))
        return p.value

    def free(self, ptr: int) -> None:
        call("th_pool_free", self._h, ctypes.c_void_p(ptr))

    def info(self) -> tuple[int, int, int]:
        """(base address, reserved bytes, mapped bytes)."""
        b, r, m = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint64()
        call("th_pool_info", self._h, ctypes.byref(b), ctypes.byref(r), ctypes.byref(m))
        return b.value, r.value, m.value

    def destroy(self) -> None:
        """Give the range back; blocks still taken keep it until the last of
        them is freed (th_pool_destroy), so the handle stays for their frees."""
        if not self._closed:
            self._closed = True
            call("th_pool_destroy", self._h)

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class PoolSlots:
    """The slots of one executable taken from a Pool one by one, freed with it."""

    def __init__(self, pool: Pool, sizes: Sequence[int], align: int = 256):
        self.pool = pool
        self.addresses = [pool.alloc(n, align) for n in sizes]
        self.bytes = sum(sizes)

    def destroy(self) -> None:
        for a in self.addresses:
            self.pool.free(a)
        self.addresses = []

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Executable:
    """A prepared program: its storage, launches and (once captured) graph.
    Its slots lie in one arena slab, or, given a Pool, are taken from the
    pool's reserved range one by one."""

    def __init__(self, program: Program, target: HIPTarget, inputs: Sequence[torch.Tensor], point: bool = True,
                 pool: Pool | None = None):
        self.program = program
        self.target = target
        self.storage = storage(program)
        self.arena = Arena(self.storage.sizes) if pool is None else PoolSlots(pool, self.storage.sizes)
        self.own: dict[str, torch.Tensor] = {}
        self.bound: dict[str, torch.Tensor] = {}
        self.addresses: dict[str, int] = {}
        # The results share one allocation, each at a 256-byte boundary, so a
        # call returns them with one copy and reads its numbers at once.
        self.result_at: dict[str, tuple[int, int]] = {}
        at = 0
        for name, v in program.values.items():
            if v.role == "result":
                nbytes = max(1, v.count) * _ELEMENT[v.dtype]
                self.result_at[name] = (at, nbytes)
                at += (nbytes + 255) // 256 * 256
        self.results = target.allocate(torch.uint8, max(at, 256))
        for name, v in program.values.items():
            if v.role == "stored":
                self.addresses[name] = self.arena.addresses[self.storage.slots[name]]
            elif v.role == "result":
                off, nbytes = self.result_at[name]
                t = self.results[off:off + nbytes].view(v.dtype)
                self.own[name] = t
                self.addresses[name] = t.data_ptr()
        self._check(inputs)
        for name, x in zip(program.inputs, inputs):
            self._take(name, x, point)
        self.launches = [g.build(dict(self.addresses)) for g in program.groups]
        self._place_workspaces(pool)
        self.graph: Graph | Direct | None = None
        self._moved: set[int] = set()

    def _place_workspaces(self, pool: Pool | None) -> None:
        """Give each launch's workspace (attention's dS', split sums, ...) a
        slot beside the program's: the slots and workspaces are laid out
        again in one arena (or taken from the pool), the launches repointed
        to it.  The first arena, built before the workspaces were known,
        goes."""
        self.workspaces = [l.workspace() for l in self.launches]
        if not any(self.workspaces):
            return
        sizes = list(self.storage.sizes) + [w for w in self.workspaces if w]
        arena = Arena(sizes) if pool is None else PoolSlots(pool, sizes)
        for name, v in self.program.values.items():
            if v.role == "stored":
                self.addresses[name] = arena.addresses[self.storage.slots[name]]
        for g, l in zip(self.program.groups, self.launches):
            for i, v in enumerate(g.values):
                if v in self.program.values and self.program.values[v].role == "stored":
                    l.repoint(i, self.addresses[v])
        j = len(self.storage.sizes)
        for l, w in zip(self.launches, self.workspaces):
            if w:
                l.set_workspace(arena.addresses[j])
                j += 1
        self.arena.destroy()
        self.arena = arena

    # -- binding -------------------------------------------------------------

    def _check(self, inputs: Sequence[torch.Tensor]) -> None:
        if len(inputs) != len(self.program.inputs):
            raise ValueError(f"{self.program.name} takes {len(self.program.inputs)} arrays, got {len(inputs)}")
        for name, x in zip(self.program.inputs, inputs):
            v = self.program.values[name]
            if not isinstance(x, torch.Tensor) or x.dtype != v.dtype or x.numel() != v.count:
                raise ValueError(f"{self.program.name}: argument {name} must be {v.count} elements of {v.dtype}, "
                                 f"got {getattr(x, 'dtype', type(x))} x {getattr(x, 'numel', lambda: '?')()}")

    def _take(self, name: str, x: torch.Tensor, point: bool) -> None:
        v = self.program.values[name]
        if point and self.target.pointable(x, x.data_ptr()):
            self.bound[name] = x
            self.addresses[name] = x.data_ptr()
            self.own.pop(name, None)
        else:
            buf = self.own.get(name)
            if buf is None:
                buf = self.target.allocate(v.dtype, v.count)
                self.own[name] = buf
            self.target.upload_into(buf, x.reshape(-1))
            self.bound.pop(name, None)
            self.addresses[name] = buf.data_ptr()

    def bind(self, *inputs: torch.Tensor) -> "Executable":
        """bind!(ex, inputs...) (runtime.jl:719): copy into own buffers."""
        return self._rebind(inputs, point=False)

    def point(self, *inputs: torch.Tensor) -> "Executable":
        """point!(ex, inputs...) (runtime.jl:818): the caller's arrays become storage."""
        return self._rebind(inputs, point=True)

    def _rebind(self, inputs, point: bool) -> "Executable":
        self._check(inputs)
        for name, x in zip(self.program.inputs, inputs):
            before = self.addresses[name]
            self._take(name, x, point)
            after = self.addresses[name]
            if after != before:
                for k, (g, l) in enumerate(zip(self.program.groups, self.launches)):
                    for i, v in enumerate(g.values):
                        if v == name:
                            l.repoint(i, after)
                            self._moved.add(k)
        return self

    # -- running --------------------------------------------------------------

    def execute(self) -> "Executable":
        """execute!(ex) (runtime.jl:1158): each launch in order."""
        for l in self.launches:
            l()
        self._moved.clear()  # the launches themselves carry the new addresses
        return self

    def capture(self, graph: bool | None = None) -> "Executable":
        """capture!(ex) (runtime.jl:1185): one graph of every launch, or the
        launches themselves where the target measures direct launches faster
        for this many kernels (HIPTarget.graph_pays); ``graph`` forces it."""
        if self.graph is not None:
            self.graph = self.target.recapture(self.graph, self.launches, as_graph=graph)
        else:
            self.graph = self.target.capture(self.launches, graph=graph)
        self._moved.clear()
        return self

    @property
    def graphed(self) -> bool:
        """Whether what capture recorded replays as a graph."""
        return isinstance(self.graph, Graph)

    def replay(self) -> "Executable":
        """replay!(ex) (runtime.jl:1208): retarget what moved, then one graph launch."""
        if self.graph is None:
            raise RuntimeError("replay before capture")
        if isinstance(self.graph, Graph):
            for k in sorted(self._moved):
                self.target.retarget(self.graph, k,
                                     [Move(n, 0, self.addresses[n], 0) for n in self.program.groups[k].values],
                                     lambda: None)
        self._moved.clear()
        self.target.replay(self.graph)
        return self

    def outputs(self) -> list[torch.Tensor]:
        """outputs(ex): the result buffers themselves (the next run overwrites them)."""
        out = []
        for name in self.program.outputs:
            v = self.program.values[name]
            t = self.own[name]
            out.append(t[0] if v.scalar else t.view(*reversed(v.dims)) if len(v.dims) > 1 else t)
        return out

    def work(self) -> tuple[float, float]:
        """Algorithmic bytes and flops of one run, summed over launches."""
        b = f = 0.0
        for l in self.launches:
            w = l.work()
            b += w.bytes
            f += w.flops
        return b, f

    def explain(self) -> str:
        """explain (runtime.jl:1216-1238): each kernel and what runs it."""
        ws = sum(1 for w in self.workspaces if w)
        lines = [f"{self.program.name}: {len(self.launches)} launches, arena {self.arena.bytes} bytes "
                 f"in {len(self.storage.sizes)} slots" + (f" and {ws} workspaces" if ws else "")]
        for g, l in zip(self.program.groups, self.launches):
            lines.append(f"  {g.name}: reads {', '.join(g.reads)}; writes {', '.join(g.writes)}; {l.describe()}")
        if self.graph is not None:
            lines.append("  replays as " + ("one graph" if self.graphed else "its launches, one by one (cheaper "
                                            "than a graph for this many kernels on this device)"))
        return "\n".join(lines)


def prepare(program: Program, target: HIPTarget, *inputs: torch.Tensor, point: bool = True,
            pool: Pool | None = None) -> Executable:
    return Executable(program, target, inputs, point=point, pool=pool)


class Compiled:
    """compile(f, args...) for a planned program (compile.jl:48-62, 310-349)."""

    def __init__(self, program: Program, target: HIPTarget, inputs: Sequence[torch.Tensor], capture: bool = True):
        self.executable = ex = prepare(program, target, *inputs)
        self.signature = [(x.dtype, tuple(x.shape)) for x in inputs]
        if capture:
            ex.capture()
        # Where each result lies in the executable's result allocation, and
        # the span holding the numbers (read to the host in one copy).
        self._layout = []
        for name in program.outputs:
            v = program.values[name]
            off, nbytes = ex.result_at[name]
            self._layout.append((off, nbytes, v.dtype, v.scalar, tuple(reversed(v.dims)) if len(v.dims) > 1 else None))
        spans = [(off, off + nbytes) for off, nbytes, _, scalar, _ in self._layout if scalar]
        self._numbers = (min(a for a, _ in spans), max(b for _, b in spans)) if spans else None

    def __call__(self, *args: torch.Tensor):
        sig = [(getattr(x, "dtype", None), tuple(getattr(x, "shape", ()))) for x in args]
        if sig != self.signature:
            raise ValueError(f"call does not match the compiled signature {self.signature}: {sig}")
        ex = self.executable
        ex.point(*args)
        ex.replay() if ex.graph is not None else ex.execute()
        return self.returned()

    def returned(self):
        """Arrays copied, numbers read to the host (compile.jl:334-349): one
        copy of the result allocation, whose views are the arrays returned,
        then one read of the span holding the numbers."""
        fresh = self.executable.results.clone()
        host = None
        if self._numbers is not None:
            lo, hi = self._numbers
            host = fresh[lo:hi].cpu()
        out = []
        for off, nbytes, dtype, scalar, shape in self._layout:
            if scalar:
                out.append(host[off - self._numbers[0]:off - self._numbers[0] + nbytes].view(dtype)[0].item())
            else:
                t = fresh[off:off + nbytes].view(dtype)
                out.append(t.view(*shape) if shape is not None else t)
        return tuple(out)


def compile(program: Program, target: HIPTarget, *inputs: torch.Tensor, capture: bool = True) -> Compiled:
    return Compiled(program, target, inputs, capture=capture)
