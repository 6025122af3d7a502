"""``HIPTarget``: the reference's Target protocol on one MI355X.

Mirrors src/Compiler/runtime/target.jl (the protocol, :1-658) as the CUDA
target implements it (ext/CUDAExt.jl), over libtempest_hip.  Names follow the
protocol; Julia's ``f!`` become ``f`` here where Python has no ``!``
(``upload!`` -> ``upload_into``, ``download!`` -> ``download_into``,
``retarget!`` -> ``retarget``).  Caller arrays are torch tensors on the GPU
(the role CuArray plays); torch is plumbing for memory and streams only.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib
from ._lib import call
from .launch import Launch

# Kernels assume 16-byte aligned storage; the arena and torch align more.
ALIGNMENT = 16


@dataclass
class Move:
    """A value's storage moved: retarget!'s ``(value, from, to, bytes)``
    (src/Compiler/runtime/target.jl:552-565)."""

    value: str
    src: int
    dst: int
    bytes: int


class Graph:
    """What ``capture`` recorded: a th_graph* and the launches it keeps alive."""

    def __init__(self, handle: ctypes.c_void_p, steps: Sequence[Launch]):
        self._h = handle
        self.steps = list(steps)  # `keep`: alive until release

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("graph used after release")
        return self._h

    def release(self) -> None:
        if self._h is not None:
            call("th_graph_release", self._h)
            self._h = None
            self.steps = []

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class Direct:
    """What ``capture`` records where launching the steps one by one costs
    less than replaying them as a graph: the launches themselves, which carry
    their own (repointed) arguments."""

    def __init__(self, steps: Sequence[Launch]):
        self.steps = list(steps)

    def release(self) -> None:
        self.steps = []


_initialised: int | None = None


class HIPTarget:
    """Run on one MI355X (gfx950) through libtempest_hip.

    Options as CUDATarget's (target.jl:30-75): ``precision`` for products of
    fp32 factors, ``"full"`` (fp32 on the fp32 matrix cores) or ``"bf16x3"``
    (each factor split hi + lo in bf16 and three bf16 products summed in
    fp32, TH_GEMM_BF16X3: the counterpart of CUDA's ``:tf32x3``); half
    factors always accumulate in fp32.  ``online`` (permits the online
    softmax), ``rounded_backward``, ``deterministic`` (every kernel here folds
    in a fixed order but the floor's folds by key, which add by atomics unless
    their groups run in order, FloorGroup(ordered=True)).
    """

    def __init__(self, implementations: Sequence = (), device: int = 0, precision: str = "full",
                 online: bool = True, rounded_backward: bool = True, deterministic: bool = False):
        if precision not in ("full", "bf16x3"):
            raise ValueError(f"precision must be 'full' or 'bf16x3' on this target, got {precision!r}")
        self.implementations = tuple(implementations)
        self.device = device
        self.precision = precision
        self.online = online
        self.rounded_backward = rounded_backward
        self.deterministic_ = deterministic
        self._dispatch: tuple[float, float, float] | None = None
        self._init()

    # -- device -----------------------------------------------------------------

    def _init(self) -> None:
        global _initialised
        if _initialised is None:
            if not torch.cuda.is_available():
                raise RuntimeError("HIPTarget needs a visible AMD GPU (torch.cuda.is_available() is False)")
            torch.cuda.set_device(self.device)
            call("th_init", self.device)
            _initialised = self.device
        elif _initialised != self.device:
            raise RuntimeError(f"this process drives device {_initialised}; one device per process")
        # Launch on torch's current stream, so torch's work on the same arrays
        # (allocation, filling, copies) is ordered with ours.
        call("th_set_stream", ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream))

    def device_name(self) -> str:  # target.jl:583
        buf = ctypes.create_string_buffer(512)
        call("th_device_name", buf, len(buf))
        return buf.value.decode()

    def toolchain(self) -> list[tuple[str, str]]:  # target.jl:594
        buf = ctypes.create_string_buffer(1024)
        call("th_toolchain", buf, len(buf))
        return [tuple(kv.split("=", 1)) for kv in buf.value.decode().split(";")]

    def measurable(self) -> bool:  # target.jl:597
        return True

    def device_rates(self) -> dict:  # ext/CUDAExt.jl:913-921
        r = _lib.Rates()
        call("th_device_rates", ctypes.byref(r))
        return {"launch": r.launch, "cached": r.cached, "bandwidth": r.bandwidth, "cache": r.cache,
                "blocks": r.blocks}

    def numerics(self) -> str:  # target.jl:194-196
        return self.precision + ("" if self.online else "-two-pass") + \
            ("" if self.rounded_backward else "-exact-backward") + ("-deterministic" if self.deterministic_ else "")

    def permits_rewrites(self) -> bool:
        return self.online

    def deterministic(self) -> bool:
        return self.deterministic_

    def product_class(self, dtype: torch.dtype) -> str:  # cover/cost.jl:132
        """Half factors by their type; fp32 ones by the precision they run in."""
        return {torch.bfloat16: "BFloat16", torch.float16: "Float16"}.get(dtype, self.precision)

    def product_options(self, dtype: torch.dtype) -> dict:
        """The gemm keywords this target's precision gives a product of `dtype` factors."""
        return {"bf16x3": True} if dtype == torch.float32 and self.precision == "bf16x3" else {}

    # -- storage ------------------------------------------------------------------

    def allocate(self, dtype: torch.dtype, n: int) -> torch.Tensor:  # target.jl:241
        return torch.empty(n, dtype=dtype, device=f"cuda:{self.device}")

    def upload(self, x) -> torch.Tensor:  # target.jl:249
        t = torch.as_tensor(x)
        return t.to(device=f"cuda:{self.device}").contiguous()

    def upload_into(self, buffer: torch.Tensor, x) -> torch.Tensor:  # upload!, target.jl:258
        buffer.copy_(torch.as_tensor(x).reshape(buffer.shape))
        return buffer

    def download_into(self, x, buffer: torch.Tensor):  # download!, target.jl:267
        x.copy_(buffer.reshape(x.shape))
        return x

    def bindable(self, x) -> bool:  # target.jl:270
        return isinstance(x, torch.Tensor) and x.is_cuda and x.is_contiguous()

    def pointable(self, x, at: int) -> bool:  # target.jl:281; ext/CUDAExt.jl:40-42
        return self.bindable(x) and at % ALIGNMENT == 0

    # -- streams ------------------------------------------------------------------

    def task_stream(self):  # target.jl:483
        p = ctypes.c_void_p()
        call("th_get_stream", ctypes.byref(p))
        return p.value

    def quiesce(self) -> None:  # target.jl:493,617
        call("th_quiesce")

    # -- graphs ---------------------------------------------------------------------

    def dispatch_costs(self) -> tuple[float, float, float]:
        """(graph_base, in_graph, direct): device seconds, back to back, of a
        graph replay beyond its launches, a launch inside a replayed graph and
        a direct launch (th_dispatch_costs; measured once per process)."""
        if self._dispatch is None:
            a, b, c = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
            call("th_dispatch_costs", ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
            self._dispatch = (a.value, b.value, c.value)
        return self._dispatch

    def graph_pays(self, steps: Sequence[Launch]) -> bool:
        """Whether K kernels replay faster as one graph than launched one by
        one: graph_base + K in_graph < K direct."""
        k = sum(s.work().kernels for s in steps)
        base, gap, direct = self.dispatch_costs()
        return base + k * gap < k * direct

    def capture(self, steps: Sequence[Launch], keep=None, graph: bool | None = None) -> Graph | Direct:
        """capture(target, steps, keep) (target.jl:541; CUDAExt.jl:565): one
        graph of the steps, or, where launching them directly measures faster
        on this device (``graph_pays``), the steps themselves; ``graph``
        forces the choice."""
        if not (self.graph_pays(steps) if graph is None else graph):
            return Direct(steps)
        arr = (ctypes.c_void_p * len(steps))(*[s.handle.value for s in steps])
        out = ctypes.c_void_p()
        call("th_graph_capture", arr, len(steps), ctypes.byref(out))
        return Graph(out, steps)

    def recapture(self, graph: Graph | Direct, steps: Sequence[Launch], keep=None,
                  as_graph: bool | None = None) -> Graph | Direct:  # target.jl:550
        graph.release()
        return self.capture(steps, keep, as_graph)

    def retarget(self, graph: Graph, step: int, moves: Sequence[Move], repoint) -> bool:
        """retarget!(target, graph, steps, moves, repoint) (target.jl:552-565,
        ext/CUDAExt.jl:614-623): point the launch (``repoint()``), then the
        graph's nodes of that step take its arguments in place.  Our kernels'
        argument layouts are known, so nothing is learned and no re-record is
        needed: always true."""
        repoint()
        if isinstance(graph, Graph):
            call("th_graph_retarget", graph.handle, step)
        return True

    def replay(self, graph: Graph | Direct) -> None:  # target.jl:568; CUDAExt.jl:739
        if isinstance(graph, Direct):
            for s in graph.steps:
                s()
        else:
            call("th_graph_replay", graph.handle)

    def release(self, graph: Graph) -> None:  # target.jl:571
        graph.release()

    # -- timing ---------------------------------------------------------------------

    def time_launch(self, launch: Launch, samples: int = 0) -> float:  # target.jl:609; CUDAExt.jl:760
        s = ctypes.c_double()
        call("th_time_launch", launch.handle, samples, ctypes.byref(s))
        return s.value

    def time_graph(self, graph: Graph, warmup: int = 3, reps: int = 20) -> float:  # CUDAExt.jl:886 (batched)
        s = ctypes.c_double()
        call("th_time_graph", graph.handle, warmup, reps, ctypes.byref(s))
        return s.value

    def time_run(self, launch: Launch, warmup: int = 3, reps: int = 20) -> float:
        s = ctypes.c_double()
        call("th_time_run", launch.handle, warmup, reps, ctypes.byref(s))
        return s.value
