"""tempest_hip: the host side of Tempest's MI355X execution backend.

The reference's boundary is two Julia protocols: the Target protocol
(src/Compiler/runtime/target.jl) and the Implement interface
(src/Compiler/Implement/).  This package mirrors them over the C ABI of
libtempest_hip (include/tempest_hip.h): ``HIPTarget`` is the target,
``launch`` holds the claims' builds, ``runtime`` the executable (slots,
binding, execute/capture/replay) and ``programs`` the plans of the hot path's
programs.  No path here falls back to the CPU: without the library, or
without a GPU, construction raises.
"""
from ._lib import HIPError, LIBRARY, load  # noqa: F401
from .launch import Launch  # noqa: F401
from .runtime import Compiled, Executable, Group, Pool, Program, Value, compile, prepare, storage  # noqa: F401
from .target import Direct, Graph, HIPTarget, Move  # noqa: F401
from . import programs  # noqa: F401

__all__ = ["HIPError", "LIBRARY", "load", "Launch", "Compiled", "Executable", "Group", "Program", "Value",
           "compile", "prepare", "storage", "Direct", "Graph", "HIPTarget", "Move", "Pool", "programs"]
