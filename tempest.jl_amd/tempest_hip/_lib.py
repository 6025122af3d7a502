"""ctypes binding of libtempest_hip.so (include/tempest_hip.h).

The library is loaded from the package's parent directory, where
tempest.jl_amd/build.py puts it.  There is no fallback: a missing library is
an error, and every non-zero status raises ``HIPError`` with the library's
message, as the reference turns a failed build into an exception that its
cover catches (src/Compiler/cover/choose.jl:1014-1025).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

# TEMPEST_HIP_LIBRARY names another build of the same ABI (the host-only
# sanitized check build); by default the in-tree library.
LIBRARY = pathlib.Path(os.environ.get("TEMPEST_HIP_LIBRARY") or
                       pathlib.Path(__file__).resolve().parent.parent / "libtempest_hip.so")

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_u64 = ctypes.c_uint64
c_f32 = ctypes.c_float
c_size = ctypes.c_size_t
c_char_p = ctypes.c_char_p
c_double = ctypes.c_double
P = ctypes.POINTER


class Rates(ctypes.Structure):
    _fields_ = [("launch", c_double), ("cached", c_double), ("bandwidth", c_double),
                ("cache", c_double), ("blocks", c_double)]


class Work(ctypes.Structure):
    _fields_ = [("bytes", c_double), ("flops", c_double), ("blocks", c_i64),
                ("kernels", c_i32), ("values", c_i32)]


class GemmDesc(ctypes.Structure):
    """th_gemm_desc (include/tempest_hip.h)."""
    _fields_ = [("m", c_i32), ("n", c_i32), ("k", c_i32), ("c_dtype", c_i32), ("epilogue", c_i32),
                ("tile", c_i32), ("a", c_void_p), ("a_m", c_i64), ("a_k", c_i64), ("b", c_void_p),
                ("b_k", c_i64), ("b_n", c_i64), ("c", c_void_p), ("c_ld", c_i64), ("bias", c_void_p),
                ("aux", c_void_p), ("aux_ld", c_i64), ("aux_out", c_void_p), ("row_sums", c_void_p),
                ("loss", c_void_p), ("batch", c_i32), ("flags", c_i32), ("a_batch", c_i64), ("b_batch", c_i64),
                ("c_batch", c_i64), ("d", c_void_p), ("d_ld", c_i64), ("d_batch", c_i64), ("splits", c_i32),
                ("reserved2", c_i32)]


class AttentionDesc(ctypes.Structure):
    """th_attention_desc (include/tempest_hip.h)."""
    _fields_ = [("batch", c_i32), ("heads", c_i32), ("kv_heads", c_i32), ("seq", c_i32), ("head_dim", c_i32),
                ("causal", c_i32), ("scale", c_f32), ("flags", c_i32), ("q", c_void_p), ("k", c_void_p),
                ("v", c_void_p), ("o", c_void_p), ("lse", c_void_p), ("dout", c_void_p), ("dq", c_void_p),
                ("dk", c_void_p), ("dv", c_void_p), ("q_strides", c_i64 * 3), ("k_strides", c_i64 * 3),
                ("kv_seq", c_i32), ("reserved", c_i32), ("starts", c_void_p), ("lengths", c_void_p)]


class DeltaNetDesc(ctypes.Structure):
    """th_deltanet_desc (include/tempest_hip.h)."""
    _fields_ = [("batch", c_i32), ("heads", c_i32), ("seq", c_i32), ("dk", c_i32), ("dv", c_i32), ("chunk", c_i32),
                ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("a", c_void_p), ("beta", c_void_p),
                ("o", c_void_p), ("dout", c_void_p), ("dq", c_void_p), ("dk_out", c_void_p), ("dv_out", c_void_p),
                ("da", c_void_p), ("dbeta", c_void_p), ("strides", c_i64 * 3), ("gate_strides", c_i64 * 3)]


FLOOR_RANK = 4


class Part(ctypes.Structure):
    _fields_ = [("kind", c_i32), ("reserved", c_i32), ("divisor", c_i64), ("coeff", c_i64), ("constant", c_i64),
                ("inner", c_i64 * FLOOR_RANK)]


class Affine(ctypes.Structure):
    _fields_ = [("constant", c_i64), ("coeff", c_i64 * FLOOR_RANK), ("gather", c_i32), ("reserved", c_i32),
                ("gather_coeff", c_i64), ("part", Part * 2)]


class FloorValue(ctypes.Structure):
    _fields_ = [("dtype", c_i32), ("reserved", c_i32), ("length", c_i64), ("ptr", c_void_p)]


class TermStruct(ctypes.Structure):
    _fields_ = [("op", c_i32), ("fn", c_i32), ("args", c_i32 * 3), ("ref", c_i32),
                ("observe", c_i32), ("lit", c_f32), ("index", Affine)]


class FoldStruct(ctypes.Structure):
    _fields_ = [("kind", c_i32), ("phase", c_i32), ("body", c_i32), ("weight", c_i32), ("scan", c_i32),
                ("n_inner", c_i32), ("inner", c_i64 * FLOOR_RANK)]


class OutputStruct(ctypes.Structure):
    _fields_ = [("value", c_i32), ("term", c_i32), ("full", c_i32), ("accumulate", c_i32),
                ("index", Affine)]


class FloorDesc(ctypes.Structure):
    _fields_ = [("kind", c_i32), ("rank", c_i32), ("extents", c_i64 * FLOOR_RANK),
                ("reduced", ctypes.c_uint32), ("n_values", c_i32), ("n_terms", c_i32),
                ("n_folds", c_i32), ("n_outputs", c_i32), ("flags", c_i32),
                ("values", ctypes.POINTER(FloorValue)), ("terms", ctypes.POINTER(TermStruct)),
                ("folds", ctypes.POINTER(FoldStruct)), ("outputs", ctypes.POINTER(OutputStruct))]


class HIPError(RuntimeError):
    """A libtempest_hip entry point returned a non-zero status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code


# name -> argtypes; every entry returns int.
SIGNATURES: dict[str, list] = {
    "th_init": [c_int],
    "th_shutdown": [],
    "th_device_name": [c_char_p, c_size],
    "th_toolchain": [c_char_p, c_size],
    "th_device_rates": [P(Rates)],
    "th_set_stream": [c_void_p],
    "th_get_stream": [P(c_void_p)],
    "th_quiesce": [],
    "th_alloc": [c_size, P(c_void_p)],
    "th_free": [c_void_p],
    "th_upload": [c_void_p, c_void_p, c_size],
    "th_download": [c_void_p, c_void_p, c_size],
    "th_copy": [c_void_p, c_void_p, c_size],
    "th_build_copy": [c_void_p, c_void_p, c_u64, P(c_void_p)],
    "th_matrix_rate": [ctypes.c_int, P(ctypes.c_double), P(ctypes.c_double)],
    "th_lds_rate": [ctypes.c_int, ctypes.c_int, P(ctypes.c_double), P(ctypes.c_double), P(ctypes.c_double)],
    "th_read_rate": [ctypes.c_int, P(ctypes.c_double)],
    "th_arena_create": [P(c_u64), c_int, c_u64, P(c_void_p)],
    "th_arena_slot": [c_void_p, c_int, P(c_void_p)],
    "th_arena_bytes": [c_void_p, P(c_u64)],
    "th_arena_destroy": [c_void_p],
    "th_pool_create": [c_u64, P(c_void_p)],
    "th_pool_alloc": [c_void_p, c_u64, c_u64, P(c_void_p)],
    "th_pool_free": [c_void_p, c_void_p],
    "th_pool_info": [c_void_p, P(c_void_p), P(c_u64), P(c_u64)],
    "th_pool_destroy": [c_void_p],
    "th_launch_run": [c_void_p],
    "th_launch_repoint": [c_void_p, c_int, c_void_p],
    "th_launch_work": [c_void_p, P(Work)],
    "th_launch_describe": [c_void_p, c_char_p, c_size],
    "th_launch_destroy": [c_void_p],
    "th_graph_capture": [P(c_void_p), c_int, P(c_void_p)],
    "th_graph_replay": [c_void_p],
    "th_graph_retarget": [c_void_p, c_int],
    "th_graph_release": [c_void_p],
    "th_time_launch": [c_void_p, c_int, P(c_double)],
    "th_time_graph": [c_void_p, c_int, c_int, P(c_double)],
    "th_time_run": [c_void_p, c_int, c_int, P(c_double)],
    "th_launch_workspace": [c_void_p, P(c_u64)],
    "th_launch_set_workspace": [c_void_p, c_void_p],
    "th_dispatch_costs": [P(c_double), P(c_double), P(c_double)],
    "th_build_softmax_grad": [c_i64, c_i32, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, P(c_void_p)],
    "th_softmax_grad_noalloc": [c_i64, c_i32, c_i64, c_void_p, c_void_p, c_void_p, c_void_p],
    "th_build_layernorm_grad": [c_i64, c_i32, c_i64, c_f32, c_void_p, c_void_p, c_void_p, c_void_p, P(c_void_p)],
    "th_build_softmax_fwd": [c_i64, c_i32, c_i64, c_void_p, c_void_p, P(c_void_p)],
    "th_build_layernorm_fwd": [c_i64, c_i32, c_i64, c_f32, c_void_p, c_void_p, P(c_void_p)],
    "th_build_sum": [c_i64, c_void_p, c_void_p, P(c_void_p)],
    "th_build_gemm": [P(GemmDesc), P(c_void_p)],
    "th_build_gemm_grouped": [P(GemmDesc), c_int, P(c_void_p)],
    "th_gemm_tune": [P(GemmDesc), P(c_i32), P(c_i32), P(c_double)],
    "th_build_attention_fwd": [P(AttentionDesc), P(c_void_p)],
    "th_build_attention_bwd": [P(AttentionDesc), P(c_void_p)],
    "th_build_deltanet_fwd": [P(DeltaNetDesc), P(c_void_p)],
    "th_build_deltanet": [P(DeltaNetDesc), P(c_void_p)],
    "th_build_floor": [P(FloorDesc), P(c_void_p)],
    "th_floor_source": [P(FloorDesc), c_char_p, c_size, P(c_size)],
    "th_floor_compile": [P(FloorDesc)],
    "th_floor_cache_counts": [P(c_i64), P(c_i64)],
    "th_build_tanh_layer_grad": [c_i32, c_i32, c_i32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_void_p, P(c_void_p)],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The library, loaded once; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIBRARY.exists():
                raise FileNotFoundError(
                    f"{LIBRARY} is missing: build it with `python tempest.jl_amd/build.py` "
                    "(or __graft_entry__.build()); there is no fallback path")
            lib = ctypes.CDLL(str(LIBRARY))
            for name, args in SIGNATURES.items():
                f = getattr(lib, name)
                f.argtypes = args
                f.restype = c_int
            lib.th_last_error.argtypes = []
            lib.th_last_error.restype = c_char_p
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call entry point ``name``; raise HIPError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise HIPError(name, rc, lib.th_last_error().decode(errors="replace"))


def out_ptr() -> c_void_p:
    return c_void_p()
