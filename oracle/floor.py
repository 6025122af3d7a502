"""TEST INFRASTRUCTURE ONLY: ctypes binding of the Float32 CPU floor (floor.c).

The library is built by ``make -C oracle`` (also by __graft_entry__.build()).
Each function takes numpy float32 arrays in the layout the kernels use and
runs on one thread.  Pinning: tests/test_oracle_rows.py and
tests/test_oracle_tiny.py check the row and config-1 functions against the
Float64 interpreter within Float32 rounding; tests/test_oracle_cpu_floor.py
checks the product and attention slices against numpy and the interpreter.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB = None

_f32p = ctypes.POINTER(ctypes.c_float)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = _HERE / "libfloor.so"
        if not path.exists():
            raise FileNotFoundError(f"{path} is missing: run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int32, ctypes.c_float
        L.floor_softmax_grad.argtypes = [i64, i32, i64, _f32p, _f32p, _f32p, _f32p]
        L.floor_layernorm_grad.argtypes = [i64, i32, i64, f32, _f32p, _f32p, _f32p, _f32p]
        L.floor_softmax_fwd.argtypes = [i64, i32, i64, _f32p, _f32p]
        L.floor_layernorm_fwd.argtypes = [i64, i32, i64, f32, _f32p, _f32p]
        L.floor_tanh_layer_grad.argtypes = [i32, i32, i32, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p]
        u16p = ctypes.POINTER(ctypes.c_uint16)
        L.floor_matmul_bf16.argtypes = [i32, i32, u16p, i64, i64, u16p, i64, i64, _f32p, i64, i32, i32]
        L.floor_attention_sample.argtypes = [i32, i32, f32, u16p, u16p, u16p, u16p, i64, i32, i32,
                                             _f32p, _f32p, _f32p, _f32p]
        for f in (L.floor_softmax_grad, L.floor_layernorm_grad, L.floor_softmax_fwd,
                  L.floor_layernorm_fwd, L.floor_tanh_layer_grad, L.floor_matmul_bf16,
                  L.floor_attention_sample):
            f.restype = None
        _LIB = L
    return _LIB


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and (a.flags["C_CONTIGUOUS"] or a.flags["F_CONTIGUOUS"])
    return a.ctypes.data_as(_f32p)


def _rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.ndim == 2
    return x


def softmax_grad(x: np.ndarray, g: np.ndarray):
    x, g = _rows(x), _rows(g)
    dx = np.empty_like(x)
    loss = np.zeros(1, np.float32)
    lib().floor_softmax_grad(x.shape[0], x.shape[1], x.shape[1], _p(x), _p(g), _p(dx), _p(loss))
    return float(loss[0]), dx


def layernorm_grad(x: np.ndarray, g: np.ndarray, eps: float = 1e-5):
    x, g = _rows(x), _rows(g)
    dx = np.empty_like(x)
    loss = np.zeros(1, np.float32)
    lib().floor_layernorm_grad(x.shape[0], x.shape[1], x.shape[1], eps, _p(x), _p(g), _p(dx), _p(loss))
    return float(loss[0]), dx


def softmax_fwd(x: np.ndarray) -> np.ndarray:
    x = _rows(x)
    y = np.empty_like(x)
    lib().floor_softmax_fwd(x.shape[0], x.shape[1], x.shape[1], _p(x), _p(y))
    return y


def layernorm_fwd(x: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = _rows(x)
    y = np.empty_like(x)
    lib().floor_layernorm_fwd(x.shape[0], x.shape[1], x.shape[1], eps, _p(x), _p(y))
    return y


def tanh_layer_grad(w: np.ndarray, b: np.ndarray, x: np.ndarray):
    """w d x h, b h, x d x c as Julia matrices; stored column-major here."""
    d, h = w.shape
    c = x.shape[1]
    wf = np.asfortranarray(w, dtype=np.float32)
    xf = np.asfortranarray(x, dtype=np.float32)
    bf = np.ascontiguousarray(b, dtype=np.float32)
    loss = np.zeros(1, np.float32)
    dw = np.zeros((d, h), np.float32, order="F")
    db = np.zeros(h, np.float32)
    dx = np.zeros((d, c), np.float32, order="F")
    dz = np.zeros((h, c), np.float32, order="F")
    lib().floor_tanh_layer_grad(d, h, c, _p(wf), _p(bf), _p(xf), _p(loss), _p(dw), _p(db), _p(dx), _p(dz))
    return float(loss[0]), dw, db, dx


def _u16(a: np.ndarray):
    assert a.dtype == np.uint16
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def matmul_bf16(a_bits: np.ndarray, a_m: int, a_k: int, b_bits: np.ndarray, b_k: int, b_n: int,
                m: int, k: int, j0: int, j1: int) -> np.ndarray:
    """Columns j0 .. j1-1 of C = A B (m x k times k x n, bf16 bits with the
    given element strides), each element a sequential fp32 fold over k;
    returned as an m x (j1 - j0) float32 array, column-major."""
    c = np.zeros((m, j1 - j0), np.float32, order="F")
    lib().floor_matmul_bf16(m, k, _u16(a_bits), a_m, a_k, _u16(b_bits), b_k, b_n, _p(c), m, j0, j1)
    return c


def attention_sample(q, k, v, dout, scale: float, q0: int, step: int):
    """One (batch, head): q, k, v, dout are seq x d bf16 bits (row per
    position).  Returns dq of the sampled queries (q0, q0 + step, ...) and the
    dk, dv those queries contribute (seq x d)."""
    seq, d = q.shape
    rows = len(range(q0, seq, step))
    dq = np.zeros((rows, d), np.float32)
    dk = np.zeros((seq, d), np.float32)
    dv = np.zeros((seq, d), np.float32)
    p = np.zeros(seq, np.float32)
    qs, ks, vs, gs = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v, dout))
    lib().floor_attention_sample(seq, d, scale, _u16(qs), _u16(ks), _u16(vs), _u16(gs), d, q0, step,
                                 _p(dq), _p(dk), _p(dv), _p(p))
    return dq, dk, dv
