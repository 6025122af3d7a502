"""TEST INFRASTRUCTURE ONLY: inputs the reference's tests use.

``data(dims...; scale) = 2 .* sin.(scale .* reshape(1:prod(dims), dims...))``
in Float64 (test/setup.jl:33) and ``single`` = Float32 (test/setup.jl:36).
Julia arrays are column-major, so ``data`` returns a Fortran-ordered array
whose first axis is fastest, element k (0-based, linear) = 2 sin(scale (k+1)).
"""
from __future__ import annotations

import numpy as np


def data(*dims: int, scale: float = 1.0) -> np.ndarray:
    n = int(np.prod(dims)) if dims else 1
    flat = 2.0 * np.sin(scale * np.arange(1, n + 1, dtype=np.float64))
    return flat.reshape(dims, order="F")


def single(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32, order="F")


def agree(a, b, rtol: float) -> bool:
    """``agree`` of test/setup.jl:41-42: Julia's isapprox per leaf with
    ``atol = rtol * 1e-2``, i.e. norm(a - b) <= max(atol, rtol * max(norm(a), norm(b)))."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    d = np.linalg.norm((a - b).ravel())
    return bool(d <= max(rtol * 1e-2, rtol * max(np.linalg.norm(a.ravel()), np.linalg.norm(b.ravel()))))


def relative(a, b) -> float:
    """Norm-wise relative difference of ``a`` from ``b`` (the quantity agree bounds)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    nb = np.linalg.norm(b.ravel())
    return float(np.linalg.norm((a - b).ravel()) / (nb if nb > 0 else 1.0))


def bf16_bits(x) -> np.ndarray:
    """Float32 values rounded to bfloat16 (nearest, ties to even), as uint16 bits:
    BFloat16s' conversion (BFloat16s.jl 0.6.5, the reference's bf16 type)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_value(bits) -> np.ndarray:
    """The float32 value of bfloat16 bits."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    return bf16_value(bf16_bits(x)).reshape(np.shape(x))
