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
