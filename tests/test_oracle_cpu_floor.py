"""The CPU floor's product and attention slices (oracle/floor.c), which time
configs 3 and 4 on one core: pinned against numpy products and against the
Float64 attention gradients of the interpreter."""
import numpy as np
import pytest

from oracle import floor, interpret
from oracle.data import bf16_bits, bf16_value, relative


def _bits(rng, shape):
    return bf16_bits(rng.standard_normal(shape).astype(np.float32)).reshape(shape)


@pytest.mark.parametrize("layout", ["mk", "km"])
def test_matmul_slice_matches_numpy(layout):
    rng = np.random.default_rng(3)
    m, k, n = 37, 53, 11
    A = _bits(rng, (m, k))
    B = _bits(rng, (k, n))
    a_store = np.asfortranarray(A) if layout == "mk" else np.ascontiguousarray(A)
    a_m, a_k = (1, m) if layout == "mk" else (k, 1)
    b_store = np.asfortranarray(B)
    flat_a = a_store.ravel(order="K")
    flat_b = b_store.ravel(order="K")
    c = floor.matmul_bf16(flat_a, a_m, a_k, flat_b, 1, k, m, k, 3, 9)
    want = bf16_value(A).astype(np.float64) @ bf16_value(B).astype(np.float64)[:, 3:9]
    assert relative(c, want) < 1e-6


@pytest.mark.parametrize("q0,step", [(0, 1), (2, 5)])
def test_attention_sample_matches_interpreter(q0, step):
    rng = np.random.default_rng(q0 * 10 + step)
    S, D = 40, 16
    q, k, v, g = (_bits(rng, (S, D)) for _ in range(4))
    scale = 1 / np.sqrt(D)
    dq, dk, dv = floor.attention_sample(q, k, v, g, scale, q0, step)
    sampled = np.arange(q0, S, step)
    gm = bf16_value(g).copy()
    keep = np.zeros(S, bool)
    keep[sampled] = True
    gm[~keep] = 0.0  # unsampled queries contribute nothing to dk, dv
    f = lambda x: bf16_value(x)[None, :, None, :].astype(np.float64)  # noqa: E731
    rdq, rdk, rdv = interpret.attention_bwd(f(q), f(k), f(v), gm[None, :, None, :].astype(np.float64),
                                           causal=True, scale=scale)
    assert relative(dq, rdq[0, sampled, 0]) < 1e-5
    assert relative(dk, rdk[0, :, 0]) < 1e-5
    assert relative(dv, rdv[0, :, 0]) < 1e-5
