"""The golden vectors (tests/golden/golden.json, made by make_golden.py):
the oracle reproduces them, and the reference's own known answers hold."""
import json
import pathlib

import numpy as np
import pytest

from oracle import folds, interpret
from oracle.data import relative
from golden.make_golden import attention_inputs

GOLDEN = json.loads((pathlib.Path(__file__).resolve().parent / "golden" / "golden.json").read_text())


def arr(d):
    return np.asarray(d["data"], dtype=np.float64).reshape(d["shape"])


def test_reference_known_answers():
    k = GOLDEN["kats"]
    assert folds.fold(folds.SumFold(), [x * x for x in k["sum_abs2_1234"]["input"]]) == k["sum_abs2_1234"]["output"]
    rec = folds.GenericFold(init_fn=lambda: (1.0, 0.0), lift_fn=lambda e: tuple(e),
                            combine_fn=lambda a, b: (b[0] * a[0], b[0] * a[1] + b[1]), observe_fn=lambda s: s[-1])
    assert folds.accumulate(rec, k["linear_recurrence"]["input"]) == k["linear_recurrence"]["output"]
    assert [2 * x for x in k["bind_execute_double"]["input"]] == k["bind_execute_double"]["output"]


@pytest.mark.parametrize("name", ["softmax_columns", "layernorm"])
def test_row_programs(name):
    g = GOLDEN[name]
    f = interpret.softmax_grad if name == "softmax_columns" else interpret.layernorm_grad
    loss, dx = f(arr(g["x"]), arr(g["g"]))
    assert abs(loss - g["loss"]) < 1e-12 and relative(dx, arr(g["dx"])) < 1e-12


def test_tanh_layer():
    g = GOLDEN["tanh_layer"]
    loss, dw, db, dx = interpret.tanh_layer_grad(arr(g["w"]), arr(g["b"]), arr(g["x"]))
    assert abs(loss - g["loss"]) < 1e-10
    for a, key in ((dw, "dw"), (db, "db"), (dx, "dx")):
        assert relative(a, arr(g[key])) < 1e-12


def test_mlp_and_attention():
    g = GOLDEN["mlp"]
    res = interpret.mlp_grad(*(arr(g[k]) for k in ("W1", "b1", "W2", "b2", "x")))
    assert abs(res[0] - g["loss"]) < 1e-10
    for a, key in zip(res[1:], ("dW1", "db1", "dW2", "db2", "dx")):
        assert relative(a, arr(g[key])) < 1e-12
    g = GOLDEN["attention"]
    q, k, v, do = attention_inputs(g["recipe"])
    rows = g["rows"]
    o, lse = interpret.attention_fwd(q, k, v, True)
    assert relative(o[0, rows, 0], arr(g["o"])) < 1e-12 and relative(lse, arr(g["lse"])) < 1e-12
    grads = interpret.attention_bwd(q, k, v, do, True)
    for a, key in zip(grads, ("dq", "dk", "dv")):
        assert relative(a[0, rows, 0], arr(g[key])) < 1e-12
