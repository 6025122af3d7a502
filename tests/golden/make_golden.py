"""Write tests/golden/golden.json: small input/output vectors of the hot
path's programs at the reference tests' closed-form inputs.

The reference stores no golden arrays; its tests compare every program with
its Float64 interpreter on ``data(dims...; scale) = 2 .* sin.(scale .* (1:n))``
inputs (test/setup.jl:33).  These vectors are that comparison's right-hand
side, computed by the oracle's Float64 restatement (oracle/interpret.py),
which tests/test_oracle_*.py pin against torch autograd, central differences
and closed forms.  The reference's own known answers are stored beside them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import interpret  # noqa: E402
from oracle.data import bf16_round, data  # noqa: E402


ATTENTION_ROWS = [0, 1, 63, 64, 127]


def attention_inputs(recipe: dict):
    """The golden attention case's inputs from their recipe."""
    S, D = recipe["seq"], recipe["d"]
    return [bf16_round(data(D * S, scale=recipe["scales"][n]).reshape(1, S, 1, D)) for n in ("q", "k", "v", "dout")]


def _arr(a) -> dict:
    a = np.asarray(a, dtype=np.float64)
    return {"shape": list(a.shape), "data": [float(x) for x in a.ravel(order="C")]}


def build() -> dict:
    out: dict = {"kats": {
        # src/Compiler/runtime/compile.jl:35-40
        "sum_abs2_1234": {"input": [1.0, 2.0, 3.0, 4.0], "output": 30.0},
        # src/Compiler/IR/folds.jl:279-288
        "linear_recurrence": {"input": [[0.5, 1.0]] * 3, "output": [1.0, 1.5, 1.75]},
        # src/Compiler/runtime/runtime.jl:708-717 (bind! then execute! of 2 .* x)
        "bind_execute_double": {"input": [3.0, 4.0], "output": [6.0, 8.0]},
    }}
    # Row programs: the reference's "softmax columns" fixture inputs
    # (test/fixtures/programs.jl:74): x = data(8, 6), g = data(8, 6; scale = 0.7),
    # each numpy row one of the reference's columns.
    x = data(8, 6).T.copy()
    g = data(8, 6, scale=0.7).T.copy()
    for name, f in (("softmax_columns", interpret.softmax_grad), ("layernorm", interpret.layernorm_grad)):
        loss, dx = f(x, g)
        out[name] = {"x": _arr(x), "g": _arr(g), "loss": loss, "dx": _arr(dx)}
    # Config 1 at its shapes.
    w, b, xx = data(32, 64), data(64, scale=0.3), data(32, 16, scale=0.7)
    loss, dw, db, dx = interpret.tanh_layer_grad(w, b, xx)
    out["tanh_layer"] = {"w": _arr(w), "b": _arr(b), "x": _arr(xx), "loss": loss, "dw": _arr(dw), "db": _arr(db),
                         "dx": _arr(dx)}
    # Config 3's program, small, bf16 inputs from data().
    h, d, bt, o = 16, 8, 8, 8
    W1 = bf16_round(data(h, d, scale=0.31) / np.sqrt(d))
    b1 = bf16_round(data(h, scale=0.17) / np.sqrt(d))
    W2 = bf16_round(data(o, h, scale=0.23) / np.sqrt(h))
    b2 = bf16_round(data(o, scale=0.11) / np.sqrt(h))
    X = bf16_round(data(d, bt, scale=0.7))
    loss, dW1, db1, dW2, db2, dX = interpret.mlp_grad(W1, b1, W2, b2, X)
    out["mlp"] = {"W1": _arr(W1), "b1": _arr(b1), "W2": _arr(W2), "b2": _arr(b2), "x": _arr(X), "loss": loss,
                  "dW1": _arr(dW1), "db1": _arr(db1), "dW2": _arr(dW2), "db2": _arr(db2), "dx": _arr(dX)}
    # Config 4's program, one head of 128 features at 128 positions, causal;
    # (batch, positions, heads, d) arrays from data().
    S, D = 128, 128
    q, k, v, do = attention_inputs({"scales": {"q": 0.37, "k": 0.53, "v": 0.71, "dout": 0.29}, "seq": S, "d": D})
    ao, lse = interpret.attention_fwd(q, k, v, True)
    dq, dk, dv = interpret.attention_bwd(q, k, v, do, True)
    # Inputs are kept as their recipe (data() at these scales, rounded to bf16,
    # reshaped to (1, 128, 1, 128)); outputs at positions ROWS, and lse whole.
    rows = ATTENTION_ROWS
    out["attention"] = {"recipe": {"scales": {"q": 0.37, "k": 0.53, "v": 0.71, "dout": 0.29}, "seq": S, "d": D},
                        "rows": rows, "o": _arr(ao[0, rows, 0]), "lse": _arr(lse),
                        "dq": _arr(dq[0, rows, 0]), "dk": _arr(dk[0, rows, 0]), "dv": _arr(dv[0, rows, 0])}
    return out


def main() -> None:
    path = HERE / "golden.json"
    path.write_text(json.dumps(build()))
    print(path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
