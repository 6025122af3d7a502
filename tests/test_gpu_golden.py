"""The GPU path against the golden vectors (tests/golden/golden.json)."""
import json
import pathlib

import numpy as np
import pytest
import torch

from conftest import announce
from oracle.data import relative
from golden.make_golden import attention_inputs

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((pathlib.Path(__file__).resolve().parent / "golden" / "golden.json").read_text())


def arr(d):
    return np.asarray(d["data"], dtype=np.float64).reshape(d["shape"])


def _f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("name", ["softmax_columns", "layernorm"])
def test_row_programs(target, name):
    import tempest_hip as th
    announce("golden", name)
    g = GOLDEN[name]
    x, gg = arr(g["x"]), arr(g["g"])
    rows, n = x.shape
    prog = th.programs.softmax_columns(rows, n) if name == "softmax_columns" else th.programs.layernorm(rows, n)
    loss, dx = th.compile(prog, target, _f32(x), _f32(gg))(_f32(x), _f32(gg))
    assert relative(dx.cpu().numpy(), arr(g["dx"])) < 1e-5
    assert abs(loss - g["loss"]) <= 1e-5 * max(1.0, abs(g["loss"]))


def test_tanh_layer(target):
    import tempest_hip as th
    announce("golden tanh layer")
    g = GOLDEN["tanh_layer"]
    args = [_f32(np.asfortranarray(arr(g[k])).T.copy() if arr(g[k]).ndim == 2 else arr(g[k])) for k in ("w", "b", "x")]
    loss, dw, db, dx = th.compile(th.programs.tanh_layer(), target, *args)(*args)
    assert abs(loss - g["loss"]) <= 1e-5 * abs(g["loss"])
    assert relative(dw.cpu().numpy().T, arr(g["dw"])) < 1e-5
    assert relative(db.cpu().numpy(), arr(g["db"])) < 1e-5
    assert relative(dx.cpu().numpy().T, arr(g["dx"])) < 1e-5


def test_attention(target):
    import tempest_hip as th
    announce("golden attention")
    g = GOLDEN["attention"]
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).cuda()  # noqa: E731
    q, k, v, do = (bf(a) for a in attention_inputs(g["recipe"]))
    o, dq, dk, dv = th.compile(th.programs.attention(1, 1, 128), target, q, k, v, do)(q, k, v, do)
    rows = g["rows"]
    pick = lambda t: t.float().cpu().numpy().reshape(1, 128, 1, 128)[0, rows, 0]  # noqa: E731
    assert relative(pick(o), arr(g["o"])) < 2e-2
    for t, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert relative(pick(t), arr(g[key])) < 2e-2
