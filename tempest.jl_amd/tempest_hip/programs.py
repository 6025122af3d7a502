"""The hot path's programs, each as the plan Tempest's front end forms for it.

Julia's tracer and planner stay Julia's; without them in this build, each
program below states its plan: its values (inputs, results, stored values)
and its groups, each claimed by one of this backend's op classes.  The
programs are the configs the backend is measured on:

1. ``tanh_layer``  loss(w, b, x) = sum(abs2, tanh.(w' * x .+ b)) with
   withgradient: one group (the whole program fits one workgroup).
2. ``softmax_columns`` / ``layernorm``  sum(f(x) .* g) with withgradient,
   f = softmax over columns (test/fixtures/programs.jl:8,74) or LayerNorm,
   weight 1, bias 0, eps 1e-5 (programs.jl:13-17): one fused row group each
   (forward, its fold, and the gradient) and the loss's full fold.
"""
from __future__ import annotations

import torch

from . import launch as L
from .runtime import Group, Program, Value


def tanh_layer(d: int = 32, h: int = 64, c: int = 16) -> Program:
    """Config 1: loss(w, b, x) = sum(abs2, tanh.(w'x .+ b)), w d x h, b h, x d x c."""
    f32 = torch.float32
    values = {
        "w": Value("w", f32, (d, h), "input"),
        "b": Value("b", f32, (h,), "input"),
        "x": Value("x", f32, (d, c), "input"),
        "loss": Value("loss", f32, (), "result"),
        "dw": Value("dw", f32, (d, h), "result"),
        "db": Value("db", f32, (h,), "result"),
        "dx": Value("dx", f32, (d, c), "result"),
    }
    names = ("w", "b", "x", "loss", "dw", "db", "dx")
    group = Group("tanh layer and its gradient", names, ("w", "b", "x"), ("loss", "dw", "db", "dx"),
                  lambda a: L.tanh_layer_grad(d, h, c, *(a[n] for n in names)))
    return Program("tanh_layer", values, [group], ["w", "b", "x"], ["loss", "dw", "db", "dx"])


def _row_program(name: str, rows: int, n: int, build) -> Program:
    f32 = torch.float32
    values = {
        "x": Value("x", f32, (n, rows), "input"),
        "g": Value("g", f32, (n, rows), "input"),
        "loss": Value("loss", f32, (), "result"),
        "dx": Value("dx", f32, (n, rows), "result"),
    }
    group = Group(f"{name}, its fold and gradient; the loss", ("x", "g", "dx", "loss"), ("x", "g"), ("dx", "loss"),
                  lambda a: build(a["x"], a["g"], a["dx"], a["loss"]))
    return Program(name, values, [group], ["x", "g"], ["loss", "dx"])


def softmax_columns(rows: int, n: int) -> Program:
    """Config 2a: (x, g) -> sum(softmax_columns(x) .* g) and its gradient; x, g n x rows."""
    return _row_program("softmax_columns", rows, n, lambda x, g, dx, loss: L.softmax_grad(rows, n, n, x, g, dx, loss))


def layernorm(rows: int, n: int, eps: float = 1e-5) -> Program:
    """Config 2b: (x, g) -> sum(layernorm(x) .* g) and its gradient; x, g n x rows."""
    return _row_program("layernorm", rows, n,
                        lambda x, g, dx, loss: L.layernorm_grad(rows, n, n, eps, x, g, dx, loss))
