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


def mlp(batch: int = 4096, d_in: int = 4096, hidden: int = 16384, d_out: int = 4096) -> Program:
    """Config 3: loss = sum(abs2, W2 * gelu.(W1 * x .+ b1) .+ b2) with withgradient
    w.r.t. (W1, b1, W2, b2, x); bf16 arrays, fp32 accumulation.

    Julia shapes: W1 hidden x d_in, b1 hidden, W2 d_out x hidden, b2 d_out,
    x d_in x batch (column-major).  Plan: six product groups, each with the
    pointwise work around it fused into its epilogue, and two stored values
    between the forward and the backward (Z1 = W1 x + b1 and H = gelu(Z1));
    dy = 2y and dZ1 = (W2' dy) .* gelu'(Z1) are stored for the weight
    products that read them.  The biases' gradients and the loss are the
    epilogues' row and full folds.
    """
    L_ = L
    bf, f32 = torch.bfloat16, torch.float32
    V = lambda name, dims, role, dt=bf: Value(name, dt, dims, role)  # noqa: E731
    values = {v.name: v for v in [
        V("W1", (hidden, d_in), "input"), V("b1", (hidden,), "input"),
        V("W2", (d_out, hidden), "input"), V("b2", (d_out,), "input"),
        V("x", (d_in, batch), "input"),
        V("Z1", (hidden, batch), "stored"), V("H", (hidden, batch), "stored"),
        V("dy", (d_out, batch), "stored"), V("dZ1", (hidden, batch), "stored"),
        V("loss", (), "result", f32), V("dW1", (hidden, d_in), "result"), V("db1", (hidden,), "result"),
        V("dW2", (d_out, hidden), "result"), V("db2", (d_out,), "result"), V("dx", (d_in, batch), "result"),
    ]}
    G = lambda name, vals, reads, writes, build: Group(name, vals, reads, writes, build)  # noqa: E731
    groups = [
        G("Z1 = W1 x .+ b1, H = gelu.(Z1)", ("W1", "x", "Z1", "b1", "", "H", "", ""), ("W1", "x", "b1"),
          ("Z1", "H"),
          lambda a: L_.gemm(hidden, batch, d_in, a["W1"], 1, hidden, a["x"], 1, d_in, a["Z1"], hidden,
                            epilogue=L_.GELU, bias=a["b1"], aux_out=a["H"])),
        G("y = W2 H .+ b2; loss = sum(y.^2); dy = 2y; db2 = sum(dy; dims=2)",
          ("W2", "H", "dy", "b2", "", "", "db2", "loss"), ("W2", "H", "b2"), ("dy", "db2", "loss"),
          lambda a: L_.gemm(d_out, batch, hidden, a["W2"], 1, d_out, a["H"], 1, hidden, a["dy"], d_out,
                            epilogue=L_.SQUARE_LOSS, bias=a["b2"], row_sums=a["db2"], loss=a["loss"])),
        G("dW2 = dy H'", ("dy", "H", "dW2", "", "", "", "", ""), ("dy", "H"), ("dW2",),
          lambda a: L_.gemm(d_out, hidden, batch, a["dy"], 1, d_out, a["H"], hidden, 1, a["dW2"], d_out)),
        G("dZ1 = (W2' dy) .* gelu'(Z1); db1 = sum(dZ1; dims=2)", ("W2", "dy", "dZ1", "", "Z1", "", "db1", ""),
          ("W2", "dy", "Z1"), ("dZ1", "db1"),
          lambda a: L_.gemm(hidden, batch, d_out, a["W2"], d_out, 1, a["dy"], 1, d_out, a["dZ1"], hidden,
                            epilogue=L_.GELU_BACKWARD, aux=a["Z1"], aux_ld=hidden, row_sums=a["db1"])),
        G("dW1 = dZ1 x'", ("dZ1", "x", "dW1", "", "", "", "", ""), ("dZ1", "x"), ("dW1",),
          lambda a: L_.gemm(hidden, d_in, batch, a["dZ1"], 1, hidden, a["x"], d_in, 1, a["dW1"], hidden)),
        G("dx = W1' dZ1", ("W1", "dZ1", "dx", "", "", "", "", ""), ("W1", "dZ1"), ("dx",),
          lambda a: L_.gemm(d_in, batch, hidden, a["W1"], hidden, 1, a["dZ1"], 1, hidden, a["dx"], d_in)),
    ]
    return Program("mlp", values, groups, ["W1", "b1", "W2", "b2", "x"], ["loss", "dW1", "db1", "dW2", "db2", "dx"])


def attention(batch: int = 8, heads: int = 16, seq: int = 4096, head_dim: int = 128, causal: bool = True,
              kv_heads: int = 0, recompute_dq: bool = False) -> Program:
    """Config 4: (q, k, v, dout) -> attention(q, k, v; causal) and the gradients
    of sum(attention(q, k, v) .* dout) w.r.t. q, k, v; bf16 (d, heads, positions,
    batch) arrays, fp32 statistics (test/fixtures/operations.jl:21-70).  With
    kv_heads < heads, k, v, dk and dv have kv_heads heads, query head h reading
    kv head h / (heads / kv_heads) (test/cuda/attention.jl:132-140).  With
    recompute_dq the dQ sweep recomputes S and dP instead of reading the dS'
    the dK/dV sweep stores.

    Plan: the forward's product, softmax and product fold into one online
    sweep over keys (the online-softmax rewrite, plan/rewrites.jl:29-41),
    storing o and lse; the backward recomputes the weights from lse."""
    bf, f32 = torch.bfloat16, torch.float32
    kv_heads = kv_heads or heads
    dims, kdims = (head_dim, heads, seq, batch), (head_dim, kv_heads, seq, batch)
    values = {
        "q": Value("q", bf, dims, "input"), "k": Value("k", bf, kdims, "input"), "v": Value("v", bf, kdims, "input"),
        "dout": Value("dout", bf, dims, "input"),
        "o": Value("o", bf, dims, "result"), "lse": Value("lse", f32, (1, heads, seq, batch), "stored"),
        "dq": Value("dq", bf, dims, "result"), "dk": Value("dk", bf, kdims, "result"),
        "dv": Value("dv", bf, kdims, "result"),
    }
    fwd = Group("o = attention(q, k, v); lse", ("q", "k", "v", "o", "lse"), ("q", "k", "v"), ("o", "lse"),
                lambda a: L.attention_fwd(batch, heads, kv_heads, seq, a["q"], a["k"], a["v"], a["o"], a["lse"],
                                          causal=causal))
    bwd = Group("dq, dk, dv", ("q", "k", "v", "o", "lse", "dout", "dq", "dk", "dv"),
                ("q", "k", "v", "o", "lse", "dout"), ("dq", "dk", "dv"),
                lambda a: L.attention_bwd(batch, heads, seq, a["q"], a["k"], a["v"], a["o"], a["lse"], a["dout"],
                                          a["dq"], a["dk"], a["dv"], causal=causal, kv_heads=kv_heads,
                                          recompute_dq=recompute_dq))
    return Program("attention", values, [fwd, bwd], ["q", "k", "v", "dout"], ["o", "dq", "dk", "dv"])


def deltanet(batch: int = 4, heads: int = 16, seq: int = 8192, d: int = 128) -> Program:
    """Config 5: (q, k, v, a, beta, dout) -> o = gated DeltaNet (chunks of 64)
    and the gradients of sum(o .* dout) w.r.t. q, k, v, a, beta.  q, k, v bf16
    (d, heads, positions, batch); a (log-gates) and beta fp32 (heads,
    positions, batch).  Plan: one group, its chunk-local products, the
    recurrence across chunks and their gradients (examples/deltanet.jl:58-86)."""
    bf, f32 = torch.bfloat16, torch.float32
    dims, gdims = (d, heads, seq, batch), (heads, seq, batch)
    values = {
        "q": Value("q", bf, dims, "input"), "k": Value("k", bf, dims, "input"), "v": Value("v", bf, dims, "input"),
        "a": Value("a", f32, gdims, "input"), "beta": Value("beta", f32, gdims, "input"),
        "dout": Value("dout", bf, dims, "input"),
        "o": Value("o", bf, dims, "result"), "dq": Value("dq", bf, dims, "result"),
        "dk": Value("dk", bf, dims, "result"), "dv": Value("dv", bf, dims, "result"),
        "da": Value("da", f32, gdims, "result"), "dbeta": Value("dbeta", f32, gdims, "result"),
    }
    names = ("q", "k", "v", "a", "beta", "o", "dout", "dq", "dk", "dv", "da", "dbeta")
    group = Group("o = deltanet(q, k, v, a, beta) and its gradient", names,
                  ("q", "k", "v", "a", "beta", "dout"), ("o", "dq", "dk", "dv", "da", "dbeta"),
                  lambda x: L.deltanet(batch, heads, seq, *(x[n] for n in names), d=d))
    return Program("deltanet", values, [group], ["q", "k", "v", "a", "beta", "dout"],
                   ["o", "dq", "dk", "dv", "da", "dbeta"])


# ---- config 2 through the generated floor ------------------------------------

def _floor_row_program(name: str, rows: int, n: int, row_group) -> Program:
    """sum(f(x) .* g) and its gradient as the floor forms it: a reduction
    group over each column (its folds in phases, dx at every position and the
    column's share of the loss once), then the loss's full fold."""
    from .floor import FloorGroup

    f32 = torch.float32
    values = {
        "x": Value("x", f32, (n, rows), "input"),
        "g": Value("g", f32, (n, rows), "input"),
        "loss": Value("loss", f32, (), "result"),
        "dx": Value("dx", f32, (n, rows), "result"),
        "r": Value("r", f32, (rows,), "stored"),
    }
    g1 = FloorGroup("reduction", (n, rows), reduced=(0,), name=f"{name}: its folds and gradient")
    for v in ("x", "g", "dx"):
        g1.value(v, "f32", n * rows)
    g1.value("r", "f32", rows)
    row_group(g1, g1.load("x", (1, n)), g1.load("g", (1, n)))
    g2 = FloorGroup("reduction", (rows,), reduced=(0,), name=f"{name}: the loss")
    g2.value("r", "f32", rows)
    g2.value("loss", "f32", 1)
    g2.output("loss", g2.fold("sum", g2.load("r", (1,))).value, full=False)
    return Program(name, values, [g1.as_group(), g2.as_group()], ["x", "g"], ["loss", "dx"])


def floor_softmax_columns(rows: int, n: int) -> Program:
    """Config 2a through the generated floor: y = exp.(x .- logsumexp(x; dims = 1))
    (test/fixtures/programs.jl:8), r = sum(y .* g; dims = 1),
    dx = y .* (g .- r)."""
    def row(g, x, t):
        e = g.fold("exp", x)                        # phase 1: the column's log-sum-exp
        y = g.apply("exp", x - e.logsumexp)
        s = g.fold("sum", y * t, phase=2)           # phase 2: sum(y .* g)
        g.output("dx", y * (t - s.value), (1, n))
        g.output("r", s.value, (0, 1), full=False)
    return _floor_row_program("floor_softmax_columns", rows, n, row)


def floor_layernorm(rows: int, n: int, eps: float = 1e-5) -> Program:
    """Config 2b through the generated floor, in the program's two passes
    (test/fixtures/programs.jl:13-17, weight 1): m = sum(x)/n,
    v = sum(abs2, x .- m)/n, y = (x .- m) ./ sqrt(v + eps), r = sum(y .* g),
    dx = (g .- sum(g)/n .- y .* r/n) ./ sqrt(v + eps)."""
    def row(g, x, t):
        m = g.fold("sum", x).value / n                               # phase 1
        v = g.fold("sum", g.apply("abs2", x - m), phase=2).value / n  # phase 2
        rs = g.apply("inv", g.apply("sqrt", v + eps))
        y = (x - m) * rs
        sg = g.fold("sum", t, phase=3).value                         # phase 3
        r = g.fold("sum", y * t, phase=3).value
        g.output("dx", (t - sg / n - y * (r / n)) * rs, (1, n))
        g.output("r", r, (0, 1), full=False)
    return _floor_row_program("floor_layernorm", rows, n, row)
