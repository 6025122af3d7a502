"""Benchmark of libtempest_hip on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

The headline workload is config 2 of BASELINE.json, the one the metric's
"GB/s fused reduce" is quoted on: two compiled programs over X, G of
32768 x 8192 fp32 (the reference's 8192 x 32768 column-major arrays):
sum(softmax_columns(X) .* G) and sum(layernorm(X) .* G), each with its
gradient w.r.t. X.  A step replays both programs' captured graphs once.
``value`` = algorithmic bytes per step (read X, read G, write dX for each
program: 6 x 2^30 bytes) / seconds per step, inputs resident in HBM.

The same JSON line carries the roofline of the dominant kernel (timed with
events on the stream it runs on, inside the timed region), the CPU baseline
(the oracle's single-threaded Float32 floor on a stated sample of rows) and
the other configs' figures measured in the same run.
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for p in (ROOT, ROOT / "tempest.jl_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
BF16_PEAK = 2.5e15         # MI355X dense bf16 MFMA, flop/s
ROWS, N = 32768, 8192


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_vs_direct(target, ex, reps: int, warmup: int = 2) -> dict:
    """One step of an executable replayed as a graph and launched kernel by
    kernel, each the device time per step from events around `reps` steps
    back to back, and which of the two its capture chose from the device's
    measured dispatch costs."""
    import torch
    g = target.capture(ex.launches, graph=True)
    try:
        t_graph = target.time_graph(g, warmup, reps)
    finally:
        g.release()
    for _ in range(warmup):
        ex.execute()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        ex.execute()
    e1.record()
    torch.cuda.synchronize()
    t_direct = e0.elapsed_time(e1) * 1e-3 / reps
    return {"us_graph": t_graph * 1e6, "us_direct": t_direct * 1e6,
            "kernels": sum(l.work().kernels for l in ex.launches),
            "chosen": "graph" if ex.graphed else "direct"}


def rows_grad_exact(name: str, x, g):
    """Float64 gradient of sum(f(x) .* g) over each row of x (the reference's
    columns): f = softmax, dx = y .* (g .- sum(y .* g)); f = LayerNorm (weight
    1, bias 0, eps 1e-5), dx = (g .- mean(g) .- y .* mean(g .* y)) ./ sigma.
    The bench's own parity check on sampled rows (torch, not the oracle)."""
    import torch
    x, g = x.double(), g.double()
    if name == "softmax":
        y = torch.softmax(x, dim=1)
        return y * (g - (y * g).sum(dim=1, keepdim=True))
    mu = x.mean(dim=1, keepdim=True)
    sigma = torch.sqrt(((x - mu) ** 2).mean(dim=1, keepdim=True) + 1e-5)
    y = (x - mu) / sigma
    return (g - g.mean(dim=1, keepdim=True) - y * (g * y).mean(dim=1, keepdim=True)) / sigma


def _relative(a, b) -> float:
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def config2(target, steps: int, warmup: int):
    import torch
    import tempest_hip as th

    gen = torch.Generator(device="cuda").manual_seed(20261201)
    x = torch.randn(ROWS, N, device="cuda", generator=gen)
    g = torch.randn(ROWS, N, device="cuda", generator=gen)
    cs = th.compile(th.programs.softmax_columns(ROWS, N), target, x, g)
    cl = th.compile(th.programs.layernorm(ROWS, N), target, x, g)
    es, el = cs.executable, cl.executable
    for _ in range(warmup):
        es.replay()
        el.replay()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    t0 = time.perf_counter()
    for e in ev:
        e[0].record()
        es.replay()
        e[1].record()
        el.replay()
        e[2].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    s_soft = sum(e[0].elapsed_time(e[1]) for e in ev) / steps * 1e-3
    s_ln = sum(e[1].elapsed_time(e[2]) for e in ev) / steps * 1e-3
    step_s = (t1 - t0) / steps
    bytes_soft, _ = es.work()
    bytes_ln, _ = el.work()
    # Algorithmic bytes: X, G read and dX written per program (the loss's
    # per-row partials are 1/8192 of that and counted in work() too).
    alg = 3.0 * 4 * ROWS * N
    # A quick parity check on sampled rows (outside the timed region).
    parity = {}
    try:
        idx = torch.tensor([0, 777, 16384, ROWS - 1], device="cuda")
        xs, gs = x.index_select(0, idx), g.index_select(0, idx)
        for name, ex in (("softmax", es), ("layernorm", el)):
            _, dx = ex.outputs()
            parity[name] = _relative(dx.index_select(0, idx), rows_grad_exact(name, xs, gs))
    except Exception as err:  # the bench's number stands without it
        parity["error"] = repr(err)
    dispatch = {"softmax": graph_vs_direct(target, es, steps), "layernorm": graph_vs_direct(target, el, steps)}
    return dict(x=x, g=g, step_s=step_s, s_soft=s_soft, s_ln=s_ln, alg=alg, bytes_soft=bytes_soft,
                bytes_ln=bytes_ln, parity=parity, dispatch=dispatch, describe=es.explain() + "\n" + el.explain())


def config2_floor(target, x, g, steps: int = 10, warmup: int = 3):
    """Config 2's programs through the generated floor (kernels written from
    the groups' terms and compiled at run time), on the same X, G: per-program
    device time and GB/s of the same algorithmic bytes, and sampled-row parity."""
    import torch
    import tempest_hip as th

    out = {}
    alg = 3.0 * 4 * ROWS * N
    for name, make in (("softmax", th.programs.floor_softmax_columns), ("layernorm", th.programs.floor_layernorm)):
        c = th.compile(make(ROWS, N), target, x, g)
        ex = c.executable
        for _ in range(warmup):
            ex.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            ex.replay()
        e1.record()
        torch.cuda.synchronize()
        s = e0.elapsed_time(e1) * 1e-3 / steps
        entry = {"us": s * 1e6, "GB/s": alg / s / 1e9, "frac_of_hbm_peak": alg / s / HBM_PEAK,
                 "plan": ex.explain().splitlines()[1].strip()[:400]}
        try:
            idx = torch.tensor([0, 777, 16384, ROWS - 1], device="cuda")
            entry["parity_rel"] = _relative(ex.outputs()[1].index_select(0, idx),
                                            rows_grad_exact(name, x.index_select(0, idx), g.index_select(0, idx)))
        except Exception as err:
            entry["parity_rel"] = repr(err)
        out[name] = entry
        del c, ex
    # A scan through the floor: y = cumsum(x; dims = 1) over the same X, a
    # workgroup per column (read x, write y: 8 bytes an element).
    from tempest_hip.floor import FloorGroup
    sg = FloorGroup("scan", (N, ROWS), reduced=(0,), name="cumsum(x; dims = 1)")
    sg.value("x", "f32", ROWS * N)
    sg.value("y", "f32", ROWS * N)
    sg.output("y", sg.fold("sum", sg.load("x", (1, N)), scan="inclusive").value, (1, N))
    y = torch.empty_like(x)
    sl = sg.build({"x": x.data_ptr(), "y": y.data_ptr()})
    sl()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        sl()
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / steps
    idx = torch.tensor([0, 16384, ROWS - 1], device="cuda")
    ref = torch.cumsum(x.index_select(0, idx).double(), dim=1)
    out["cumsum_scan"] = {"us": t * 1e6, "GB/s": 8.0 * ROWS * N / t / 1e9, "plan": sg.source().splitlines()[0][22:],
                          "parity_rel": float((y.index_select(0, idx).double() - ref).norm() / ref.norm())}
    del y
    out["note"] = ("generated floor: one reduction group per program (the column's folds in phases, loads kept in "
                   "registers, dx written once) and the loss's full fold; events bracket both launches; "
                   "cumsum_scan: a scan group over the same X")
    return out


def cpu_baseline(x, g, budget_s: float = 10.0):
    """The oracle's Float32 floor (oracle/floor.c, one thread) over the whole
    X, G (both programs, all 32768 rows, 1024 at a time), repeated until the
    budget is spent."""
    from oracle import floor

    xs, gs = x.cpu().numpy(), g.cpu().numpy()
    passes, spent = 0, 0.0
    chunk = 1024
    while spent < budget_s or passes == 0:
        t = time.perf_counter()
        for r in range(0, ROWS, chunk):
            floor.softmax_grad(xs[r:r + chunk], gs[r:r + chunk])
            floor.layernorm_grad(xs[r:r + chunk], gs[r:r + chunk])
        spent += time.perf_counter() - t
        passes += 1
        if passes >= 8:
            break
    step_s = spent / passes
    rate = 2 * 3.0 * 4 * ROWS * N / step_s / 1e9
    return {"value": rate, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle/floor.c (the reference's CPU floor restated in C, -O2, 1 thread): both programs "
                      f"over all {ROWS} rows, {passes} passes ({spent:.1f} s)",
            "seconds_full_step": step_s}


def host_info() -> dict:
    """The GPU box's host as the CPU baselines ran on it: logical CPUs the
    process may use (nproc), those the machine has, and the CPU model."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": len(os.sched_getaffinity(0)), "cpus_online": os.cpu_count(), "cpu_model": model}


def _one_thread():
    from threadpoolctl import threadpool_limits
    return threadpool_limits(1)


def cpu_config1(reps: int = 2000):
    """Config 1 on one core: the floor's order (oracle/floor.c), microseconds a step."""
    import numpy as np
    from oracle import floor
    rng = np.random.default_rng(1)
    w, b, x = rng.standard_normal((32, 64)), rng.standard_normal(64), rng.standard_normal((32, 16))
    floor.tanh_layer_grad(w, b, x)
    t = time.perf_counter()
    for _ in range(reps):
        floor.tanh_layer_grad(w, b, x)
    s = (time.perf_counter() - t) / reps
    return {"value": s * 1e6, "unit": "us/step", "cores": 1, "kind": "port",
            "sample": f"oracle/floor.c tanh_layer_grad, {reps} steps (host wrappers included)"}


def cpu_config3(cols: int = 4):
    """Config 3's six products on one core, each on `cols` of its output
    columns (every element a sequential fp32 fold over bf16 factors, the
    floor's order), extrapolated by the columns: the products are 2mnk flops
    each and their elements independent, so the slice's share of the work is
    exactly cols / n.  The fused element-wise work is left out (< 0.1 %)."""
    import numpy as np
    from oracle import floor
    rng = np.random.default_rng(3)
    batch, d_in, hidden, d_out = 4096, 4096, 16384, 4096
    # Operand bits for timing: normal values truncated to bf16, one buffer
    # large enough for every product's A (its contents do not change the work).
    pool = (rng.standard_normal(hidden * d_in, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)

    def bits(n):
        return pool[:n]
    # (m, n, k, A layout (a_m, a_k) with A m x k stored as the product reads it, B k-contiguous)
    shapes = [("Z1 = W1 x", hidden, batch, d_in, (1, hidden)), ("y = W2 H", d_out, batch, hidden, (1, d_out)),
              ("dW2 = dy H'", d_out, hidden, batch, (1, d_out)), ("dZ1 = W2' dy", hidden, batch, d_out, (d_out, 1)),
              ("dW1 = dZ1 x'", hidden, d_in, batch, (1, hidden)), ("dx = W1' dZ1", d_in, batch, hidden, (hidden, 1))]
    total, spent, flops_done = 0.0, 0.0, 0.0
    for name, m, n, k, (a_m, a_k) in shapes:
        a = bits(m * k)
        b = bits(k * cols)
        t = time.perf_counter()
        floor.matmul_bf16(a, a_m, a_k, b, 1, k, m, k, 0, cols)
        dt = time.perf_counter() - t
        spent += dt
        flops_done += 2.0 * m * k * cols
        total += dt * n / cols
    return {"value": 6 * 2.0 * batch * hidden * d_in / total / 1e9, "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle/floor.c matmul_bf16: {cols} output columns of each of the six products "
                      f"({flops_done / 1e9:.2f} GFLOP in {spent:.1f} s), extrapolated by n / {cols}",
            "seconds_full_step_extrapolated": total}


def cpu_config4(step: int = 4):
    """Config 4 on one core: forward and backward of one (batch, head) for
    every `step`-th query (oracle/floor.c attention_sample, the program's
    folds in sequence), extrapolated by (query, key) pairs: the work of a
    query is proportional to the keys it sees, so the full step is the
    sample's time x (all pairs / sampled pairs) x batch x heads."""
    import numpy as np
    from oracle import floor
    B, H, S, D = 8, 16, 4096, 128
    rng = np.random.default_rng(4)
    q, k, v, g = ((rng.standard_normal((S, D), dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)
                  for _ in range(4))
    t = time.perf_counter()
    floor.attention_sample(q, k, v, g, 1 / np.sqrt(D), 0, step)
    dt = time.perf_counter() - t
    sampled = sum(i + 1 for i in range(0, S, step))
    pairs = S * (S + 1) // 2
    total = dt * pairs / sampled * B * H
    flops = 4 * B * H * S * S * D / 2 * 3.5
    return {"value": flops / total / 1e9, "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle/floor.c attention_sample: one (batch, head), every {step}th query "
                      f"({sampled} of {pairs} pairs, {dt:.1f} s), extrapolated by pairs x {B * H}",
            "seconds_full_step_extrapolated": total}


def cpu_config5():
    """Config 5 on one core: the oracle's chunked DeltaNet forward and
    gradient (oracle/interpret.py, float64, BLAS held to one thread) for one
    (batch, head) sequence, times batch x heads (the sequences are independent)."""
    import numpy as np
    from oracle import interpret
    B, H, T = 4, 16, 8192
    rng = np.random.default_rng(5)
    unit = lambda x: x / np.linalg.norm(x, axis=-1, keepdims=True)  # noqa: E731
    q, k = unit(rng.standard_normal((1, T, 1, 128))), unit(rng.standard_normal((1, T, 1, 128)))
    v, do = rng.standard_normal((1, T, 1, 128)), rng.standard_normal((1, T, 1, 128))
    a = -np.logaddexp(0, rng.standard_normal((1, T, 1)))
    beta = 1 / (1 + np.exp(-rng.standard_normal((1, T, 1))))
    with _one_thread():
        t = time.perf_counter()
        interpret.deltanet_grad(q, k, v, a, beta, do)
        dt = time.perf_counter() - t
    return {"value": dt * B * H * 1e3, "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"oracle/interpret.py deltanet_grad (chunked, float64, one BLAS thread): one (batch, head) "
                      f"sequence of {T} in {dt:.2f} s, times {B * H}",
            "seconds_full_step_extrapolated": dt * B * H}


def config1(target):
    import torch
    import tempest_hip as th

    gen = torch.Generator(device="cuda").manual_seed(1)
    w = torch.randn(64, 32, device="cuda", generator=gen)   # Julia w 32 x 64
    b = torch.randn(64, device="cuda", generator=gen)
    x = torch.randn(16, 32, device="cuda", generator=gen)   # Julia x 32 x 16
    comp = th.compile(th.programs.tanh_layer(), target, w, b, x)
    ex = comp.executable
    dispatch = graph_vs_direct(target, ex, reps=2000, warmup=20)
    for _ in range(50):
        comp(w, b, x)
    torch.cuda.synchronize()
    n = 500
    t = time.perf_counter()
    for _ in range(n):
        comp(w, b, x)  # point, replay, copy dw/db/dx, read the loss
    call_s = (time.perf_counter() - t) / n
    return {"us_per_step_graph": dispatch["us_graph"], "us_per_step_execute": dispatch["us_direct"],
            "recording": dispatch["chosen"], "us_per_compiled_call_host": call_s * 1e6,
            "note": "graph/execute: device time per step from events around 2000 back-to-back replays/runs; "
                    "compiled call: host wall time of c(w, b, x) incl. result copies and the loss read"}


def config3(target, steps: int = 20, warmup: int = 10):
    """The 2-layer MLP's gradient at 4096 / 16384 / 4096, batch 4096, bf16:
    six products, 3.299e12 flops a step."""
    import torch
    import tempest_hip as th

    batch, d_in, hidden, d_out = 4096, 4096, 16384, 4096
    gen = torch.Generator(device="cuda").manual_seed(3)
    bf = torch.bfloat16
    W1 = (torch.randn(d_in, hidden, device="cuda", generator=gen) / d_in ** 0.5).to(bf)
    b1 = (torch.randn(hidden, device="cuda", generator=gen) / d_in ** 0.5).to(bf)
    W2 = (torch.randn(hidden, d_out, device="cuda", generator=gen) / hidden ** 0.5).to(bf)
    b2 = (torch.randn(d_out, device="cuda", generator=gen) / hidden ** 0.5).to(bf)
    x = torch.randn(batch, d_in, device="cuda", generator=gen).to(bf)
    comp = th.compile(th.programs.mlp(batch, d_in, hidden, d_out), target, W1, b1, W2, b2, x)
    ex = comp.executable
    flops = 6 * 2.0 * batch * hidden * d_in
    for _ in range(warmup):
        ex.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ex.replay()
    e1.record()
    torch.cuda.synchronize()
    step_s = e0.elapsed_time(e1) * 1e-3 / steps
    per = {}
    for g, l in zip(ex.program.groups, ex.launches):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        l()
        evs[0].record()
        for _ in range(3):
            l()
        evs[1].record()
        torch.cuda.synchronize()
        s = evs[0].elapsed_time(evs[1]) * 1e-3 / 3
        per[g.name] = {"us": s * 1e6, "TFLOP/s": l.work().flops / s / 1e12}
    return {"ms_per_step": step_s * 1e3, "TFLOP/s": flops / step_s / 1e12,
            "frac_of_bf16_peak": flops / step_s / BF16_PEAK, "flops_per_step": flops, "per_launch": per,
            "dispatch": graph_vs_direct(target, ex, steps)}


def config4(target, steps: int = 10, warmup: int = 5, recompute_dq: bool = False):
    """Causal attention fwd+bwd, B8 H16 S4096 D128 bf16: 1.924e12 flops a step
    (forward 4 B H S^2 D / 2, backward 2.5x that).  recompute_dq: the
    backward's dQ sweep recomputes S and dP rather than reading stored dS'."""
    import torch
    import tempest_hip as th

    B, H, S, D = 8, 16, 4096, 128
    gen = torch.Generator(device="cuda").manual_seed(4)
    q, k, v, g = (torch.randn(B, S, H, D, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
    comp = th.compile(th.programs.attention(B, H, S, recompute_dq=recompute_dq), target, q, k, v, g)
    ex = comp.executable
    fwd, bwd = ex.launches
    f_fwd, f_bwd = fwd.work().flops, bwd.work().flops
    for _ in range(warmup):
        ex.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    t_f = t_b = 0.0
    for _ in range(steps):
        ev[0].record()
        fwd()
        ev[1].record()
        bwd()
        ev[2].record()
        torch.cuda.synchronize()
        t_f += ev[0].elapsed_time(ev[1]) * 1e-3
        t_b += ev[1].elapsed_time(ev[2]) * 1e-3
    t_f /= steps
    t_b /= steps
    total = f_fwd + f_bwd
    dispatch = graph_vs_direct(target, ex, reps=3, warmup=1)
    return {"ms_per_step": (t_f + t_b) * 1e3, "TFLOP/s": total / (t_f + t_b) / 1e12, "dispatch": dispatch,
            "frac_of_bf16_peak": total / (t_f + t_b) / BF16_PEAK, "flops_per_step": total,
            "fwd": {"ms": t_f * 1e3, "TFLOP/s": f_fwd / t_f / 1e12},
            "bwd": {"ms": t_b * 1e3, "TFLOP/s": f_bwd / t_b / 1e12,
                    "note": "FA2 convention, 2.5x forward flops; deterministic: " +
                            ("the dQ sweep recomputes S and dP" if recompute_dq else
                             "the dK/dV sweep stores dS, a dQ sweep reads it")}}


def attention_head_dims(target, steps: int = 3, warmup: int = 1):
    """Causal attention forward + backward at B8 H16 S4096 with head dims 64
    and 256 (the matrix-core kernels for head dims other than the tuned
    128), bf16, and 128 at S4095, a length the tuned kernels do not take.
    TFLOP/s counts the FA2 flops of the visible (query, key) pairs:
    forward 4 D pairs per (batch, head), backward 2.5x that."""
    import torch
    import tempest_hip.launch as L
    out = {}
    for D, S in ((64, 4096), (256, 4096), (128, 4095)):
        B, H = 8, 16
        gen = torch.Generator(device="cuda").manual_seed(40 + D)
        q, k, v, g = (torch.randn(B, S, H, D, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(4))
        o, lse = torch.empty_like(q), torch.empty(B, S, H, device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        fwd = L.attention_fwd(B, H, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              causal=True, head_dim=D)
        bwd = L.attention_bwd(B, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              g.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), causal=True, head_dim=D)
        for _ in range(warmup):
            fwd()
            bwd()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        t_f = t_b = 0.0
        for _ in range(steps):
            ev[0].record()
            fwd()
            ev[1].record()
            bwd()
            ev[2].record()
            torch.cuda.synchronize()
            t_f += ev[0].elapsed_time(ev[1]) * 1e-3 / steps
            t_b += ev[1].elapsed_time(ev[2]) * 1e-3 / steps
        ff, fb = fwd.work().flops, bwd.work().flops
        out[f"B{B}_H{H}_S{S}_d{D}_causal"] = {
            "fwd": {"ms": t_f * 1e3, "TFLOP/s": ff / t_f / 1e12}, "bwd": {"ms": t_b * 1e3, "TFLOP/s": fb / t_b / 1e12},
            "ms_per_step": (t_f + t_b) * 1e3, "TFLOP/s": (ff + fb) / (t_f + t_b) / 1e12,
            "frac_of_bf16_peak": (ff + fb) / (t_f + t_b) / BF16_PEAK, "kernels": [fwd.describe(), bwd.describe()]}
        log(f"attention d{D} S{S}:", json.dumps({kk: out[f"B{B}_H{H}_S{S}_d{D}_causal"][kk]
                                                 for kk in ("ms_per_step", "TFLOP/s")}))
    return out


def gemm_tiles(target, runs: int = 20):
    """The product's tile choices (not a config of its own): for each shape,
    every kernel that takes it at the split the library would choose, timed as
    claims are (th_time_launch), then run `runs` times back to back so a
    kernel trace or counter run sees each variant by its kernel's name; and
    what th_gemm_tune chose.  bf16 factors, A k-contiguous, B n-contiguous,
    an fp32 result."""
    import torch
    import tempest_hip.launch as L
    gen = torch.Generator(device="cuda").manual_seed(7)
    out = {}
    for m, n, k in ((512, 512, 512), (1024, 1024, 1024), (2048, 2048, 1024), (256, 256, 8192), (4096, 4096, 4096)):
        a = torch.randn(m, k, device="cuda", generator=gen).to(torch.bfloat16)  # A(i, l) at i k + l
        b = torch.randn(k, n, device="cuda", generator=gen).to(torch.bfloat16)  # B(l, j) at l n + j
        c = torch.empty(n, m, device="cuda")
        args = (m, n, k, a.data_ptr(), k, 1, b.data_ptr(), n, 1, c.data_ptr(), m)
        flops = 2.0 * m * n * k
        row = {}
        for tile in (L.TILE_256, L.TILE_128X128, L.TILE_128X64, L.TILE_64X128, L.TILE_64X64, L.TILE_GENERAL):
            try:
                launch = L.gemm(*args, c_dtype=L.F32, tile=tile)
            except Exception:  # the kernel does not take the shape
                continue
            t = target.time_launch(launch)
            for _ in range(runs):
                launch()
            torch.cuda.synchronize()
            row[L.TILE_NAMES[tile]] = {"us": t * 1e6, "TFLOP/s": flops / t / 1e12,
                                       "workgroups": launch.work().blocks, "kernels": launch.describe()}
        tile, splits, t = L.gemm_tune(*args, c_dtype=L.F32)
        row["chosen"] = {"tile": L.TILE_NAMES[tile], "splits": splits, "us": t * 1e6, "TFLOP/s": flops / t / 1e12}
        out[f"{m}x{n}x{k}"] = row
        log(f"gemm tiles {m}x{n}x{k}:", json.dumps(row["chosen"]))
    out["fp32"] = gemm_f32_rows(target, runs)
    return out


def gemm_f32_rows(target, runs: int = 20):
    """fp32 factors: in full precision on the fp32 matrix cores (the 128 x 128
    kernel, K split where the tiles alone do not fill the device) and as split
    bf16 (bf16x3) on the bf16 tile kernels; each timed as claims are
    (th_time_launch), then run `runs` times for a kernel trace.  A k-contiguous,
    B n-contiguous, an fp32 result.  TFLOP/s counts the fp32 product's 2mnk."""
    import torch
    import tempest_hip.launch as L
    gen = torch.Generator(device="cuda").manual_seed(8)
    out = {}
    for m, n, k in ((4096, 4096, 4096), (256, 256, 8192), (1024, 1024, 1024)):
        a = torch.randn(m, k, device="cuda", generator=gen)
        b = torch.randn(k, n, device="cuda", generator=gen)
        c = torch.empty(n, m, device="cuda")
        args = (m, n, k, a.data_ptr(), k, 1, b.data_ptr(), n, 1, c.data_ptr(), m)
        flops = 2.0 * m * n * k
        row = {}
        for name, kw in (("full", {}), ("bf16x3", {"bf16x3": True})):
            launch = L.gemm(*args, c_dtype=L.F32, factors=L.F32, **kw)
            t = target.time_launch(launch)
            for _ in range(runs):
                launch()
            torch.cuda.synchronize()
            row[name] = {"us": t * 1e6, "TFLOP/s": flops / t / 1e12, "workgroups": launch.work().blocks,
                         "kernels": launch.describe()}
            # Norm-wise error against the float64 product (torch's, as the checker).
            want = (a.double() @ b.double()).T
            row[name]["rel_err_vs_f64"] = float((c.double() - want).norm() / want.norm())
        out[f"{m}x{n}x{k}"] = row
        log(f"gemm fp32 {m}x{n}x{k}:", json.dumps({kk: v["TFLOP/s"] for kk, v in row.items()}))
    return out


def config5(target, steps: int = 10, warmup: int = 5):
    """Chunked gated DeltaNet forward + gradient, B4 H16 T8192, d 128, chunk 64."""
    import torch
    import tempest_hip as th

    B, H, T = 4, 16, 8192
    gen = torch.Generator(device="cuda").manual_seed(5)
    r = lambda *s: torch.randn(*s, device="cuda", generator=gen)  # noqa: E731
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)  # noqa: E731
    q, k = unit(r(B, T, H, 128)).to(torch.bfloat16), unit(r(B, T, H, 128)).to(torch.bfloat16)
    v, do = r(B, T, H, 128).to(torch.bfloat16), r(B, T, H, 128).to(torch.bfloat16)
    a = (-torch.nn.functional.softplus(r(B, T, H))).contiguous()
    beta = torch.sigmoid(r(B, T, H)).contiguous()
    comp = th.compile(th.programs.deltanet(B, H, T), target, q, k, v, a, beta, do)
    ex = comp.executable
    (l,) = ex.launches
    w = l.work()
    for _ in range(warmup):
        ex.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ex.replay()
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) * 1e-3 / steps
    dispatch = graph_vs_direct(target, ex, reps=3, warmup=1)
    return {"ms_per_step": s * 1e3, "TFLOP/s": w.flops / s / 1e12, "GB/s": w.bytes / s / 1e9, "dispatch": dispatch,
            "flops_per_step": w.flops, "bytes_per_step": w.bytes,
            "note": "fp32 products as split bf16 on the matrix cores (chunk prep, column-split state scan, outputs, reverse "
                    "state-gradient scan, chunk-local backward); flops/bytes are the algorithmic estimates of "
                    "th_launch_work"}


def matrix_rate(target) -> dict:
    """The matrix cores' sustained bf16 rate on this device (th_matrix_rate):
    register-only products on every SIMD, with one operand pair throughout
    and with random operands changing every product, and the shader clock
    the waves ran at.  The ceiling a product kernel's data meets here."""
    import ctypes
    from tempest_hip import _lib
    out = {}
    for name, vary in (("constant_operands", 0), ("random_operands", 1)):
        f, c = ctypes.c_double(), ctypes.c_double()
        _lib.call("th_matrix_rate", vary, ctypes.byref(f), ctypes.byref(c))
        out[name] = {"PFLOP/s": f.value / 1e15, "frac_of_bf16_peak": f.value / BF16_PEAK, "clock_GHz": c.value / 1e9}
    log("matrix rate:", json.dumps(out))
    return out


def lds_rate(target) -> dict:
    """The LDS read rate on this device (th_lds_rate): ds_read_b128 and
    ds_read_b64_tr_b16 at one and two workgroups of four waves a CU, alone
    and with one product per 1 KB read (32 flops a byte, the attention
    sweeps' ratio), in bytes a clock a CU at the clock the waves ran at."""
    import ctypes
    from tempest_hip import _lib
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = {}
    for mode, name in ((0, "b128"), (1, "tr_b64_pairs"), (2, "b128_with_products"), (3, "tr_b64_pairs_with_products")):
        for per_cu in (1, 2):
            b, f, c = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
            _lib.call("th_lds_rate", mode, per_cu, ctypes.byref(b), ctypes.byref(f), ctypes.byref(c))
            row = {"TB/s": b.value / 1e12, "B/clk/CU": b.value / c.value / cus, "clock_GHz": c.value / 1e9}
            if mode >= 2:
                row["PFLOP/s"] = f.value / 1e15
            out[f"{name}_{per_cu}wg"] = row
    log("lds rate:", json.dumps(out))
    return out


def read_rate(target) -> dict:
    """The HBM read rate on this device (th_read_rate): one workgroup of four
    waves a CU, eight 1 KB loads in flight a wave, over a 2 MB stream a wave
    and over the attention dQ sweep's dS' reads at config 4's shape."""
    import ctypes
    from tempest_hip import _lib
    out = {}
    for mode, name in ((0, "stream_2MB_a_wave"), (1, "dq_sweep_dS_reads")):
        b = ctypes.c_double()
        _lib.call("th_read_rate", mode, ctypes.byref(b))
        out[name] = {"TB/s": b.value / 1e12}
    log("read rate:", json.dumps(out))
    return out


# The reference's own recorded times (NVIDIA GB10, µs) for the programs
# reference_benchmarks runs: TRIALS.md:2155-2158 (bf16 attention forward and
# training step, the later of its records), :2183-2187 (TF32), and
# test/bench/coverage-NVIDIA_GB10.tsv (the coverage compositions of
# test/fixtures/compositions.jl).
REFERENCE_US = {
    "attention_bf16_D64_H8_B2_S1024_causal": {"fwd": 36.2, "step": 191.0},
    "attention_bf16_D64_H8_B2_S2048_causal": {"fwd": 123.7, "step": 597.0},
    "attention_f32_D64_H8_B2_S1024_causal": {"fwd": 95.0, "step": 410.0},
    "attention_f32_D64_H8_B2_S2048_causal": {"fwd": 330.0, "step": 1408.0},
    "attention_f32_D64_H4_S256_B2_causal": {"fwd": 123.61, "step": 195.41},
    "softmax_through_logsumexp_512x1024": {"fwd": 5.56},
    "layer_norm_two_passes_512x1024": {"fwd": 10.07},
    "rmsnorm_divided_by_the_root_512x1024": {"fwd": 9.89},
    "rmsnorm_times_the_inverse_root_512x1024": {"fwd": 9.78},
    "layer_norm_from_the_mean_of_squares_512x1024": {"fwd": 9.99},
    "softmax_shifted_by_the_maximum_512x1024": {"fwd": 5.69},
    "softmax_exp_computed_once_512x1024": {"fwd": 4.94},
    "rmsnorm_training_step_512x1024": {"step": 13.88},
    "linear_bias_gelu_256x384x512_f32": {"fwd": 13.44},
}


def _graph_step_us(launches, samples: int = 15, milliseconds: float = 4.0) -> float:
    """Device microseconds of one step of `launches`, as the reference's coverage
    bench takes it (test/bench/coverage.jl:21-28): the step captured enough times
    into one graph to run a few milliseconds, the minimum over samples of one
    replay's device time over the repetitions."""
    import ctypes
    from tempest_hip import _lib
    for l in launches:
        l()  # workspaces are taken at the first run
    def timed(reps: int, warm: int, n: int) -> list[float]:
        hs = [l.handle.value for l in launches] * reps
        g = ctypes.c_void_p()
        _lib.call("th_graph_capture", (ctypes.c_void_p * len(hs))(*hs), len(hs), ctypes.byref(g))
        try:
            out = []
            for i in range(n):
                sec = ctypes.c_double()
                _lib.call("th_time_graph", g, warm if i == 0 else 0, 1, ctypes.byref(sec))
                out.append(sec.value / reps)
            return out
        finally:
            _lib.call("th_graph_release", g)
    once = min(timed(1, 3, 3))
    reps = max(1, min(200, round(milliseconds * 1e-3 / once)))
    return min(timed(reps, 1, samples)) * 1e6


def reference_benchmarks(target) -> dict:
    """This path's programs at the shapes the reference itself times, beside
    the reference's recorded times on its GB10 (REFERENCE_US): causal attention
    (64 features, one key head per query head) forward and training step
    (loss = sum(abs2, o): o, the loss and dO = 2o by one floor group, then the
    backward) in bf16 and fp32 (the reference's numbers at fp32 are TF32), the
    coverage suite's attention (64 x 4 heads x 256 positions x 2, fp32) and its
    column programs over a 512 x 1024 fp32 matrix (softmax through logsumexp,
    the two-pass layer norm and RMSNorm with a weight, and linear, bias, GELU at
    256 x 384 x 512 in fp32, test/fixtures/compositions.jl:41-138).  Inputs are
    the reference's sample(dims; scale) = 2 sin(scale (1:prod(dims)))
    (compositions.jl:36).  Each result is checked against float64 torch:
    rel_err = |ours - exact| / |exact| over the output (attention: o, dq, dk, dv)."""
    import torch
    import tempest_hip.launch as L
    from tempest_hip.floor import FloorGroup

    def sample(n, scale, dtype):
        return (2.0 * torch.sin(scale * torch.arange(1, n + 1, device="cuda", dtype=torch.float64))).to(dtype)

    def rel(a, b):
        a, b = a.detach().double(), b.detach().double()
        return float((a - b).norm() / b.norm())

    out = {}
    # ---- attention
    shapes = [("bf16", 64, 8, 2, 1024, (0.1, 0.2, 0.3)), ("bf16", 64, 8, 2, 2048, (0.1, 0.2, 0.3)),
              ("f32", 64, 8, 2, 1024, (0.1, 0.2, 0.3)), ("f32", 64, 8, 2, 2048, (0.1, 0.2, 0.3)),
              ("f32", 64, 4, 2, 256, (0.1, 0.2, 0.3))]
    for dt, D, H, B, S, scales in shapes:
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        n = D * H * S * B
        q, k, v = (sample(n, sc, tdt).view(B, S, H, D) for sc in scales)  # (d, heads, positions, batch)
        o, g = torch.empty_like(q), torch.empty_like(q)
        lse = torch.empty(B, S, H, device="cuda")
        loss = torch.zeros(1, device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        f32 = dt == "f32"
        fwd = L.attention_fwd(B, H, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              causal=True, head_dim=D, f32=f32)
        lg = FloorGroup("reduction", (n,), reduced=(0,), name="loss = sum(abs2, o), dO = 2o")
        lg.value("o", dt, n)
        lg.value("g", dt, n)
        lg.value("loss", "f32", 1)
        oo = lg.load("o", (1,))
        lg.output("g", oo * 2.0, (1,))
        lg.output("loss", lg.fold("sum", lg.apply("abs2", oo)).value, full=False)
        lossl = lg.build({"o": o.data_ptr(), "g": g.data_ptr(), "loss": loss.data_ptr()})
        bwd = L.attention_bwd(B, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                              g.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), causal=True, head_dim=D,
                              f32=f32)
        t_fwd = _graph_step_us([fwd])
        t_step = _graph_step_us([fwd, lossl, bwd])
        fwd(), lossl(), bwd()
        torch.cuda.synchronize()
        # float64 reference: loss = sum(abs2, attention(q, k, v)) and its gradients.
        qq, kk, vv = (t.double().permute(0, 2, 1, 3).contiguous().requires_grad_(True) for t in (q, k, v))
        sc = qq @ kk.transpose(-1, -2).contiguous() / D ** 0.5
        mask = torch.ones(S, S, device="cuda", dtype=torch.bool).triu(1)
        p = torch.softmax(sc.masked_fill(mask, float("-inf")), dim=-1)
        oref = p @ vv
        (oref * oref).sum().backward()
        back = lambda t: t.permute(0, 2, 1, 3)  # noqa: E731
        name = f"attention_{dt}_D{D}_H{H}_B{B}_S{S}_causal" if H == 8 else f"attention_{dt}_D{D}_H{H}_S{S}_B{B}_causal"
        ref = REFERENCE_US[name]
        out[name] = {"us_fwd": t_fwd, "us_step": t_step, "reference_us_gb10": ref,
                     "speedup_fwd": ref["fwd"] / t_fwd, "speedup_step": ref["step"] / t_step,
                     "rel_err": {"o": rel(o, back(oref)), "dq": rel(dq, back(qq.grad)), "dk": rel(dk, back(kk.grad)),
                                 "dv": rel(dv, back(vv.grad))},
                     "kernels": [fwd.describe(), bwd.describe()]}
        for l in (fwd, lossl, bwd):
            l.destroy()
        del qq, kk, vv, sc, p, oref
        log(name, json.dumps({kk_: out[name][kk_] for kk_ in ("us_fwd", "us_step", "speedup_fwd", "speedup_step")}))
    # ---- column programs over X (512 x 1024), w (512)
    N, M = 512, 1024
    x = sample(N * M, 0.3, torch.float32)
    w = sample(N, 0.1, torch.float32)
    y = torch.empty_like(x)
    X, Wt = x.double().view(M, N).T, w.double()  # Julia's N x M, column-major
    def col_group(name):
        g = FloorGroup("reduction", (N, M), reduced=(0,), name=name)
        g.value("x", "f32", N * M)
        g.value("w", "f32", N)
        g.value("y", "f32", N * M)
        return g, g.load("x", (1, N)), g.load("w", (1, 0))
    progs = {}
    g, xx, ww = col_group("softmax through logsumexp")
    g.output("y", g.apply("exp", xx - g.fold("exp", xx).logsumexp), (1, N))
    progs["softmax_through_logsumexp_512x1024"] = (g, torch.softmax(X, dim=0))
    g, xx, ww = col_group("layer norm, two passes")
    m = g.fold("sum", xx).value / float(N)
    var = g.fold("sum", g.apply("abs2", xx - m), phase=2).value / float(N)
    g.output("y", (xx - m) / g.apply("sqrt", var + 1e-5) * ww, (1, N))
    mu = X.mean(dim=0, keepdim=True)
    progs["layer_norm_two_passes_512x1024"] = (
        g, (X - mu) / torch.sqrt(((X - mu) ** 2).mean(dim=0, keepdim=True) + 1e-5) * Wt[:, None])
    g, xx, ww = col_group("RMSNorm, divided by the root")
    g.output("y", xx / g.apply("sqrt", g.fold("sum", g.apply("abs2", xx)).value / float(N) + 1e-5) * ww, (1, N))
    progs["rmsnorm_divided_by_the_root_512x1024"] = (
        g, X / torch.sqrt((X ** 2).sum(dim=0, keepdim=True) / N + 1e-5) * Wt[:, None])
    g, xx, ww = col_group("RMSNorm, times the inverse root")
    g.output("y", ww * xx * g.apply("inv", g.apply("sqrt", g.fold("sum", xx * xx).value * (1.0 / N) + 1e-5)), (1, N))
    progs["rmsnorm_times_the_inverse_root_512x1024"] = (
        g, X / torch.sqrt((X ** 2).sum(dim=0, keepdim=True) / N + 1e-5) * Wt[:, None])
    g, xx, ww = col_group("layer norm, from the mean of squares")
    m = g.fold("sum", xx).value / float(N)
    var = g.fold("sum", xx * xx).value / float(N) - m * m  # x .^ 2: Julia's literal power is x * x
    g.output("y", ww * (xx - m) / g.apply("sqrt", var + 1e-5), (1, N))
    progs["layer_norm_from_the_mean_of_squares_512x1024"] = (
        g, (X - mu) / torch.sqrt(((X - mu) ** 2).mean(dim=0, keepdim=True) + 1e-5) * Wt[:, None])
    g, xx, ww = col_group("softmax shifted by the maximum")
    mx = g.fold("max", xx).value
    e = g.apply("exp", xx - mx)
    g.output("y", e / g.fold("sum", e, phase=2).value, (1, N))
    progs["softmax_shifted_by_the_maximum_512x1024"] = (g, torch.softmax(X, dim=0))
    g, xx, ww = col_group("softmax, exp computed once")
    e = g.apply("exp", xx)
    g.output("y", e / g.fold("sum", e).value, (1, N))
    progs["softmax_exp_computed_once_512x1024"] = (g, torch.softmax(X, dim=0))
    for name, (g, exact) in progs.items():
        l = g.build({"x": x.data_ptr(), "w": w.data_ptr(), "y": y.data_ptr()})
        t = _graph_step_us([l])
        l()
        torch.cuda.synchronize()
        out[name] = {"us_fwd": t, "reference_us_gb10": REFERENCE_US[name], "speedup_fwd": REFERENCE_US[name]["fwd"] / t,
                     "rel_err": rel(y.view(M, N).T, exact)}
        l.destroy()
        log(name, json.dumps({kk_: out[name][kk_] for kk_ in ("us_fwd", "speedup_fwd", "rel_err")}))
    # ---- RMSNorm, a training step: loss = sum(abs2, rmsnorm(x, w)) and (dx, dw).  Per column c,
    # r = (sum(x^2)/N + eps)^(-1/2), y = x r w, L_c = sum(y^2), dx = 2 r w y - 2 r^2 L_c x / N;
    # dw = sum over columns of 2 x^2 r^2 w; loss = sum L_c.  Three groups: the columns, the rows, the loss.
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    rcol, lcol, loss1 = torch.empty(M, device="cuda"), torch.empty(M, device="cuda"), torch.empty(1, device="cuda")
    g1 = FloorGroup("reduction", (N, M), reduced=(0,), name="RMSNorm's columns: y, L_c, dx")
    for v_, n_ in (("x", N * M), ("w", N), ("dx", N * M), ("r", M), ("L", M)):
        g1.value(v_, "f32", n_)
    xx, ww = g1.load("x", (1, N)), g1.load("w", (1, 0))
    r = g1.apply("inv", g1.apply("sqrt", g1.fold("sum", g1.apply("abs2", xx)).value / float(N) + 1e-5))
    yv = xx * r * ww
    lc = g1.fold("sum", g1.apply("abs2", yv), phase=2).value
    g1.output("dx", 2.0 * r * ww * yv - 2.0 * r * r * lc * xx / float(N), (1, N))
    g1.output("r", r, (0, 1), full=False)
    g1.output("L", lc, (0, 1), full=False)
    g2 = FloorGroup("reduction", (N, M), reduced=(1,), name="RMSNorm's rows: dw")
    for v_, n_ in (("x", N * M), ("w", N), ("r", M), ("dw", N)):
        g2.value(v_, "f32", n_)
    xx, rr, ww = g2.load("x", (1, N)), g2.load("r", (0, 1)), g2.load("w", (1, 0))
    g2.output("dw", g2.fold("sum", 2.0 * xx * xx * rr * rr * ww).value, (1, 0), full=False)
    g3 = FloorGroup("reduction", (M,), reduced=(0,), name="RMSNorm's loss")
    g3.value("L", "f32", M)
    g3.value("loss", "f32", 1)
    g3.output("loss", g3.fold("sum", g3.load("L", (1,))).value, full=False)
    ptr = {"x": x.data_ptr(), "w": w.data_ptr(), "dx": dx.data_ptr(), "dw": dw.data_ptr(), "r": rcol.data_ptr(),
           "L": lcol.data_ptr(), "loss": loss1.data_ptr()}
    ls = [gg.build({k_: ptr[k_] for k_ in gg.values}) for gg in (g1, g2, g3)]
    t = _graph_step_us(ls)
    for l in ls:
        l()
    torch.cuda.synchronize()
    Xg, Wg = X.clone().requires_grad_(True), Wt.clone().requires_grad_(True)
    yr = Xg / torch.sqrt((Xg ** 2).sum(dim=0, keepdim=True) / N + 1e-5) * Wg[:, None]
    lr_ = (yr ** 2).sum()
    lr_.backward()
    name = "rmsnorm_training_step_512x1024"
    out[name] = {"us_step": t, "us_fwd": t, "reference_us_gb10": REFERENCE_US[name],
                 "speedup_step": REFERENCE_US[name]["step"] / t,
                 "rel_err": {"loss": rel(loss1, lr_.reshape(1)), "dx": rel(dx.view(M, N).T, Xg.grad),
                             "dw": rel(dw, Wg.grad)}}
    for l in ls:
        l.destroy()
    log(name, json.dumps({kk_: out[name][kk_] for kk_ in ("us_step", "speedup_step", "rel_err")}))
    # ---- linear, bias, GELU: gelu.(W * Z .+ b), W 256 x 384, Z 384 x 512, b 256, fp32
    m_, k_, n_ = 256, 384, 512
    Wm, Zm, bv = sample(m_ * k_, 0.01, torch.float32), sample(k_ * n_, 0.2, torch.float32), sample(m_, 0.3, torch.float32)
    c = torch.empty(m_ * n_, device="cuda")
    yo = torch.empty_like(c)
    prod = L.gemm(m_, n_, k_, Wm.data_ptr(), 1, m_, Zm.data_ptr(), 1, k_, c.data_ptr(), m_, c_dtype=L.F32,
                  factors=L.F32)
    eg = FloorGroup("pointwise", (m_, n_), name="gelu.(c .+ b)")
    eg.value("c", "f32", m_ * n_)
    eg.value("b", "f32", m_)
    eg.value("y", "f32", m_ * n_)
    z = eg.load("c", (1, m_)) + eg.load("b", (1, 0))
    eg.output("y", z / 2.0 * (1.0 + eg.apply("tanh", 0.7978846 * (z + 0.044715 * z * z * z))), (1, m_))
    epi = eg.build({"c": c.data_ptr(), "b": bv.data_ptr(), "y": yo.data_ptr()})
    t = _graph_step_us([prod, epi])
    prod(), epi()
    torch.cuda.synchronize()
    Zd = (Wm.double().view(k_, m_).T @ Zm.double().view(n_, k_).T) + bv.double()[:, None]
    exact = Zd / 2 * (1 + torch.tanh(0.7978846 * (Zd + 0.044715 * Zd ** 3)))
    name = "linear_bias_gelu_256x384x512_f32"
    out[name] = {"us_fwd": t, "reference_us_gb10": REFERENCE_US[name], "speedup_fwd": REFERENCE_US[name]["fwd"] / t,
                 "rel_err": rel(yo.view(n_, m_).T, exact), "kernels": [prod.describe(), epi.describe()]}
    prod.destroy(), epi.destroy()
    log(name, json.dumps({kk_: out[name][kk_] for kk_ in ("us_fwd", "speedup_fwd", "rel_err")}))
    return out


def dispatch_costs(target, reps: int = 2000):
    """Where a graph replay's time goes on this device: graphs of 1, 9 and 40
    near-empty launches (16-byte copies, th_build_copy), replayed back to back
    (device time per replay from events) with the host time of each
    th_graph_replay (hipGraphLaunch) call, against the same launches run
    directly (th_launch_run)."""
    import ctypes
    import torch
    from tempest_hip import _lib
    buf = torch.zeros(64, dtype=torch.uint8, device="cuda")
    out = {}
    for nodes in (1, 9, 40):
        hs = []
        for _ in range(nodes):
            h = ctypes.c_void_p()
            _lib.call("th_build_copy", buf.data_ptr() + 32, buf.data_ptr(), ctypes.c_uint64(16), ctypes.byref(h))
            hs.append(h)
        g = ctypes.c_void_p()
        _lib.call("th_graph_capture", (ctypes.c_void_p * nodes)(*[h.value for h in hs]), nodes, ctypes.byref(g))
        try:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            row = {}
            for how in ("graph", "direct"):
                for _ in range(50):
                    if how == "graph":
                        _lib.call("th_graph_replay", g)
                    else:
                        for h in hs:
                            _lib.call("th_launch_run", h)
                torch.cuda.synchronize()
                e0.record()
                t0 = time.perf_counter()
                for _ in range(reps):
                    if how == "graph":
                        _lib.call("th_graph_replay", g)
                    else:
                        for h in hs:
                            _lib.call("th_launch_run", h)
                host = (time.perf_counter() - t0) / reps
                e1.record()
                torch.cuda.synchronize()
                row[how] = {"us_device_per_step": e0.elapsed_time(e1) * 1e3 / reps, "us_host_per_step": host * 1e6}
            out[f"{nodes}_launches"] = row
        finally:
            _lib.call("th_graph_release", g)
            for h in hs:
                _lib.call("th_launch_destroy", h)
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-config2", action="store_true",
                    help="config 2 alone, no CPU baseline (for counter runs)")
    ap.add_argument("--only", choices=["config1", "config2_floor", "config3", "config4", "config4_recompute",
                                       "config5", "gemm_tiles", "gemm_f32", "dispatch", "attention_head_dims",
                                       "matrix_rate", "lds_rate", "read_rate", "reference_benchmarks"],
                    default=None,
                    help="run one other config alone and print its figures (for kernel traces and counter runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy, 10 times: the known-size kernel that "
                         "scales FETCH_SIZE / WRITE_SIZE counters to bytes")
    a = ap.parse_args()
    if a.copy_calibration:
        import torch
        src = torch.ones(2**28, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 2**30, "copy_bytes_written": 2**30, "copies": 10}))
        return 0
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for {a.gpus}); "
              "the per-GPU share shards by rows with no exchange.", file=sys.stderr)
        return 2
    import torch
    import tempest_hip as th

    target = th.HIPTarget()
    log("device:", target.device_name())
    if a.only == "config2_floor":
        gen = torch.Generator(device="cuda").manual_seed(20261201)
        x = torch.randn(ROWS, N, device="cuda", generator=gen)
        g = torch.randn(ROWS, N, device="cuda", generator=gen)
        print(json.dumps({a.only: config2_floor(target, x, g, a.steps, a.warmup)}), flush=True)
        return 0
    if a.only:
        fn = {"config1": config1, "config3": config3, "config4": config4, "config5": config5, "gemm_tiles": gemm_tiles,
              "dispatch": dispatch_costs, "gemm_f32": gemm_f32_rows, "attention_head_dims": attention_head_dims,
              "matrix_rate": matrix_rate, "lds_rate": lds_rate, "read_rate": read_rate,
              "reference_benchmarks": reference_benchmarks,
              "config4_recompute": lambda t: config4(t, recompute_dq=True)}[a.only]
        print(json.dumps({a.only: fn(target)}), flush=True)
        return 0
    c2 = config2(target, a.steps, a.warmup)
    log(c2["describe"])
    step_s = c2["step_s"]
    value = 2 * c2["alg"] / step_s / 1e9
    dominant = ("softmax_grad_resident", c2["s_soft"]) if c2["s_soft"] >= c2["s_ln"] else \
        ("layernorm_grad_resident", c2["s_ln"])
    achieved = c2["alg"] / dominant[1]
    traffic = None
    tf = ROOT / "profiles" / "traffic_config2.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get(dominant[0])
    roofline = {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": achieved / HBM_PEAK, "traffic": traffic, "kernel": dominant[0],
                "kernel_us": dominant[1] * 1e6,
                "per_kernel": {"softmax_grad": {"us": c2["s_soft"] * 1e6, "GB/s": c2["alg"] / c2["s_soft"] / 1e9},
                               "layernorm_grad": {"us": c2["s_ln"] * 1e6, "GB/s": c2["alg"] / c2["s_ln"] / 1e9}},
                "note": "per-program events bracket the fused row kernel and the loss's one-block sum"}
    configs = {"config2_parity_rel": c2["parity"], "config2_dispatch": c2["dispatch"]}
    if not a.only_config2:
        try:
            configs["config2_floor"] = config2_floor(target, c2["x"], c2["g"])
        except Exception as err:
            configs["config2_floor"] = {"error": repr(err)}
        log("config2_floor:", json.dumps(configs["config2_floor"]))
        try:
            configs["config1_tanh_layer"] = config1(target)
        except Exception as err:
            configs["config1_tanh_layer"] = {"error": repr(err)}
        try:
            configs["config3_mlp"] = config3(target)
        except Exception as err:
            configs["config3_mlp"] = {"error": repr(err)}
        try:
            configs["config3_mlp"]["matrix_rate"] = matrix_rate(target)
        except Exception as err:
            configs["config3_mlp"]["matrix_rate"] = {"error": repr(err)}
        log("config3:", json.dumps(configs["config3_mlp"]))
        try:
            configs["config4_attention"] = config4(target)
        except Exception as err:
            configs["config4_attention"] = {"error": repr(err)}
        try:
            configs["config4_attention"]["lds_rate"] = lds_rate(target)
        except Exception as err:
            configs["config4_attention"]["lds_rate"] = {"error": repr(err)}
        try:
            configs["config4_attention"]["read_rate"] = read_rate(target)
        except Exception as err:
            configs["config4_attention"]["read_rate"] = {"error": repr(err)}
        log("config4:", json.dumps(configs["config4_attention"]))
        try:
            configs["attention_head_dims"] = attention_head_dims(target)
        except Exception as err:
            configs["attention_head_dims"] = {"error": repr(err)}
        try:
            configs["reference_benchmarks"] = reference_benchmarks(target)
        except Exception as err:
            configs["reference_benchmarks"] = {"error": repr(err)}
        try:
            configs["config5_deltanet"] = config5(target)
        except Exception as err:
            configs["config5_deltanet"] = {"error": repr(err)}
        log("config5:", json.dumps(configs["config5_deltanet"]))
    cpu = None
    if not (a.no_cpu or a.only_config2):
        try:
            cpu = cpu_baseline(c2["x"], c2["g"])
        except Exception as err:
            cpu = {"error": repr(err)}
        if isinstance(cpu, dict):
            cpu.update(host_info())
        log("cpu_baseline:", json.dumps(cpu))
        # The other configs' CPU paths, each beside its own figures.
        for key, fn in (("config1_tanh_layer", cpu_config1), ("config3_mlp", cpu_config3),
                        ("config4_attention", cpu_config4), ("config5_deltanet", cpu_config5)):
            try:
                r = fn()
            except Exception as err:
                r = {"error": repr(err)}
            if isinstance(r, dict):
                r.update(host_info())
            if isinstance(configs.get(key), dict):
                configs[key]["cpu_baseline"] = r
            log(key, "cpu:", json.dumps(r))
    line = {
        "metric": "GB/s fused reduce (config 2: softmax and LayerNorm fwd+grad over X 32768x8192 fp32)",
        "value": value, "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": step_s * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (torch Philox N(0,1) on device, seed 20261201)",
        "config": {"workload": "config2: sum(softmax_columns(X).*G) and sum(layernorm(X).*G), withgradient, "
                               "X,G 8192x32768 column-major fp32", "rows": ROWS, "n": N,
                   "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu, "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
