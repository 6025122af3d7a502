"""The rates the cover prices HIP claims with, measured on the device.

The reference keeps, per device, a rates file of named numbers that its cost
model reads (src/Compiler/cover/rates/NVIDIA_GB10.cold.rates.tsv, written by
calibrate!, src/Compiler/cover/calibrate.jl).  This module measures the same
quantities for this backend on an MI355X, with the same probes and fits, and
writes them in the same format (a key, a tab, a number per line):

- ``device bandwidth / cache / blocks``: th_device_rates (record.jl:195).
- ``floor memory latency / bandwidth``: sum(x; dims = 1) over 1024-row
  columns at MEMORY_COLUMNS sizes (64 KB to 1 GiB) through the generated floor, each timed as
  claims are (th_time_launch: caches cleared, the minimum of samples, less a
  replay's overhead); the bandwidth is the least-squares slope of seconds on
  bytes, the latency the smallest fold's time less its bytes at that
  bandwidth, per launch (fit_memory!, calibrate.jl:438-465).  ``floor memory
  refold`` is 0: the floor's claims state no steps.
- ``HIP memory latency / bandwidth``: this library claims no plain column
  fold, so the device's launch and cached rates, as fit_memory! keeps for a
  package without one; both are measured (th_device_rates: an empty kernel's
  share of a long replayed graph, and the read rate of 64 MiB the caches
  hold).
- ``HIP BFloat16 latency / rate / split / recompute``: the bf16 product at
  two sizes; the rate is the slope of seconds on flops, the latency the
  smaller's time less its flops at that rate; the products neither split
  their sums nor recompute folds, so split and recompute are the rate (as the
  GB10 file's cuBLAS lines are).
- ``applied streamed any <f>``: the seconds per application of each of
  APPLIED in a fold over APPLIED_TIMES applications of it on an
  APPLIED_SHAPE array, beyond the fold alone (calibrate.jl:71-82, 89-99,
  139-140); never below 0.

    python -m tempest_hip.calibrate --out rates/AMD_Instinct_MI355X.cold.rates.tsv
"""
from __future__ import annotations

import argparse
import pathlib
import sys

import torch

from .floor import FloorGroup
from . import launch as L

TIMING_BASIS = 2.0  # the reference's definition of a launch's time (record.jl:182)
# The reference's columns (16, 256, 1024, 4096: at most 16 MB) are latency-bound
# on MI355X (16 MB moves in ~2 us, a launch's time), so a line through them
# overstates the bandwidth (12 TB/s); columns up to 1 GiB put the slope where
# the folds are bandwidth-bound, and the smallest still gives the latency.
MEMORY_COLUMNS = (16, 4096, 65536, 262144)
APPLIED_SHAPE = (4096, 512)
APPLIED_TIMES = 8
# (name in the rates file, how one application is written), as the
# reference's apply_chain (src/Compiler/cover/calibrate.jl:236-239) applies
# each: a unary function to y; a binary one to y and the constant 1.5; ^ as
# y^3 (Julia's literal power, two products); a cast as the cast of y plus 1.5.
APPLIED = [(name, (lambda g, y, f=name: g.apply(f, y))) for name in
           ("exp", "log", "tanh", "sqrt", "sin", "cos", "abs", "abs2", "inv")]
APPLIED += [(name, (lambda g, y, f=name: g.apply(f, y, 1.5))) for name in ("*", "+", "-", "/", "max", "min")]
APPLIED += [("^", lambda g, y: y * y * y), ("identity", lambda g, y: y), ("Float32", lambda g, y: y + 1.5),
            ("BFloat16", lambda g, y: g.apply("bfloat16", y) + 1.5)]
SAMPLES = 10


def _fit_line(xs, ys):
    """Least squares y = a + b x: (a, b)."""
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    b = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    return my - b * mx, b


def _column_sum(rows: int, n: int, body=None) -> FloorGroup:
    g = FloorGroup("reduction", (rows, n), reduced=(0,), name=f"sum(x; dims = 1), {rows} x {n}")
    g.value("x", "f32", rows * n)
    g.value("r", "f32", n)
    x = g.load("x", (1, rows))
    g.output("r", g.fold("sum", x if body is None else body(g, x)).value, (0, 1), full=False)
    return g


def _timed(target, group: FloorGroup, buffers: dict) -> tuple[float, float, int]:
    launch = group.build({k: v.data_ptr() for k, v in buffers.items()})
    t = target.time_launch(launch, SAMPLES)
    w = launch.work()
    return t, w.bytes, w.kernels


def calibrate(target) -> dict[str, float]:
    rates: dict[str, float] = {"timing basis": TIMING_BASIS}
    dev = target.device_rates()
    rates.update({"device bandwidth": dev["bandwidth"], "device cache": dev["cache"], "device blocks": dev["blocks"]})

    # The floor's memory: column sums at the reference's sizes.
    gen = torch.Generator(device="cuda").manual_seed(7)
    secs, bytes_, launches = [], [], []
    for n in MEMORY_COLUMNS:
        x = torch.randn(1024 * n, device="cuda", generator=gen)
        r = torch.zeros(n, device="cuda")
        t, b, k = _timed(target, _column_sum(1024, n), {"x": x, "r": r})
        secs.append(t)
        bytes_.append(b)
        launches.append(k)
    _, per_byte = _fit_line(bytes_, secs)
    bandwidth = 1.0 / per_byte if per_byte > 0 else dev["bandwidth"]
    latency = max(0.0, (secs[0] - bytes_[0] / bandwidth) / launches[0])
    rates.update({"floor memory latency": latency, "floor memory bandwidth": bandwidth, "floor memory refold": 0.0})
    rates.update({"HIP memory latency": dev["launch"], "HIP memory bandwidth": dev["cached"], "HIP memory refold": 0.0})

    # The bf16 products: two sizes, the rate the slope of seconds on flops.
    pts = []
    for m in (4096, 8192):  # sizes that fill the device (a 256 x 256 tile per CU and more)
        a = torch.randn(m, m, device="cuda", generator=gen).to(torch.bfloat16)
        b = torch.randn(m, m, device="cuda", generator=gen).to(torch.bfloat16)
        c = torch.empty(m, m, device="cuda", dtype=torch.bfloat16)
        # C (m x m, column-major) = A B with A, B column-major: A(i, l) at i + m l.
        launch = L.gemm(m, m, m, a.data_ptr(), 1, m, b.data_ptr(), 1, m, c.data_ptr(), m)
        pts.append((2.0 * m ** 3, target.time_launch(launch, SAMPLES)))
    (f1, t1), (f2, t2) = pts
    rate = (f2 - f1) / (t2 - t1) if t2 > t1 else f2 / t2
    plat = max(0.0, t1 - f1 / rate)
    for what, v in (("latency", plat), ("rate", rate), ("split", rate), ("recompute", rate)):
        rates[f"HIP BFloat16 {what}"] = v

    # Functions applied in a streamed fold: APPLIED_TIMES applications beyond the fold alone.
    rows, n = APPLIED_SHAPE
    x = (torch.rand(rows * n, device="cuda", generator=gen) * 0.5 + 0.25)  # in (0.25, 0.75): every f finite
    r = torch.zeros(n, device="cuda")
    alone, _, _ = _timed(target, _column_sum(rows, n), {"x": x, "r": r})
    for name, once in APPLIED:
        def body(g, t, once=once):
            y = t
            for _ in range(APPLIED_TIMES):
                y = once(g, y)
            return y
        t, _, _ = _timed(target, _column_sum(rows, n, body), {"x": x, "r": r})
        rates[f"applied streamed any {name}"] = max(0.0, (t - alone) / (APPLIED_TIMES * rows * n))
    return rates


def write(rates: dict[str, float], path: pathlib.Path) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w") as f:
        for k, v in rates.items():
            f.write(f"{k}\t{v!r}\n")


def read(path: pathlib.Path) -> dict[str, float]:
    out = {}
    for line in pathlib.Path(path).read_text().splitlines():
        if line.strip():
            k, v = line.rsplit("\t", 1)
            out[k] = float(v)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", required=True)
    a = ap.parse_args(argv)
    from .target import HIPTarget
    target = HIPTarget()
    rates = calibrate(target)
    write(rates, pathlib.Path(a.out))
    for k, v in rates.items():
        print(f"{k}\t{v:.6g}", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
