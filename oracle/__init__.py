"""TEST INFRASTRUCTURE ONLY: the oracle for libtempest_hip.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or the timed CPU baseline; the product
(tempest.jl_amd/) never does.

- ``interpret``: Float64 restatement of the reference's plan-free interpreter
  (src/Compiler/program/interpret.jl) for the hot path's programs.
- ``folds``: the fold algebra (src/Compiler/IR/folds.jl) as plain Python.
- ``floor``: ctypes binding of ``floor.c``, the single-threaded Float32 CPU
  floor (src/Compiler/runtime/target.jl:308-350), built by ``make -C oracle``.
- ``data``: the reference tests' closed-form inputs (test/setup.jl:33-36).

Parity status of each function is stated in its module's header.
"""
