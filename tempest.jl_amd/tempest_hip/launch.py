"""Launches: what an implementation's build returns, owned on the host.

A ``Launch`` wraps a ``th_launch*``: one claim's kernels with their
arguments.  Calling it runs the kernels (a step of ``execute!``);
``repoint`` is the reference's ``Implement.repoint!(launch, value, buffer)``
(src/Compiler/Implement/Implement.jl; ext/CUDAExt.jl:1086-1090), by the value
numbers its builder gave.  The builders below are the entry points of
include/tempest_hip.h, one per op class and sketch.
"""
from __future__ import annotations

import ctypes
import os

from . import _lib
from ._lib import call


class Launch:
    def __init__(self, handle: ctypes.c_void_p, values: tuple[str, ...]):
        self._h = handle
        self.values = values  # value number -> the name the program gave it

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("launch used after destroy")
        return self._h

    def __call__(self) -> None:
        call("th_launch_run", self.handle)

    def repoint(self, value: int | str, ptr: int) -> None:
        if isinstance(value, str):
            value = self.values.index(value)
        call("th_launch_repoint", self.handle, value, ctypes.c_void_p(ptr))

    def work(self) -> _lib.Work:
        w = _lib.Work()
        call("th_launch_work", self.handle, ctypes.byref(w))
        return w

    def workspace(self) -> int:
        """Bytes of device memory the launch's kernels use beyond its values
        (th_launch_workspace): allocated at the first run unless given."""
        n = ctypes.c_uint64()
        call("th_launch_workspace", self.handle, ctypes.byref(n))
        return n.value

    def set_workspace(self, ptr: int) -> None:
        """Use the memory at ``ptr`` (256-byte aligned) as the workspace."""
        call("th_launch_set_workspace", self.handle, ctypes.c_void_p(ptr))

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(2048)
        call("th_launch_describe", self.handle, buf, len(buf))
        return buf.value.decode()

    def destroy(self) -> None:
        if self._h is not None:
            call("th_launch_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def _built(name: str, values: tuple[str, ...], *args) -> Launch:
    out = ctypes.c_void_p()
    call(name, *args, ctypes.byref(out))
    return Launch(out, values)


def _p(ptr: int) -> ctypes.c_void_p:
    return ctypes.c_void_p(int(ptr))


# ---- op class (a) -----------------------------------------------------------

def softmax_grad(rows: int, n: int, ld: int, x: int, g: int, dx: int, loss: int) -> Launch:
    return _built("th_build_softmax_grad", ("x", "g", "dx", "loss"), rows, n, ld, _p(x), _p(g), _p(dx), _p(loss))


def layernorm_grad(rows: int, n: int, ld: int, eps: float, x: int, g: int, dx: int, loss: int) -> Launch:
    return _built("th_build_layernorm_grad", ("x", "g", "dx", "loss"), rows, n, ld, eps, _p(x), _p(g), _p(dx),
                  _p(loss))


def softmax_fwd(rows: int, n: int, ld: int, x: int, y: int) -> Launch:
    return _built("th_build_softmax_fwd", ("x", "y"), rows, n, ld, _p(x), _p(y))


def layernorm_fwd(rows: int, n: int, ld: int, eps: float, x: int, y: int) -> Launch:
    return _built("th_build_layernorm_fwd", ("x", "y"), rows, n, ld, eps, _p(x), _p(y))


def full_sum(count: int, x: int, out: int) -> Launch:
    return _built("th_build_sum", ("x", "out"), count, _p(x), _p(out))


# ---- config 1 ---------------------------------------------------------------

def tanh_layer_grad(d: int, h: int, c: int, w: int, b: int, x: int, loss: int, dw: int, db: int, dx: int) -> Launch:
    return _built("th_build_tanh_layer_grad", ("w", "b", "x", "loss", "dw", "db", "dx"), d, h, c, _p(w), _p(b),
                  _p(x), _p(loss), _p(dw), _p(db), _p(dx))


# ---- op class (b) -----------------------------------------------------------

F32, BF16, F16 = 0, 1, 4
STORE, GELU, SQUARE_LOSS, GELU_BACKWARD = 0, 1, 2, 3
F32_FACTORS, F16_FACTORS, ACCUMULATE, BF16X3 = 1, 2, 4, 8  # TH_GEMM_*
# TH_TILE_*: which kernel and output tile a product runs on.
TILE_AUTO, TILE_256, TILE_128X128, TILE_128X64, TILE_64X128, TILE_64X64, TILE_GENERAL = range(7)
TILE_NAMES = {TILE_256: "256x256", TILE_128X128: "128x128", TILE_128X64: "128x64", TILE_64X128: "64x128",
              TILE_64X64: "64x64", TILE_GENERAL: "general 64x64 fp32"}


def _gemm_desc(m, n, k, a, a_m, a_k, b, b_k, b_n, c, c_ld, c_dtype=BF16, epilogue=STORE, bias=0, aux=0, aux_ld=0,
               aux_out=0, row_sums=0, loss=0, batch=1, a_batch=0, b_batch=0, c_batch=0, factors=BF16, d=0, d_ld=0,
               d_batch=0, splits=0, tile=TILE_AUTO, bf16x3=False):
    flags = {BF16: 0, F32: F32_FACTORS, F16: F16_FACTORS}[factors] | (ACCUMULATE if d else 0) | (BF16X3 if bf16x3 else 0)
    return _lib.GemmDesc(m=m, n=n, k=k, c_dtype=c_dtype, epilogue=epilogue, tile=tile, a=a, a_m=a_m, a_k=a_k, b=b,
                         b_k=b_k, b_n=b_n, c=c, c_ld=c_ld, bias=bias or None, aux=aux or None, aux_ld=aux_ld,
                         aux_out=aux_out or None, row_sums=row_sums or None, loss=loss or None, batch=batch,
                         flags=flags, a_batch=a_batch, b_batch=b_batch, c_batch=c_batch, d=d or None, d_ld=d_ld,
                         d_batch=d_batch, splits=splits)


def gemm(m: int, n: int, k: int, a: int, a_m: int, a_k: int, b: int, b_k: int, b_n: int, c: int, c_ld: int,
         c_dtype: int = BF16, epilogue: int = STORE, bias: int = 0, aux: int = 0, aux_ld: int = 0,
         aux_out: int = 0, row_sums: int = 0, loss: int = 0, batch: int = 1, a_batch: int = 0, b_batch: int = 0,
         c_batch: int = 0, factors: int = BF16, d: int = 0, d_ld: int = 0, d_batch: int = 0,
         splits: int = 0, tile: int = TILE_AUTO, bf16x3: bool = False) -> Launch:
    """C (m x n, column-major at c_ld) = A (m x k) * B (k x n) (+ D with d), for
    each of `batch` products; A(i, l) at a[i*a_m + l*a_k], B(l, j) at
    b[l*b_k + j*b_n], product z's operands *_batch elements further; factors
    BF16, F32 or F16; tile: TILE_* (the kernel and its output tile, TILE_AUTO
    chosen); splits: parts of K (0 chosen, 1 none); bf16x3: fp32 factors as
    hi + lo bf16 on the bf16 tile kernels (TH_GEMM_BF16X3).  With TEMPEST_HIP_TUNE=1
    in the environment a product left to the library (TILE_AUTO, splits 0)
    takes th_gemm_tune's measured choice instead, as the Julia binding's build
    does (not D + A B in place, which each measurement would add again)."""
    desc = _gemm_desc(m, n, k, a, a_m, a_k, b, b_k, b_n, c, c_ld, c_dtype, epilogue, bias, aux, aux_ld, aux_out,
                      row_sums, loss, batch, a_batch, b_batch, c_batch, factors, d, d_ld, d_batch, splits, tile,
                      bf16x3)
    if tile == TILE_AUTO and splits == 0 and os.environ.get("TEMPEST_HIP_TUNE") == "1" and not (d and d == c):
        t, sp, sec = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_double()
        call("th_gemm_tune", ctypes.byref(desc), ctypes.byref(t), ctypes.byref(sp), ctypes.byref(sec))
        desc.tile, desc.splits = t.value, sp.value
    return _built("th_build_gemm", ("a", "b", "c", "bias", "aux", "aux_out", "row_sums", "loss", "d"),
                  ctypes.byref(desc))


def gemm_tune(m: int, n: int, k: int, a: int, a_m: int, a_k: int, b: int, b_k: int, b_n: int, c: int, c_ld: int,
              **extra) -> tuple[int, int, float]:
    """(tile, splits, seconds): the product's fastest choice, measured on the
    device on these arrays (th_gemm_tune: every tile that takes it, then the
    splits of the best; kept for the process).  extra: gemm's keywords."""
    desc = _gemm_desc(m, n, k, a, a_m, a_k, b, b_k, b_n, c, c_ld, **extra)
    tile, splits, seconds = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_double()
    call("th_gemm_tune", ctypes.byref(desc), ctypes.byref(tile), ctypes.byref(splits), ctypes.byref(seconds))
    return tile.value, splits.value, seconds.value


# ---- op class (c) -----------------------------------------------------------

def _attention_desc(batch, heads, kv_heads, seq, q, k, v, o, lse=0, dout=0, dq=0, dk=0, dv=0, causal=True,
                    scale=0.0, q_strides=None, k_strides=None, head_dim=128, flags=0, kv_seq=0, starts=0, lengths=0,
                    f32=False):
    ks_n = kv_seq or seq
    qs = q_strides or (head_dim, heads * head_dim, seq * heads * head_dim)
    ks = k_strides or (head_dim, kv_heads * head_dim, ks_n * kv_heads * head_dim)
    d = _lib.AttentionDesc(batch=batch, heads=heads, kv_heads=kv_heads, seq=seq, head_dim=head_dim,
                           causal=int(causal), scale=scale, flags=flags | (ATTN_F32 if f32 else 0), q=q, k=k, v=v,
                           o=o, lse=lse or None, dout=dout or None, dq=dq or None, dk=dk or None, dv=dv or None,
                           kv_seq=kv_seq, starts=starts or None, lengths=lengths or None)
    d.q_strides[:] = list(qs)
    d.k_strides[:] = list(ks)
    return d


ATTN_F32 = 2  # TH_ATTN_F32


def attention_fwd(batch: int, heads: int, kv_heads: int, seq: int, q: int, k: int, v: int, o: int, lse: int = 0,
                  causal: bool = True, scale: float = 0.0, **extra) -> Launch:
    """o = attention(q, k, v; causal) over (d, heads, positions, batch) arrays
    (bf16, or fp32 with f32=True); lse fp32.  extra: head_dim, kv_seq (keys'
    positions), starts (int32 (positions, batch), 1-based first key of each
    query), lengths (int32 (batch), keys of each sequence), q_strides, k_strides."""
    d = _attention_desc(batch, heads, kv_heads, seq, q, k, v, o, lse, causal=causal, scale=scale, **extra)
    return _built("th_build_attention_fwd", ("q", "k", "v", "o", "lse", "starts", "lengths"), ctypes.byref(d))


RECOMPUTE_DQ = 1  # TH_ATTN_RECOMPUTE_DQ


def attention_bwd(batch: int, heads: int, seq: int, q: int, k: int, v: int, o: int, lse: int, dout: int, dq: int,
                  dk: int, dv: int, causal: bool = True, scale: float = 0.0, recompute_dq: bool = False,
                  kv_heads: int = 0, **extra) -> Launch:
    """dq, dk, dv of sum(attention(q, k, v) .* dout), from the forward's o and lse.
    kv_heads (default heads): k, v, dk, dv have kv_heads heads, each read by
    heads / kv_heads query heads; dk and dv sum over them.
    recompute_dq: the dQ sweep recomputes S and dP instead of reading the dS
    the dK/dV sweep stores (the path taken anyway past 16 GiB of dS)."""
    d = _attention_desc(batch, heads, kv_heads or heads, seq, q, k, v, o, lse, dout, dq, dk, dv, causal=causal,
                        scale=scale, flags=RECOMPUTE_DQ if recompute_dq else 0, **extra)
    return _built("th_build_attention_bwd",
                  ("q", "k", "v", "o", "lse", "dout", "dq", "dk", "dv", "starts", "lengths"), ctypes.byref(d))


# ---- config 5 ---------------------------------------------------------------

def deltanet(batch: int, heads: int, seq: int, q: int, k: int, v: int, a: int, beta: int, o: int, dout: int = 0,
             dq: int = 0, dk: int = 0, dv: int = 0, da: int = 0, dbeta: int = 0, d: int = 128) -> Launch:
    """Chunked gated DeltaNet over (d, heads, positions, batch) bf16 arrays and
    (heads, positions, batch) fp32 gates; the gradient too when dout is given."""
    desc = _lib.DeltaNetDesc(batch=batch, heads=heads, seq=seq, dk=d, dv=d, chunk=64, q=q, k=k, v=v, a=a, beta=beta,
                             o=o, dout=dout or None, dq=dq or None, dk_out=dk or None, dv_out=dv or None,
                             da=da or None, dbeta=dbeta or None)
    desc.strides[:] = [d, heads * d, seq * heads * d]
    desc.gate_strides[:] = [1, heads, seq * heads]
    name = "th_build_deltanet" if dout else "th_build_deltanet_fwd"
    return _built(name, ("q", "k", "v", "a", "beta", "o", "dout", "dq", "dk", "dv", "da", "dbeta"),
                  ctypes.byref(desc))
