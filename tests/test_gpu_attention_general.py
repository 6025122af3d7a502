"""Attention the matrix-core kernels do not take, on the general kernels:
the reference's attention fixtures at their own shapes (D = 4, fp32,
test/fixtures/programs.jl:110-113), the generated-attention cases of
test/cuda/attention.jl:10-16 (D 8..32, odd lengths, grouped heads), bf16 at
head dims 64 and 256 with lengths that are not multiples of 128, packed
documents (a first key per query, rebound to other layouts as the reference's
bind! does) and decode over a cache whose lengths the device holds.  Forward
and backward against the float64 oracle on the same inputs."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import data, relative

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5   # fp32 attention (fp32 arithmetic): 1e-5 relative, norm-wise
TOL_BF16 = 2e-2  # bf16 arrays: 2e-2 relative of the float64 oracle


def _run(q, k, v, g, causal, f32, starts=None, lengths=None, kv_heads=None, scale=0.0):
    """q (B, S, H, D), k, v (B, Sk, Hk, D) device tensors; returns o, lse, dq, dk, dv."""
    import tempest_hip.launch as L
    B, S, H, D = q.shape
    Sk, Hk = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(B, S, H, device="cuda")
    extra = dict(head_dim=D, kv_seq=Sk, f32=f32, scale=scale)
    if starts is not None:
        extra["starts"] = starts.data_ptr()
    if lengths is not None:
        extra["lengths"] = lengths.data_ptr()
    fwd = L.attention_fwd(B, H, Hk, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          causal=causal, **extra)
    fwd()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd = L.attention_bwd(B, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          g.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), causal=causal, kv_heads=Hk,
                          **extra)
    bwd()
    torch.cuda.synchronize()
    return (o, lse, dq, dk, dv), (fwd, bwd)


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _check(outs, q, k, v, g, causal, tol, starts=None, lengths=None, scale=None):
    o, lse, dq, dk, dv = (_np(t) for t in outs)
    st = None if starts is None else starts.cpu().numpy().T  # (S, B) column-major -> (B, S)
    ln = None if lengths is None else lengths.cpu().numpy()
    ro, rl = interpret.attention_fwd(_np(q), _np(k), _np(v), causal, scale, st, ln)
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), causal, scale, st, ln)
    assert relative(o, ro) < tol, relative(o, ro)
    assert np.max(np.abs(lse - rl)) < 1e-4 * max(1.0, np.abs(rl).max())
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(got, ref) < tol, (name, relative(got, ref))


@pytest.mark.parametrize("causal", [False, True])
def test_reference_attention_fixtures(target, causal):
    """"attention, grouped heads" and "causal attention with a residual":
    q data(4, 4, 6, 2; 0.3), k data(4, 2, 6, 2; 0.2), v data(4, 2, 6, 2; 0.1)."""
    announce("attn general fixture", causal)
    mk = lambda shape, s: torch.from_numpy(np.ascontiguousarray(np.transpose(data(*shape, scale=s), (3, 2, 1, 0))))
    q, k, v = (mk(sh, s).float().cuda() for sh, s in (((4, 4, 6, 2), 0.3), ((4, 2, 6, 2), 0.2), ((4, 2, 6, 2), 0.1)))
    g = mk((4, 4, 6, 2), 0.5).float().cuda()
    outs, _ = _run(q, k, v, g, causal, True)
    _check(outs, q, k, v, g, causal, TOL_F32)


@pytest.mark.parametrize("D,H,KV,S,B,causal", [(16, 2, 2, 200, 2, True), (16, 4, 2, 200, 2, True),
                                               (16, 4, 2, 200, 2, False), (32, 3, 1, 70, 3, True),
                                               (8, 1, 1, 133, 1, False)])
def test_generated_attention_cases_fp32(target, D, H, KV, S, B, causal):
    """test/cuda/attention.jl:10-16 at their shapes, fp32."""
    announce("attn general fp32", D, H, KV, S, B, causal)
    gen = torch.Generator(device="cuda").manual_seed(D * S + H)
    q = torch.randn(B, S, H, D, device="cuda", generator=gen) * 0.5
    k = torch.randn(B, S, KV, D, device="cuda", generator=gen) * 0.5
    v = torch.randn(B, S, KV, D, device="cuda", generator=gen)
    g = torch.randn(B, S, H, D, device="cuda", generator=gen)
    outs, _ = _run(q, k, v, g, causal, True)
    _check(outs, q, k, v, g, causal, TOL_F32)


@pytest.mark.parametrize("D,H,KV,S,Sk,causal", [(64, 4, 2, 300, 300, True), (256, 2, 2, 200, 200, False),
                                                (128, 2, 1, 129, 129, True), (64, 2, 2, 96, 250, False),
                                                (100, 3, 3, 77, 77, True)])
def test_bf16_head_dims_and_lengths(target, D, H, KV, S, Sk, causal):
    """bf16 at head dims the matrix-core kernels do not take (64, 100, 256),
    128 at a length that is not a multiple of 128, and more keys than queries."""
    announce("attn general bf16", D, H, KV, S, Sk, causal)
    gen = torch.Generator(device="cuda").manual_seed(D + S + Sk)
    q = torch.randn(2, S, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    k = torch.randn(2, Sk, KV, D, device="cuda", generator=gen).to(torch.bfloat16)
    v = torch.randn(2, Sk, KV, D, device="cuda", generator=gen).to(torch.bfloat16)
    g = torch.randn(2, S, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    outs, _ = _run(q, k, v, g, causal, False)
    _check(outs, q, k, v, g, causal, TOL_BF16)


def _starts(lengths):
    return [sum(lengths[:i]) + 1 for i in range(len(lengths)) for _ in range(lengths[i])]


def test_packed_documents_and_rebinding(target):
    """Documents packed in sequences (test/cuda/attention.jl:218-246): D 16,
    2 heads, 300 positions, 2 sequences, causal, scale 0.25; then the same
    launches with the starts rebound to one document a sequence and to one
    document a position."""
    n = 300
    gen = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(2, n, 2, 16, device="cuda", generator=gen) * 0.3
    k = torch.randn(2, n, 2, 16, device="cuda", generator=gen) * 0.3
    v = torch.randn(2, n, 2, 16, device="cuda", generator=gen)
    g = torch.randn(2, n, 2, 16, device="cuda", generator=gen)
    # (positions, batch) column-major: memory [b][s].
    layouts = [np.stack([_starts([90, 1, 130, 40, 39]), _starts([7, 200, 93])]),
               np.ones((2, n), dtype=np.int64), np.tile(np.arange(1, n + 1), (2, 1))]
    starts = torch.from_numpy(layouts[0].astype(np.int32)).cuda()
    announce("attn general packed documents")
    outs, (fwd, bwd) = _run(q, k, v, g, True, True, starts=starts, scale=0.25)
    _check(outs, q, k, v, g, True, TOL_F32, starts=starts.T, scale=0.25)
    for layout in layouts[1:]:
        other = torch.from_numpy(layout.astype(np.int32)).cuda()
        fwd.repoint("starts", other.data_ptr())
        bwd.repoint("starts", other.data_ptr())
        fwd()
        bwd()
        torch.cuda.synchronize()
        _check(outs, q, k, v, g, True, TOL_F32, starts=other.T, scale=0.25)


def test_decode_over_lengths_the_device_holds(target):
    """One query per head over a cache of 200 keys, 8 query heads over 2 key
    heads, 3 sequences holding 37, 200 and 1 keys; then the same launches
    with lengths 200, 5, 64 (test/cuda/attention.jl:254-271)."""
    gen = torch.Generator(device="cuda").manual_seed(10)
    q = torch.randn(3, 1, 8, 16, device="cuda", generator=gen) * 0.3
    k = torch.randn(3, 200, 2, 16, device="cuda", generator=gen) * 0.3
    v = torch.randn(3, 200, 2, 16, device="cuda", generator=gen)
    g = torch.randn(3, 1, 8, 16, device="cuda", generator=gen)
    lengths = torch.tensor([37, 200, 1], dtype=torch.int32, device="cuda")
    announce("attn general decode")
    outs, (fwd, bwd) = _run(q, k, v, g, False, True, lengths=lengths, scale=0.25)
    _check(outs, q, k, v, g, False, TOL_F32, lengths=lengths, scale=0.25)
    other = torch.tensor([200, 5, 64], dtype=torch.int32, device="cuda")
    fwd.repoint("lengths", other.data_ptr())
    bwd.repoint("lengths", other.data_ptr())
    fwd()
    bwd()
    torch.cuda.synchronize()
    _check(outs, q, k, v, g, False, TOL_F32, lengths=other, scale=0.25)
