"""Attention on the matrix cores at head dims 64 and 256 (and 128 at lengths
the tuned kernels do not take): bf16 arrays, any lengths (the last query and
key tiles masked), causal or not, keys more or fewer than queries, grouped
heads.  Forward (o, lse) and backward (dq, dk, dv) against the float64
oracle on the same inputs, within the bf16 tolerance of the reference's
attention tests; the launches are the matrix-core kernels (mfma_attn_*)."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import relative

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2  # bf16 arrays: 2e-2 relative of the float64 oracle, norm-wise


def _inputs(B, S, Sk, H, KV, D, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, S, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    k = torch.randn(B, Sk, KV, D, device="cuda", generator=gen).to(torch.bfloat16)
    v = torch.randn(B, Sk, KV, D, device="cuda", generator=gen).to(torch.bfloat16)
    g = torch.randn(B, S, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    return q, k, v, g


def _run(q, k, v, g, causal):
    import tempest_hip.launch as L
    B, S, H, D = q.shape
    Sk, KV = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(B, S, H, device="cuda")
    fwd = L.attention_fwd(B, H, KV, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          causal=causal, head_dim=D, kv_seq=Sk)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    bwd = L.attention_bwd(B, H, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                          g.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), causal=causal, kv_heads=KV,
                          head_dim=D, kv_seq=Sk)
    assert "mfma_attn_fwd" in fwd.describe(), fwd.describe()
    assert "mfma_attn_dkdv" in bwd.describe() and "mfma_attn_dq" in bwd.describe(), bwd.describe()
    fwd()
    bwd()
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def _check(outs, q, k, v, g, causal):
    o, lse, dq, dk, dv = (_np(t) for t in outs)
    ro, rl = interpret.attention_fwd(_np(q), _np(k), _np(v), causal)
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), causal)
    assert relative(o, ro) < TOL_BF16, relative(o, ro)
    assert np.max(np.abs(lse - rl)) < 1e-3 * max(1.0, np.abs(rl).max()), np.max(np.abs(lse - rl))
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(got, ref) < TOL_BF16, (name, relative(got, ref))


@pytest.mark.parametrize("D,B,H,KV,S,Sk,causal", [
    (64, 2, 4, 2, 300, 300, True), (64, 2, 4, 4, 300, 300, False), (64, 1, 2, 1, 1000, 1000, True),
    (64, 2, 2, 2, 77, 250, False), (64, 2, 2, 2, 250, 77, True), (64, 1, 3, 3, 1, 1, True),
    (256, 2, 2, 2, 200, 200, False), (256, 2, 4, 2, 333, 333, True), (256, 1, 2, 2, 64, 190, False),
    (128, 2, 2, 1, 129, 129, True), (128, 1, 2, 2, 500, 300, False)])
def test_matrix_core_attention_at_head_dims_and_lengths(target, D, B, H, KV, S, Sk, causal):
    announce("attn mfma", D, B, H, KV, S, Sk, causal)
    q, k, v, g = _inputs(B, S, Sk, H, KV, D, D * 7 + S + Sk)
    outs = _run(q, k, v, g, causal)
    _check(outs, q, k, v, g, causal)


@pytest.mark.parametrize("D", [64, 256])
def test_matrix_core_attention_at_size_sampled_heads(target, D):
    """B2 H4 S2048 causal, grouped heads (2 key heads): every output checked
    for the first batch's heads against the float64 oracle."""
    announce("attn mfma at size", D)
    B, S, H, KV = 2, 2048, 4, 2
    q, k, v, g = _inputs(B, S, S, H, KV, D, 100 + D)
    o, lse, dq, dk, dv = _run(q, k, v, g, True)
    sl = slice(0, 1)
    ro, rl = interpret.attention_fwd(_np(q[sl]), _np(k[sl]), _np(v[sl]), True)
    rq, rk, rv = interpret.attention_bwd(_np(q[sl]), _np(k[sl]), _np(v[sl]), _np(g[sl]), True)
    assert relative(_np(o[sl]), ro) < TOL_BF16
    assert np.max(np.abs(_np(lse[sl]) - rl)) < 1e-3 * max(1.0, np.abs(rl).max())
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(_np(got[sl]), ref) < TOL_BF16, (name, relative(_np(got[sl]), ref))


@pytest.mark.parametrize("D,B,H,KV,S,causal,split", [
    (64, 1, 2, 2, 700, True, True), (256, 1, 2, 1, 300, False, True), (64, 4, 16, 16, 512, True, False)])
def test_split_and_whole_sweeps(target, D, B, H, KV, S, causal, split):
    """A grid under one workgroup a CU splits each sweep into parts (fp32
    partial results combined or summed in part order by launches of their
    own); a grid that fills the device sweeps whole.  Both against the
    float64 oracle."""
    import tempest_hip.launch as L
    announce("attn mfma split", D, B, H, KV, S, causal, split)
    q, k, v, g = _inputs(B, S, S, H, KV, D, 31 * D + S + H)
    outs = _run(q, k, v, g, causal)
    p = q.data_ptr()
    fwd = L.attention_fwd(B, H, KV, S, p, p, p, p, p, causal=causal, head_dim=D).describe()
    bwd = L.attention_bwd(B, H, S, p, p, p, p, p, p, p, p, p, causal=causal, kv_heads=KV, head_dim=D).describe()
    assert ("mfma_attn_combine" in fwd) == split, fwd
    assert ("mfma_attn_sum_dk" in bwd and "mfma_attn_sum_dq" in bwd) == split, bwd
    _check(outs, q, k, v, g, causal)
