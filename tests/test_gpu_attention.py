"""Op class (c) on the GPU: flash attention forward and backward against the
oracle (float64 on the same bf16 inputs), causal and not, grouped heads, and
config 4's full size on sampled heads."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import relative

pytestmark = pytest.mark.gpu

TOL = 2e-2  # bf16 attention: 2e-2 relative (norm-wise) of the fp64 reference


def _rand(shape, gen):
    return torch.randn(*shape, device="cuda", generator=gen).to(torch.bfloat16)


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("B,H,Hk,S,causal", [(1, 2, 2, 128, True), (2, 3, 3, 384, True), (1, 2, 2, 256, False),
                                             (1, 4, 2, 256, True), (1, 1, 1, 1024, True)])
def test_forward_matches_oracle(target, B, H, Hk, S, causal):
    import tempest_hip.launch as L
    announce("attn fwd", B, H, Hk, S, causal)
    gen = torch.Generator(device="cuda").manual_seed(S + H)
    q, k, v = _rand((B, S, H, 128), gen), _rand((B, S, Hk, 128), gen), _rand((B, S, Hk, 128), gen)
    o = torch.empty_like(q)
    lse = torch.empty(B, S, H, device="cuda")
    l = L.attention_fwd(B, H, Hk, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                        causal=causal)
    l()
    torch.cuda.synchronize()
    ro, rl = interpret.attention_fwd(_np(q), _np(k), _np(v), causal)
    assert relative(_np(o), ro) < TOL
    assert np.max(np.abs(lse.cpu().numpy() - rl)) < 1e-3 * max(1.0, np.abs(rl).max())


@pytest.mark.parametrize("B,H,S,causal", [(1, 2, 128, True), (2, 2, 384, True), (1, 2, 256, False),
                                          (1, 1, 1024, True)])
def test_backward_matches_oracle(target, B, H, S, causal):
    import tempest_hip as th
    announce("attn bwd", B, H, S, causal)
    gen = torch.Generator(device="cuda").manual_seed(7 * S + H)
    q, k, v, g = (_rand((B, S, H, 128), gen) for _ in range(4))
    comp = th.compile(th.programs.attention(B, H, S, causal=causal), target, q, k, v, g)
    o, dq, dk, dv = comp(q, k, v, g)
    ro, _ = interpret.attention_fwd(_np(q), _np(k), _np(v), causal)
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), causal)
    assert relative(_np(o.view(B, S, H, 128)), ro) < TOL
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(_np(got.view(B, S, H, 128)), ref) < TOL, name


@pytest.mark.parametrize("B,H,Hk,S,causal,recompute", [(1, 4, 2, 256, True, False), (2, 4, 1, 384, True, False),
                                                        (1, 6, 2, 256, False, False), (1, 4, 2, 384, True, True)])
def test_grouped_backward_matches_oracle(target, B, H, Hk, S, causal, recompute):
    """Grouped heads (test/cuda/attention.jl:132-140): dk and dv of each
    key/value head sum over the query heads that read it."""
    import tempest_hip.launch as L
    announce("attn bwd grouped", B, H, Hk, S, causal, recompute)
    gen = torch.Generator(device="cuda").manual_seed(13 * S + H + Hk)
    q, g = _rand((B, S, H, 128), gen), _rand((B, S, H, 128), gen)
    k, v = _rand((B, S, Hk, 128), gen), _rand((B, S, Hk, 128), gen)
    o, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    lse = torch.empty(B, S, H, device="cuda")
    ptr = lambda t: t.data_ptr()  # noqa: E731
    fwd = L.attention_fwd(B, H, Hk, S, ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), causal=causal)
    bwd = L.attention_bwd(B, H, S, ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), ptr(g), ptr(dq), ptr(dk), ptr(dv),
                          causal=causal, recompute_dq=recompute, kv_heads=Hk)
    fwd()
    bwd()
    torch.cuda.synchronize()
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), causal)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(_np(got), ref) < TOL, name


def test_grouped_program(target):
    """The compiled program with grouped heads, against the oracle."""
    import tempest_hip as th
    announce("attn program grouped")
    B, H, Hk, S = 1, 4, 2, 256
    gen = torch.Generator(device="cuda").manual_seed(21)
    q, g = _rand((B, S, H, 128), gen), _rand((B, S, H, 128), gen)
    k, v = _rand((B, S, Hk, 128), gen), _rand((B, S, Hk, 128), gen)
    comp = th.compile(th.programs.attention(B, H, S, kv_heads=Hk), target, q, k, v, g)
    o, dq, dk, dv = comp(q, k, v, g)
    ro, _ = interpret.attention_fwd(_np(q), _np(k), _np(v), True)
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), True)
    assert relative(_np(o.view(B, S, H, 128)), ro) < TOL
    for name, got, ref, heads in (("dq", dq, rq, H), ("dk", dk, rk, Hk), ("dv", dv, rv, Hk)):
        assert relative(_np(got.view(B, S, heads, 128)), ref) < TOL, name


@pytest.mark.parametrize("S,causal", [(384, True), (256, False)])
@pytest.mark.parametrize("recompute", [False, True])
def test_backward_both_dq_paths(target, S, causal, recompute):
    """Launch level: the dQ sweep reading the stored dS, and the one that
    recomputes S and dP, each against the oracle."""
    import tempest_hip.launch as L
    announce("attn bwd path", S, causal, "recompute" if recompute else "stored dS")
    B, H = 2, 2
    gen = torch.Generator(device="cuda").manual_seed(11 * S + int(recompute))
    q, k, v, g = (_rand((B, S, H, 128), gen) for _ in range(4))
    o, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
    lse = torch.empty(B, S, H, device="cuda")
    ptr = lambda t: t.data_ptr()  # noqa: E731
    fwd = L.attention_fwd(B, H, H, S, ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), causal=causal)
    bwd = L.attention_bwd(B, H, S, ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), ptr(g), ptr(dq), ptr(dk), ptr(dv),
                          causal=causal, recompute_dq=recompute)
    assert ("attn_bwd_dq<" if recompute else "attn_bwd_dq_frag<") in bwd.describe()
    fwd()
    bwd()
    torch.cuda.synchronize()
    rq, rk, rv = interpret.attention_bwd(_np(q), _np(k), _np(v), _np(g), causal)
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert relative(_np(got), ref) < TOL, name


def test_head_dims_route_to_the_kernels_that_take_them(target):
    """d 128 at a multiple of 128 takes the tuned matrix-core kernel; d 64,
    d 256 and d 128 at a length of 100 the other matrix-core kernels; fp32 at
    d 64 and 128 the fp32 matrix-core kernels; d 100 (bf16 or fp32) the
    general kernels; d beyond 256 is refused."""
    import tempest_hip.launch as L
    from tempest_hip import HIPError
    t = torch.zeros(1, 128, 1, 300, dtype=torch.bfloat16, device="cuda")
    p = t.data_ptr()
    tuned = L.attention_fwd(1, 1, 1, 128, p, p, p, p).describe()
    assert "attn_fwd" in tuned and "mfma_attn" not in tuned
    assert "mfma_attn_fwd_d64" in L.attention_fwd(1, 1, 1, 128, p, p, p, p, head_dim=64).describe()
    assert "mfma_attn_fwd_d256" in L.attention_fwd(1, 1, 1, 128, p, p, p, p, head_dim=256).describe()
    assert "mfma_attn_fwd_d128" in L.attention_fwd(1, 1, 1, 100, p, p, p, p).describe()
    assert "attn_gen_fwd" in L.attention_fwd(1, 1, 1, 128, p, p, p, p, head_dim=100).describe()
    assert "f32_attn_fwd_d128" in L.attention_fwd(1, 1, 1, 128, p, p, p, p, f32=True).describe()
    assert "f32_attn_fwd_d64" in L.attention_fwd(1, 1, 1, 100, p, p, p, p, f32=True, head_dim=64).describe()
    assert "attn_gen_fwd" in L.attention_fwd(1, 1, 1, 128, p, p, p, p, f32=True, head_dim=100).describe()
    with pytest.raises(HIPError, match="head_dim must be 1..256"):
        L.attention_fwd(1, 1, 1, 128, p, p, p, p, head_dim=300)


def test_config4_full_size_sampled_heads(target):
    """B8 H16 S4096 D128 causal: every output computed on the GPU; sampled
    (batch, head) pairs checked against the float64 oracle."""
    import tempest_hip as th
    announce("attn config4 full")
    B, H, S = 8, 16, 4096
    gen = torch.Generator(device="cuda").manual_seed(4)
    q, k, v, g = (_rand((B, S, H, 128), gen) for _ in range(4))
    comp = th.compile(th.programs.attention(B, H, S), target, q, k, v, g)
    o, dq, dk, dv = comp(q, k, v, g)
    for b, h in ((0, 0), (5, 11)):
        sl = lambda t: _np(t.view(B, S, H, 128)[b:b + 1, :, h:h + 1])  # noqa: E731
        ro, _ = interpret.attention_fwd(sl(q), sl(k), sl(v), True)
        rq, rk, rv = interpret.attention_bwd(sl(q), sl(k), sl(v), sl(g), True)
        assert relative(sl(o), ro) < TOL
        for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
            assert relative(sl(got), ref) < TOL, (b, h, name)
