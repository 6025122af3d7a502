"""Config 5 on the GPU: chunked gated DeltaNet forward and gradient against
the oracle (float64, on the same bf16/fp32 inputs)."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import interpret
from oracle.data import relative

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _inputs(B, T, H, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *s: torch.randn(*s, device="cuda", generator=gen)  # noqa: E731
    unit = lambda x: x / x.norm(dim=-1, keepdim=True)  # noqa: E731
    q = unit(r(B, T, H, 128)).to(torch.bfloat16)
    k = unit(r(B, T, H, 128)).to(torch.bfloat16)
    v = r(B, T, H, 128).to(torch.bfloat16)
    a = -torch.nn.functional.softplus(r(B, T, H))
    beta = torch.sigmoid(r(B, T, H))
    do = r(B, T, H, 128).to(torch.bfloat16)
    return q, k, v, a.contiguous(), beta.contiguous(), do


def _np(t):
    return t.float().cpu().numpy()


# (1, 8192, 2): config 5's sequence length, 128 chunks of state hand-off
# through the split-bf16 products.
@pytest.mark.parametrize("B,T,H", [(1, 64, 1), (1, 256, 2), (2, 192, 3), (1, 8192, 2)])
def test_forward_and_gradient_match_oracle(target, B, T, H):
    import tempest_hip as th
    announce("deltanet", B, T, H)
    q, k, v, a, beta, do = _inputs(B, T, H, T + H)
    comp = th.compile(th.programs.deltanet(B, H, T), target, q, k, v, a, beta, do)
    o, dq, dk, dv, da, dbeta = comp(q, k, v, a, beta, do)
    args = [_np(x) for x in (q, k, v, a, beta)]
    ro = interpret.deltanet_chunked(*args)
    assert relative(_np(o).reshape(B, T, H, 128), ro) < TOL
    grads = interpret.deltanet_grad(*args, _np(do))
    got = [_np(x) for x in (dq, dk, dv)] + [_np(da), _np(dbeta)]
    shapes = [(B, T, H, 128)] * 3 + [(B, T, H)] * 2
    for name, g, s, r in zip(("dq", "dk", "dv", "da", "dbeta"), got, shapes, grads):
        assert relative(g.reshape(s), r) < TOL, name


def test_forward_alone_matches_the_token_rule(target):
    import tempest_hip.launch as L
    announce("deltanet fwd")
    B, T, H = 1, 128, 2
    q, k, v, a, beta, _ = _inputs(B, T, H, 5)
    o = torch.empty_like(q)
    l = L.deltanet(B, H, T, q.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(), beta.data_ptr(), o.data_ptr())
    l()
    torch.cuda.synchronize()
    ref = interpret.deltanet_sequential(*(_np(x) for x in (q, k, v, a, beta)))
    assert relative(_np(o).reshape(B, T, H, 128), ref) < TOL


def test_config5_full_size_sampled_sequences(target):
    """B4 H16 T8192: every output computed on the GPU; two (batch, head)
    sequences checked against the float64 oracle."""
    import tempest_hip as th
    announce("deltanet config5 full")
    B, T, H = 4, 8192, 16
    q, k, v, a, beta, do = _inputs(B, T, H, 55)
    comp = th.compile(th.programs.deltanet(B, H, T), target, q, k, v, a, beta, do)
    o, dq, dk, dv, da, dbeta = comp(q, k, v, a, beta, do)
    for b, h in ((0, 0), (3, 9)):
        pick = lambda t: _np(t.view(B, T, H, -1)[b:b + 1, :, h:h + 1])  # noqa: E731
        pickg = lambda t: _np(t.view(B, T, H)[b:b + 1, :, h:h + 1])  # noqa: E731
        args = [pick(q), pick(k), pick(v), pickg(a), pickg(beta)]
        assert relative(pick(o), interpret.deltanet_chunked(*args)) < TOL
        grads = interpret.deltanet_grad(*args, pick(do))
        for name, g, r in zip(("dq", "dk", "dv", "da", "dbeta"),
                              (pick(dq), pick(dk), pick(dv), pickg(da), pickg(dbeta)), grads):
            assert relative(g, r) < TOL, (b, h, name)
