"""Config 4's oracle (attention forward and backward) against torch: the
scaled-dot-product definition in float64 and autograd for the gradients."""
import numpy as np
import pytest
import torch

from oracle import interpret
from oracle.data import relative


def _torch_attention(q, k, v, causal, scale):
    # (b, s, h, d) -> (b, h, s, d)
    qt, kt, vt = (x.permute(0, 2, 1, 3) for x in (q, k, v))
    s = qt @ kt.transpose(-1, -2) * scale
    if causal:
        S = s.shape[-1]
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    return (torch.softmax(s, dim=-1) @ vt).permute(0, 2, 1, 3), torch.logsumexp(s, dim=-1).permute(0, 2, 1)


@pytest.mark.parametrize("causal", [True, False])
def test_forward_and_backward_match_torch(causal):
    rng = np.random.default_rng(0)
    B, S, H, D = 2, 9, 3, 8
    q, k, v, g = (rng.normal(size=(B, S, H, D)) for _ in range(4))
    o, lse = interpret.attention_fwd(q, k, v, causal)
    t = [torch.tensor(a, requires_grad=True) for a in (q, k, v)]
    ot, lt = _torch_attention(*t, causal, 1 / np.sqrt(D))
    assert relative(o, ot.detach().numpy()) < 1e-13 and relative(lse, lt.detach().numpy()) < 1e-13
    (ot * torch.tensor(g)).sum().backward()
    dq, dk, dv = interpret.attention_bwd(q, k, v, g, causal)
    for ours, tt in zip((dq, dk, dv), t):
        assert relative(ours, tt.grad.numpy()) < 1e-12


def test_grouped_heads_read_their_group():
    rng = np.random.default_rng(1)
    q = rng.normal(size=(1, 5, 4, 8))
    k, v = rng.normal(size=(1, 5, 2, 8)), rng.normal(size=(1, 5, 2, 8))
    o, _ = interpret.attention_fwd(q, k, v, True)
    o2, _ = interpret.attention_fwd(q, np.repeat(k, 2, axis=2), np.repeat(v, 2, axis=2), True)
    assert np.allclose(o, o2)
    # Head 3 reads kv head 1: changing kv head 0 leaves it alone.
    k2 = k.copy()
    k2[:, :, 0] = rng.normal(size=k2[:, :, 0].shape)
    o3, _ = interpret.attention_fwd(q, k2, v, True)
    assert np.allclose(o3[:, :, 2:], o[:, :, 2:]) and not np.allclose(o3[:, :, :2], o[:, :, :2])


def test_causal_first_query_reads_only_the_first_key():
    rng = np.random.default_rng(2)
    q, k, v = (rng.normal(size=(1, 4, 1, 8)) for _ in range(3))
    o, lse = interpret.attention_fwd(q, k, v, True)
    assert np.allclose(o[0, 0, 0], v[0, 0, 0])
    assert np.isclose(lse[0, 0, 0], (q[0, 0, 0] @ k[0, 0, 0]) / np.sqrt(8))


@pytest.mark.parametrize("causal", [True, False])
def test_grouped_backward_matches_torch(causal):
    # Four query heads over two kv heads: torch's autograd through the
    # repeated keys and values sums each group's gradients.
    rng = np.random.default_rng(3)
    B, S, H, Hk, D = 2, 7, 4, 2, 8
    q, g = rng.normal(size=(B, S, H, D)), rng.normal(size=(B, S, H, D))
    k, v = rng.normal(size=(B, S, Hk, D)), rng.normal(size=(B, S, Hk, D))
    t = [torch.tensor(a, requires_grad=True) for a in (q, k, v)]
    kr, vr = (torch.repeat_interleave(x, H // Hk, dim=2) for x in t[1:])
    ot, _ = _torch_attention(t[0], kr, vr, causal, 1 / np.sqrt(D))
    (ot * torch.tensor(g)).sum().backward()
    dq, dk, dv = interpret.attention_bwd(q, k, v, g, causal)
    for ours, tt in zip((dq, dk, dv), t):
        assert ours.shape == tt.grad.shape
        assert relative(ours, tt.grad.numpy()) < 1e-12


def _sdpa(q, k, v, visible, scale):
    """torch's own scaled-dot-product attention (float64, CPU) under a boolean mask."""
    qt, kt, vt = (x.permute(0, 2, 1, 3) for x in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=torch.from_numpy(visible), scale=scale)
    return o.permute(0, 2, 1, 3)


def _starts(lengths):
    """1-based first key of each position of documents packed back to back."""
    return np.array([sum(lengths[:i]) + 1 for i in range(len(lengths)) for _ in range(lengths[i])])


@pytest.mark.parametrize("causal", [True, False])
def test_device_held_masks_match_torch(causal):
    """Packed documents (a first key per query) and key counts per sequence,
    with more keys than queries: the forward against torch's SDPA under the
    same boolean mask, the gradients against its autograd."""
    rng = np.random.default_rng(4)
    B, S, Sk, H, Hk, D = 2, 12, 12, 4, 2, 8
    q, g = rng.normal(size=(B, S, H, D)), rng.normal(size=(B, S, H, D))
    k, v = rng.normal(size=(B, Sk, Hk, D)), rng.normal(size=(B, Sk, Hk, D))
    starts = np.stack([_starts([5, 1, 6]), _starts([3, 9])])
    lengths = np.array([12, 10])
    visible = interpret.attention_visible(B, S, Sk, causal, starts, lengths)
    # Every query sees a key: its document's first key lies before it and inside the length.
    assert visible.any(axis=-1).all()
    t = [torch.tensor(a, requires_grad=True) for a in (q, k, v)]
    kr, vr = (torch.repeat_interleave(x, H // Hk, dim=2) for x in t[1:])
    ot = _sdpa(t[0], kr, vr, visible, 1 / np.sqrt(D))
    o, _ = interpret.attention_fwd(q, k, v, causal, starts=starts, lengths=lengths)
    assert relative(o, ot.detach().numpy()) < 1e-12
    (ot * torch.tensor(g)).sum().backward()
    dq, dk, dv = interpret.attention_bwd(q, k, v, g, causal, starts=starts, lengths=lengths)
    for ours, tt in zip((dq, dk, dv), t):
        assert relative(ours, tt.grad.numpy()) < 1e-12


def test_a_document_start_sees_only_itself_and_decode_reads_its_length():
    """Closed forms: a causal query at its document's first position attends
    to its own key alone, so o = v there; one query over a cache of 9 keys
    of which 4 are held is the softmax over those 4 (test/cuda/attention.jl:254-271)."""
    rng = np.random.default_rng(5)
    q, k, v = (rng.normal(size=(1, 6, 1, 4)) for _ in range(3))
    starts = _starts([2, 4])[None]
    o, _ = interpret.attention_fwd(q, k, v, True, starts=starts)
    assert np.allclose(o[0, 2, 0], v[0, 2, 0]) and np.allclose(o[0, 0, 0], v[0, 0, 0])
    qd = rng.normal(size=(1, 1, 1, 4))
    kd, vd = rng.normal(size=(1, 9, 1, 4)), rng.normal(size=(1, 9, 1, 4))
    od, lse = interpret.attention_fwd(qd, kd, vd, False, lengths=np.array([4]))
    s = kd[0, :4, 0] @ qd[0, 0, 0] / 2.0
    w = np.exp(s - s.max())
    assert np.allclose(od[0, 0, 0], (w / w.sum()) @ vd[0, :4, 0])
    assert np.isclose(lse[0, 0, 0], np.log(np.exp(s).sum()))
