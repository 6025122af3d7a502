"""fp32 attention on the matrix cores (v_mfma_f32_32x32x2_f32, exact fp32
products and sums) at head dims 64 and 128: causal or not, grouped heads,
lengths that are not multiples of the 64-position tiles, more or fewer keys
than queries.  Forward (o, lse) and backward (dq, dk, dv) against the float64
oracle on the same inputs, to the fp32 tolerance; and the kernels that ran
are the matrix-core ones."""
import pytest
import torch

from conftest import announce
from test_gpu_attention_general import TOL_F32, _check, _run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,H,KV,S,Sk,B,causal", [
    (64, 4, 2, 300, 300, 2, True), (64, 2, 2, 96, 250, 2, False), (64, 2, 2, 100, 180, 1, True),
    (128, 2, 1, 129, 129, 2, True), (128, 3, 3, 200, 77, 1, False), (64, 8, 8, 1024, 1024, 1, True),
    (128, 2, 2, 256, 256, 2, True)])
def test_fp32_attention_on_matrix_cores(target, D, H, KV, S, Sk, B, causal):
    announce("attn fp32 mfma", D, H, KV, S, Sk, B, causal)
    gen = torch.Generator(device="cuda").manual_seed(D * 7 + S + Sk + H)
    q = torch.randn(B, S, H, D, device="cuda", generator=gen) * 0.5
    k = torch.randn(B, Sk, KV, D, device="cuda", generator=gen) * 0.5
    v = torch.randn(B, Sk, KV, D, device="cuda", generator=gen)
    g = torch.randn(B, S, H, D, device="cuda", generator=gen)
    outs, (fwd, bwd) = _run(q, k, v, g, causal, True)
    assert f"f32_attn_fwd_d{D}" in fwd.describe(), fwd.describe()
    assert f"f32_attn_dkdv_d{D}" in bwd.describe() and f"f32_attn_dq_d{D}" in bwd.describe(), bwd.describe()
    _check(outs, q, k, v, g, causal, TOL_F32)


def test_fp32_attention_replays_bitwise(target):
    """No atomics: the same inputs give the same bits on every run."""
    announce("attn fp32 mfma repeat")
    gen = torch.Generator(device="cuda").manual_seed(5)
    q, k, v, g = (torch.randn(2, 384, 4, 64, device="cuda", generator=gen) for _ in range(4))
    (o, lse, dq, dk, dv), (fwd, bwd) = _run(q, k, v, g, True, True)
    first = [t.clone() for t in (o, lse, dq, dk, dv)]
    for _ in range(3):
        fwd()
        bwd()
    torch.cuda.synchronize()
    for a, b in zip(first, (o, lse, dq, dk, dv)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("D,B,H,KV,S,causal,split", [
    (64, 1, 2, 2, 700, True, True), (128, 1, 2, 1, 300, False, True), (64, 4, 16, 16, 512, True, False)])
def test_fp32_split_and_whole_sweeps(target, D, B, H, KV, S, causal, split):
    """A grid under one workgroup a CU splits each sweep into parts (partial
    results combined or summed in part order); a grid that fills the device
    sweeps whole.  Both against the float64 oracle."""
    announce("attn fp32 mfma split", D, B, H, KV, S, causal, split)
    gen = torch.Generator(device="cuda").manual_seed(17 * D + S + H)
    q = torch.randn(B, S, H, D, device="cuda", generator=gen) * 0.5
    k = torch.randn(B, S, KV, D, device="cuda", generator=gen) * 0.5
    v = torch.randn(B, S, KV, D, device="cuda", generator=gen)
    g = torch.randn(B, S, H, D, device="cuda", generator=gen)
    outs, (fwd, bwd) = _run(q, k, v, g, causal, True)
    assert ("f32_attn_combine" in fwd.describe()) == split, fwd.describe()
    assert ("f32_attn_sum_dk" in bwd.describe() and "f32_attn_sum_dq" in bwd.describe()) == split, bwd.describe()
    _check(outs, q, k, v, g, causal, TOL_F32)
