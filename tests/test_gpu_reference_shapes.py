"""The programs the reference itself times, at its shapes, through this build
(bench.py's reference_benchmarks): causal attention with 64 features (bf16 and
fp32, forward and a training step whose loss is sum(abs2, o)), the coverage
suite's column programs over a 512 x 1024 matrix (softmax through logsumexp,
the two-pass layer norm, RMSNorm) and "linear, bias, GELU" in fp32
(test/fixtures/compositions.jl:41-138; TRIALS.md:2155-2187).  Each result
against float64 torch on the same inputs, to the tolerances the north star
states: bf16 attention within 2e-2 relative, fp32 work within 1e-5."""
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2
TOL_F32 = 1e-5


def test_reference_shapes_match_float64(target):
    import bench
    announce("reference shapes")
    rows = bench.reference_benchmarks(target)
    assert set(rows) == set(bench.REFERENCE_US)
    for name, row in rows.items():
        errs = row["rel_err"] if isinstance(row["rel_err"], dict) else {"y": row["rel_err"]}
        tol = TOL_BF16 if "bf16" in name else TOL_F32
        for what, e in errs.items():
            assert e < tol, (name, what, e)
        assert row["us_fwd"] > 0 and all(v > 0 for k, v in row.items() if k.startswith("us_"))
    # bf16 attention at 64 features runs on the matrix cores; fp32 products on their own kernels.
    assert "mfma_attn_fwd_d64" in rows["attention_bf16_D64_H8_B2_S1024_causal"]["kernels"][0]
    assert "gemm_f32" in rows["linear_bias_gelu_256x384x512_f32"]["kernels"][0]
