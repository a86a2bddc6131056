"""CPU tests of the GEMM operand recipes (gemm.gemm_inputs), run on CPU tensors.

The reference recipe (bench_tensor.py:249-261) is pinned by the properties its
definition fixes: A ~ N(0, 1) and B ~ N(0, 1) / sqrt(K) (standard deviations to
within sampling error), INT8 over exactly {-1, 0, 1} in equal shares, B stored
[N][K] and contiguous, values that round-trip through the storage format, and
FP8/FP4 refused with the reference's reasons. The baseline recipe keeps the
benchmark configuration's sets.
"""

import math

import numpy as np
import pytest
import torch

from triton_chip_benchmarks_amd import gemm


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32", "fp64"])
def test_reference_recipe_scales_b_by_one_over_sqrt_k(dtype):
    m, n, k = 192, 256, 1024
    a, b, c, scales, a_values, b_values = gemm.gemm_inputs(dtype, m, n, k, "cpu", 3, inputs="reference")
    assert scales is None
    assert tuple(a.shape) == (m, k) and tuple(b.shape) == (n, k) and b.is_contiguous()
    assert tuple(c.shape) == (m, n)
    assert c.dtype == (torch.float64 if dtype == "fp64" else torch.float32)
    assert torch.equal(a_values, a.double()) and torch.equal(b_values, b.double())
    a_std, b_std = a_values.std().item(), b_values.std().item()
    # 196608 and 262144 samples: the standard deviation is within 1% of its true value.
    assert a_std == pytest.approx(1.0, rel=0.01)
    assert b_std == pytest.approx(1.0 / math.sqrt(k), rel=0.01)
    assert abs(a_values.mean().item()) < 0.01 and abs(b_values.mean().item()) < 0.01 / math.sqrt(k) * 4
    # |C| ~ N(0, 1) per entry: the scaling is what keeps one tolerance useful at every K (bench_tensor.py:250-251).
    product = a_values @ b_values.t()
    assert product.std().item() == pytest.approx(1.0, rel=0.05)


def test_reference_recipe_int8_is_ternary():
    a, b, c, _s, a_values, b_values = gemm.gemm_inputs("int8", 300, 200, 512, "cpu", 5, inputs="reference")
    assert a.dtype == torch.int8 and b.dtype == torch.int8 and c.dtype == torch.int32
    for values in (a_values, b_values):
        counts = np.bincount(values.numpy().astype(np.int64).ravel() + 1, minlength=3)
        assert len(counts) == 3 and counts.sum() == values.numel()
        assert np.all(np.abs(counts / values.numel() - 1 / 3) < 0.01)


@pytest.mark.parametrize("dtype", ["fp8", "fp4"])
def test_reference_recipe_refuses_fp8_and_fp4_as_the_reference_does(dtype):
    with pytest.raises(ValueError, match="in --mode peak only"):
        gemm.gemm_inputs(dtype, 64, 64, 256, "cpu", 0, inputs="reference")
    assert gemm.REFERENCE_REFUSAL[dtype].endswith("in --mode peak only")


def test_baseline_recipe_is_unscaled_and_keeps_its_sets():
    _a, _b, _c, _s, a_values, b_values = gemm.gemm_inputs("fp16", 128, 128, 1024, "cpu", 3)
    assert b_values.std().item() == pytest.approx(1.0, rel=0.02)
    _a, _b, _c, _s, a_values, _bv = gemm.gemm_inputs("int8", 64, 64, 512, "cpu", 3)
    assert set(np.unique(a_values.numpy())) <= set(range(-8, 9)) and a_values.abs().max().item() == 8
    with pytest.raises(ValueError):
        gemm.gemm_inputs("fp16", 64, 64, 64, "cpu", 0, inputs="other")


def test_stated_tolerance_ratio_rescales_the_allowance():
    """max_error_over_stated is the same entries' error against the configuration's looser 1e-2 bound."""
    reference = torch.tensor([[0.0, 100.0]], dtype=torch.float64)
    actual = (reference + torch.tensor([[0.001, 0.1]], dtype=torch.float64)).float()
    result = gemm.validate(actual, reference, "bf16")
    assert result["rtol"] == result["atol"] == 2e-3
    worst = max(0.001 / (2e-3), 0.1 / (2e-3 + 2e-3 * 100.0))
    assert result["max_error_over_allowed"] == pytest.approx(worst, rel=1e-6)
    assert result["stated_tolerance"] == 1e-2
    assert result["max_error_over_stated"] == pytest.approx(worst * 2e-3 / 1e-2, rel=1e-6)
    strict = gemm.validate(actual, reference, "bf16", tolerance=1e-2)
    assert strict["rtol"] == 1e-2
