"""CPU pins of the GEMM correctness rule and of the precision-probe operands.

The GEMM rule is the reference's torch.testing.assert_close(C, R, rtol=t,
atol=t) (reference bench_tensor.py:289-299): every entry must satisfy
|C - R| <= atol + rtol*|R|. Both the oracle (oracle.tensor.check_gemm) and the
product (gemm.validate, run here on CPU tensors) are pinned against
known answers chosen so that plausible mistakes fail: a normwise rule
(max|C-R| / max|R|) accepts a near-zero entry that is off by more than atol;
swapping rtol*|R| for rtol*|C|, or dropping atol, changes a boundary verdict;
NaN must fail. torch.testing.assert_close, a library routine, is the
independent referee on random cases.

The probe operands (reference bench_tensor.py:675-757) are pinned by what
they must detect: rounding the FP32 probe to TF32, BF16 or FP16 changes its
exact product with the identity, rounding the FP64 probe to FP32 changes its
product, and permuting its rows is visible. An IEEE product of each returns
it exactly.
"""

import numpy as np
import pytest
import torch

from oracle import tensor as ot
from triton_chip_benchmarks_amd import bench_tensor, gemm


def _product_passes(actual, reference, dtype):
    try:
        gemm.validate(torch.as_tensor(actual), torch.as_tensor(reference, dtype=torch.float64), dtype)
        return True
    except RuntimeError:
        return False


def _oracle_passes(actual, reference, dtype):
    try:
        ot.check_gemm(np.asarray(actual), np.asarray(reference), dtype)
        return True
    except AssertionError:
        return False


def _referee(actual, reference, tolerance):
    try:
        torch.testing.assert_close(torch.as_tensor(actual, dtype=torch.float64),
                                   torch.as_tensor(reference, dtype=torch.float64),
                                   rtol=tolerance, atol=tolerance, equal_nan=False)
        return True
    except AssertionError:
        return False


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp64"])
def test_small_entry_off_by_more_than_atol_fails_although_normwise_passes(dtype):
    tolerance = ot.GEMM_TOLERANCE[dtype]
    reference = np.array([[0.0, 100.0], [-50.0, 3.0]])
    actual = reference.copy()
    actual[0, 0] = 1.5 * tolerance            # |R| = 0, so the allowed error is atol alone
    normwise = np.abs(actual - reference).max() / np.abs(reference).max()
    assert normwise <= tolerance              # a normwise rule would accept this
    assert not _oracle_passes(actual, reference, dtype)
    assert not _product_passes(actual, reference, dtype)
    assert not _referee(actual, reference, tolerance)


@pytest.mark.parametrize("dtype", ["bf16", "fp64"])
def test_boundary_uses_the_reference_magnitude_and_keeps_atol(dtype):
    t = ot.GEMM_TOLERANCE[dtype]
    reference = np.array([1000.0, 0.0, -8.0])
    inside = reference + np.array([0.99 * (t + t * 1000.0), 0.99 * t, -0.99 * (t + 8 * t)])
    assert _oracle_passes(inside, reference, dtype) and _product_passes(inside, reference, dtype)
    # Without atol the |R| = 0 entry would fail; without rtol the large entries would.
    assert not np.all(np.abs(inside - reference) <= t * np.abs(reference))
    assert not np.all(np.abs(inside - reference) <= t)
    # rtol applies to |R|, not |C|: at R = 0, C = t(1 + t/2) is within t + t|C| but not within t + t|R|.
    reference2, actual2 = np.array([0.0]), np.array([t * (1 + t / 2)])
    assert np.abs(actual2 - reference2)[0] <= t + t * np.abs(actual2)[0]
    assert not _oracle_passes(actual2, reference2, dtype)
    assert not _product_passes(actual2, reference2, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "fp64", "int8", "fp8", "fp4"])
def test_non_finite_output_fails(dtype):
    reference = np.zeros((2, 2))
    for bad in (np.nan, np.inf):
        actual = reference.copy()
        actual[1, 1] = bad
        assert not _oracle_passes(actual, reference, dtype)
        assert not _product_passes(actual, reference, dtype)


@pytest.mark.parametrize("dtype", ["int8", "fp8", "fp4"])
def test_exact_formats_reject_one_ulp(dtype):
    reference = np.array([[256.0, -3.0]])
    actual = reference.copy()
    actual[0, 1] = np.nextafter(-3.0, 0.0, dtype=np.float32)
    assert not _oracle_passes(actual, reference, dtype)
    assert not _product_passes(actual, reference, dtype)
    assert _oracle_passes(reference.copy(), reference, dtype)
    assert _product_passes(reference.copy(), reference, dtype)


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32", "fp64"])
def test_verdicts_agree_with_torch_assert_close_on_random_perturbations(dtype):
    tolerance = ot.GEMM_TOLERANCE[dtype]
    rng = np.random.default_rng(5)
    outcomes = set()
    for trial in range(200):
        reference = rng.standard_normal((6, 5)) * 10.0 ** rng.integers(-3, 4)
        reference[rng.integers(0, 6), rng.integers(0, 5)] = 0.0
        scale = tolerance * rng.choice([0.3, 0.9, 1.1, 3.0])
        actual = reference + rng.standard_normal(reference.shape) * scale * (1 + np.abs(reference))
        expected = _referee(actual, reference, tolerance)
        outcomes.add(expected)
        assert _oracle_passes(actual, reference, dtype) == expected, trial
        assert _product_passes(actual, reference, dtype) == expected, trial
    assert outcomes == {True, False}


def test_checksum_bound_holds_for_a_passing_output_and_is_implied():
    rng = np.random.default_rng(9)
    a, b = rng.standard_normal((64, 96)), rng.standard_normal((96, 48))
    reference = ot.gemm_reference(a, b)
    t = ot.GEMM_TOLERANCE["bf16"]
    actual = reference + (t + t * np.abs(reference)) * rng.uniform(-1, 1, reference.shape)
    ot.check_gemm(actual, reference, "bf16")
    assert np.all(np.abs(actual.sum(axis=0) - reference.sum(axis=0)) <= ot.checksum_tolerance(a, b, "bf16", 0))
    assert np.all(np.abs(actual.sum(axis=1) - reference.sum(axis=1)) <= ot.checksum_tolerance(a, b, "bf16", 1))
    # A systematic error of 2x the elementwise allowance on one column breaks its checksum bound.
    broken = reference.copy()
    broken[:, 3] += 2 * (t + t * ot.gemm_reference(np.abs(a), np.abs(b))[:, 3])
    assert np.abs(broken.sum(axis=0) - reference.sum(axis=0))[3] > ot.checksum_tolerance(a, b, "bf16", 0)[3]


def _round_mantissa(values, bits):
    """Round float32 values to `bits` explicit mantissa bits, nearest-even (TF32: 10)."""
    as_int = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    drop = 23 - bits
    half = 1 << (drop - 1)
    keep = (as_int >> drop) & 1
    rounded = ((as_int + half - 1 + keep) >> drop) << drop
    return rounded.astype(np.uint32).view(np.float32).astype(np.float64)


def test_fp32_probe_detects_tf32_bf16_and_fp16_and_passes_ieee():
    a, b = ot.fp32_precision_probe()
    exact = ot.gemm_reference(a, b)
    assert np.array_equal(exact, a)
    ieee = (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float64)
    assert np.array_equal(ieee, exact)
    tf32 = ot.gemm_reference(_round_mantissa(a, 10), _round_mantissa(b, 10))
    bf16 = ot.gemm_reference(torch.from_numpy(a).to(torch.bfloat16).double().numpy(), b)
    with np.errstate(over="ignore", invalid="ignore"):
        fp16 = ot.gemm_reference(a.astype(np.float16).astype(np.float64), b)
    for rounded in (tf32, bf16, fp16):
        assert not np.array_equal(rounded, exact)
    # Each constant has its own job: 1+2^-12 is lost by TF32, 1+2^-9 only by BF16 and 2^20 only by FP16.
    assert tf32[0, 1] == exact[0, 1] and bf16[0, 1] != exact[0, 1]
    assert tf32[1, 1] != exact[1, 1]
    assert np.isinf(fp16[0, 2]) and tf32[0, 2] == exact[0, 2] and bf16[0, 2] == exact[0, 2]
    # The product's probe operand is the oracle's.
    assert np.array_equal(bench_tensor.fp32_probe_matrix().double().numpy(), a)


def test_fp64_probe_detects_fp32_fallback_and_row_permutation():
    a, b = ot.fp64_precision_probe()
    exact = ot.gemm_reference(a, b)
    assert np.array_equal(exact[:, :16], a) and not exact[:, 16:].any()
    fp32 = ot.gemm_reference(a.astype(np.float32).astype(np.float64), b)
    assert not np.array_equal(fp32, exact)
    permuted = exact[np.roll(np.arange(32), 1)]
    assert not np.array_equal(permuted, exact)
    assert sorted(map(tuple, permuted.tolist())) == sorted(map(tuple, exact.tolist()))
    assert np.array_equal(bench_tensor.fp64_probe_matrix().numpy(), a)


def test_mx_scale_blocks_layout():
    """formats.mx_scale_blocks: [rows][K/32] -> [ceil(K/256)][rows][8], block b row r group g = scale of
    row r for K elements 256b+32g.., padding 127; checked entry by entry on a ragged K."""
    from triton_chip_benchmarks_amd import formats

    rows, groups = 5, 19  # K = 608: three blocks, the last holding 3 groups
    scales = torch.arange(rows * groups, dtype=torch.uint8).view(rows, groups)
    blocks = formats.mx_scale_blocks(scales)
    assert blocks.shape == (3, rows, 8) and blocks.is_contiguous()
    for b in range(3):
        for r in range(rows):
            for g in range(8):
                expected = int(scales[r, 8 * b + g]) if 8 * b + g < groups else 127
                assert int(blocks[b, r, g]) == expected
    # One K step (block b) of rows r0..r0+n-1 is one contiguous run of 8*n bytes.
    flat = blocks.reshape(-1)
    assert flat[(1 * rows + 2) * 8:(1 * rows + 4) * 8].tolist() == blocks[1, 2:4].reshape(-1).tolist()


def test_crosscheck_bf16_library_c_is_held_to_one_bf16_ulp_of_the_exact_c():
    """The MXFP4 cross-check compares the library's BF16 C with the suite's exact FP32 C, entry by entry.

    One BF16 ulp of an exact value x = m * 2^e (0.5 <= |m| < 1) is 2^(e-8): 2 for 257 (values in [256, 512)
    are spaced by 2), 4 for 1000.25. Known answers: round-to-nearest and truncation both stay within one ulp;
    1008 for 1000.25 is 1.94 ulps off and fails; a nonzero entry where the exact C is 0 fails.
    """
    import math

    from triton_chip_benchmarks_amd import crosscheck

    exact = torch.tensor([0.0, 1.0, 3.0, 257.0, 1000.25, -5500.0, 0.75], dtype=torch.float32)
    assert [math.ldexp(1.0, math.frexp(x)[1] - 8) for x in (257.0, 1000.25)] == [2.0, 4.0]
    nearest = exact.to(torch.bfloat16)
    fields = crosscheck._agreement("fp4", nearest, exact, torch)
    assert fields["library_output"] == "bf16" and fields["elementwise_within_one_bf16_ulp"]
    assert fields["max_bf16_ulps"] <= 0.5
    truncated = (exact.view(torch.int32) & ~0xFFFF).view(torch.float32).to(torch.bfloat16)
    fields = crosscheck._agreement("fp4", truncated, exact, torch)
    assert fields["elementwise_within_one_bf16_ulp"] and 0.5 < fields["max_bf16_ulps"] < 1.0
    planted = nearest.clone()
    planted[4] = 1004.0                                          # 3.75 off: within one ulp of 4
    assert crosscheck._agreement("fp4", planted, exact, torch)["elementwise_within_one_bf16_ulp"]
    planted[4] = 1008.0                                          # 7.75 off: 1.94 ulps
    fields = crosscheck._agreement("fp4", planted, exact, torch)
    assert not fields["elementwise_within_one_bf16_ulp"] and fields["max_bf16_ulps"] == pytest.approx(7.75 / 4)
    planted = nearest.clone()
    planted[0] = 2.0**-20                                        # the exact C is 0 there
    assert not crosscheck._agreement("fp4", planted, exact, torch)["elementwise_within_one_bf16_ulp"]
    same = crosscheck._agreement("fp8", exact.clone(), exact, torch)
    assert same == {"normwise_difference": 0.0}
    rounded_sums = crosscheck._agreement("bf16", nearest, exact, torch)    # BF16 operands: normwise only
    assert set(rounded_sums) == {"normwise_difference"}
