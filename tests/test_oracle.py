"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something a plausible mistake would
fail: the reference's published numbers (tests/golden/reference_published.json,
extracted from its result files), its tests' known answers, brute force with
exact rational arithmetic, closed forms, and torch's own format conversions.
"""

from fractions import Fraction
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import memory, tensor as ot, vector as ov

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_published.json").read_text())


# ---- exact rational rounding, the brute-force checker ------------------------------------------

def round_fraction(value: Fraction, precision: int, emin: int) -> Fraction:
    """Round-to-nearest-even of an exact rational to a binary format (no overflow handling)."""
    if value == 0:
        return Fraction(0)
    sign = -1 if value < 0 else 1
    magnitude = abs(value)
    exponent = magnitude.numerator.bit_length() - magnitude.denominator.bit_length()
    if Fraction(2) ** exponent > magnitude:
        exponent -= 1
    exponent = max(exponent, emin)
    quantum = Fraction(2) ** (exponent - (precision - 1))
    scaled = magnitude / quantum
    floor = scaled.numerator // scaled.denominator
    remainder = scaled - floor
    if remainder > Fraction(1, 2) or (remainder == Fraction(1, 2) and floor % 2 == 1):
        floor += 1
    return sign * floor * quantum


F32 = (24, -126)
F16 = (11, -14)
BF16 = (8, -126)


# ---- vector oracle ----------------------------------------------------------------------------

def test_fp32_chain_matches_exact_rounding_step_by_step():
    rng = np.random.default_rng(0)
    x = rng.uniform(0.125, 1.0, 64).astype(np.float32).astype(np.float64)
    a, b = float(np.float32(1 - 2.0**-14)), float(np.float32(3 * 2.0**-16))
    inputs = np.tile(x, (8, 1))
    coefficients = np.array([a] + [b] * 8)
    emulated = ov.run_chains("fp32", inputs, coefficients, 7)[0]
    for lane in range(64):
        value = Fraction(x[lane])
        for _ in range(7):
            value = round_fraction(value * Fraction(a) + Fraction(b), *F32)
        assert emulated[lane] == float(value)


@pytest.mark.parametrize("dtype,fmt", [("fp16", F16), ("bf16", BF16)])
@pytest.mark.parametrize("widened", [False, True])
def test_narrow_chain_matches_exact_rounding(dtype, fmt, widened):
    rng = np.random.default_rng(1)
    x = ov.round_narrow(rng.uniform(-3, 3, 200), dtype)
    a = float(ov.round_narrow(np.array([0.7071]), dtype)[0])
    b = float(ov.round_narrow(np.array([0.01]), dtype)[0])
    got = ov.run_chains(dtype, np.tile(x, (8, 1)), np.array([a] + [b] * 8), 5, widened=widened)[3]
    for lane in range(200):
        value = Fraction(x[lane])
        for _ in range(5):
            exact = value * Fraction(a) + Fraction(b)
            value = round_fraction(round_fraction(exact, *F32), *fmt) if widened else round_fraction(exact, *fmt)
        assert got[lane] == float(value), (lane, got[lane], float(value))


def test_widened_and_single_rounding_differ_somewhere():
    """The two narrow semantics are distinguishable, so tests choosing one mean something."""
    rng = np.random.default_rng(2)
    x = ov.round_narrow(rng.uniform(0.5, 1.0, 20000), "bf16")
    a = ov.round_narrow(rng.uniform(0.5, 1.0, 20000), "bf16")
    # A tiny addend puts the exact sum just off a product that sits on a bf16
    # midpoint; rounding through fp32 first lands on the midpoint and ties to even.
    b = ov.round_narrow(rng.uniform(2.0**-30, 2.0**-28, 20000), "bf16")
    differ = 0
    for i in range(20000):
        single = ov.run_chains("bf16", np.full((1, 1), x[i]), np.array([a[i], b[i]]), 1, widened=False)[0, 0]
        widened = ov.run_chains("bf16", np.full((1, 1), x[i]), np.array([a[i], b[i]]), 1, widened=True)[0, 0]
        differ += single != widened
        if differ:
            break
    assert differ


def test_round_narrow_matches_torch_and_numpy_conversions():
    import torch

    rng = np.random.default_rng(3)
    values = np.concatenate([rng.standard_normal(5000) * 10.0 ** rng.integers(-8, 5, 5000),
                             [0.0, -0.0, 1e-8, 6.0e-8, 65504.0, 65519.0, 2.0**-24, 3 * 2.0**-26]])
    assert np.array_equal(ov.round_narrow(values, "fp16"), values.astype(np.float16).astype(np.float64))
    as32 = values.astype(np.float32)
    expected = torch.from_numpy(as32).to(torch.bfloat16).double().numpy()
    assert np.array_equal(ov.round_narrow(as32.astype(np.float64), "bf16"), expected)


def test_fp32_closed_form_tolerance_equals_published_value():
    """The reference's check on its default inputs yields its published bound (bw1100 and H20)."""
    golden = GOLDEN["vector_fp32"]
    assert golden["max_abs_tolerance"] == GOLDEN["vector_fp32_h20"]["max_abs_tolerance"]
    inputs, coefficients = ov.reference_inputs("fp32", 2048, np.random.default_rng(4))
    output = ov.run_chains("fp32", inputs, coefficients, golden["iterations"])
    result = ov.closed_form_check(inputs, output, coefficients, golden["iterations"], "fp32")
    assert result["max_abs_tolerance"] == pytest.approx(golden["max_abs_tolerance"], rel=1e-12)
    # The emulated error has the published magnitude (both are ~1e-4 and below the bound).
    assert 0.2 * golden["max_abs_error"] < result["max_abs_error"] < golden["max_abs_tolerance"]
    # A chain run with the wrong bias (b_6 instead of b_5) drifts well past the bound.
    output[5] = ov.run_chains("fp32", inputs[5:6], coefficients[[0, 7]], golden["iterations"])[0]
    with pytest.raises(AssertionError):
        ov.closed_form_check(inputs, output, coefficients, golden["iterations"], "fp32")


def test_fp64_closed_form_tolerance_equals_published_value():
    golden = GOLDEN["vector_fp64"]
    inputs, coefficients = ov.reference_inputs("fp64", 1024, np.random.default_rng(5))
    output = ov.run_chains("fp64", inputs, coefficients, golden["iterations"])
    result = ov.closed_form_check(inputs, output, coefficients, golden["iterations"], "fp64")
    assert result["max_abs_tolerance"] == pytest.approx(golden["max_abs_tolerance"], rel=1e-12)
    assert result["max_abs_error"] < golden["max_abs_tolerance"]
    output[0, 0] += 1e-8  # the reference's own corruption check (tests/test_vector_dtypes.py:150-160)
    with pytest.raises(AssertionError):
        ov.closed_form_check(inputs, output, coefficients, golden["iterations"], "fp64")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_involution_is_exact_and_odd_iterations_reject_identity(dtype):
    inputs, coefficients = ov.reference_inputs(dtype, 31, np.random.default_rng(6))
    for iterations in (1, 2, 3, 32, 33):
        output = ov.run_chains(dtype, inputs, coefficients, iterations)
        result = ov.closed_form_check(inputs, output, coefficients, iterations, dtype)
        assert result["max_abs_error"] == 0 and result["max_abs_tolerance"] == 0
    with pytest.raises(AssertionError):
        ov.closed_form_check(inputs, inputs, coefficients, 33, dtype)


def test_int8_dot4_brute_force_matches_transition_table():
    assert ov.signed_bytes(ov.pack_bytes(GOLDEN["int8_weights"]["weights"])) == GOLDEN["int8_weights"]["weights"]
    inputs, coefficients = ov.reference_inputs("int8", 43, np.random.default_rng(7))
    for iterations in (1, 2, 3, 32, 4096):
        output = ov.run_chains("int8", inputs, coefficients, iterations)
        ov.int8_transition_check(inputs, output, coefficients, iterations)
    output[3, 7] += 1
    with pytest.raises(AssertionError):
        ov.int8_transition_check(inputs, output, coefficients, 4096)


def test_int8_naive_recurrence_agrees_with_emulation():
    inputs, coefficients = ov.reference_inputs("int8", 16, np.random.default_rng(8))
    weights = ov.signed_bytes(coefficients[0])
    state = inputs.astype(np.int64)
    for _ in range(50):
        state = ov.dot4_reference(state, weights) + coefficients[1:, None].astype(np.int64)
    assert np.array_equal(ov.run_chains("int8", inputs, coefficients, 50), state)


def test_operation_counts_match_published_rows():
    for key in ("vector_fp32", "vector_fp32_h20"):
        golden = GOLDEN[key]
        assert ov.operation_count("fp32", golden["elements_per_chain"], golden["iterations"]) == golden["counted_flops"]
    assert ov.operation_count("int8", 17, 32) == 8 * 8 * 17 * 32  # tests/test_vector_dtypes.py:46-57


def test_baseline_inputs_bf16_are_the_degenerate_fixed_point():
    """b = 0.999 rounds to 1.0 in bf16 and c = 1e-3 is below half an ulp, so states never move."""
    inputs, coefficients = ov.baseline_inputs("bf16", 64, np.random.default_rng(9))
    assert coefficients[0] == 1.0
    assert np.array_equal(ov.run_chains("bf16", inputs, coefficients, 4096), inputs)


# ---- tensor oracle ----------------------------------------------------------------------------

def test_peak_tolerance_and_op_count_match_published_rows():
    golden = GOLDEN["tensor_bf16_peak"]
    assert ot.peak_tolerance("bf16", golden["config"]["block_k"], golden["iterations"]) == golden["atol"]
    cfg = golden["config"]
    assert ot.peak_operation_count(cfg["block_m"], cfg["block_n"], cfg["block_k"], golden["iterations"],
                                   cfg["chains"], golden["blocks"]) == golden["operation_count"]
    golden = GOLDEN["tensor_int8_peak"]
    cfg = golden["config"]
    assert ot.peak_tolerance("int8", cfg["block_k"], golden["iterations"]) == golden["atol"] == 0
    assert ot.peak_operation_count(cfg["block_m"], cfg["block_n"], cfg["block_k"], golden["iterations"],
                                   cfg["chains"], golden["blocks"]) == golden["operation_count"]
    bounds = GOLDEN["peak_tolerance"]
    tolerance = ot.peak_tolerance("bf16", bounds["bf16_block_k"], bounds["iterations"])
    assert bounds["above"] < tolerance < bounds["below"]
    assert ot.peak_tolerance("fp64", 16, 1024) < ot.peak_tolerance("fp32", 16, 1024)


def test_e2m1_table_packing_and_scales():
    golden = GOLDEN["e2m1_packing"]
    codes = np.array(golden["codes"], dtype=np.uint8)
    assert ot.pack_e2m1(codes).tolist() == golden["packed"]
    assert np.array_equal(ot.unpack_e2m1(ot.pack_e2m1(codes)), codes)
    for code, value in golden["values"].items():
        assert ot.e2m1_decode(int(code)) == value
    assert np.array_equal(ot.e2m1_decode(np.arange(16)), ot.E2M1_VALUES)
    assert ot.e8m0_decode(127) == 1.0 and ot.e8m0_decode(128) == 2.0 and np.isnan(ot.e8m0_decode(255))


def test_fp8_decoder_matches_torch_for_every_code():
    import torch

    codes = np.arange(256, dtype=np.uint8)
    expected = torch.from_numpy(codes).view(torch.float8_e4m3fn).double().numpy()
    got = ot.fp8_e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(expected))
    assert np.array_equal(got[~np.isnan(got)], expected[~np.isnan(expected)])
    values = np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0, 1 / 16, 448.0])
    assert np.array_equal(ot.fp8_e4m3fn_decode(ot.fp8_e4m3fn_encode_exact(values)), values)


def test_peak_reference_is_iterations_times_the_tile_product():
    rng = np.random.default_rng(10)
    a = ot.ternary_lattice(rng, (2, 8, 16))
    b = ot.ternary_lattice(rng, (2, 2, 16, 8))
    reference = ot.peak_reference(a, b, 5)
    brute = np.zeros_like(reference)
    for c in range(2):
        for w in range(2):
            for i in range(8):
                for j in range(8):
                    brute[c, w, i, j] = 5 * sum(a[w, i, k] * b[c, w, k, j] for k in range(16))
    assert np.array_equal(reference, brute)
    wrong = reference.copy()
    wrong[1, 1, 2, 3] += 1 / 256  # one lattice step, what a dropped dot changes
    with pytest.raises(AssertionError):
        ot.check_peak(wrong, reference, "bf16", 16, 5)


def test_one_hot_rows_have_exactly_one_entry_and_make_every_dot_a_lattice_step():
    """The reference's FP8 A (bench_tensor.py:651-658): each row one 1/16 at a K position, so against
    B = +-1/16 every dot is exactly +-1/256. A hot entry on the wrong axis, two per row, or the wrong
    value breaks one of these."""
    rng = np.random.default_rng(12)
    a = ot.one_hot_rows(rng, (3, 64, 32))
    assert a.shape == (3, 64, 32)
    assert np.array_equal(np.count_nonzero(a, axis=-1), np.ones((3, 64), dtype=np.int64))
    assert set(np.unique(a)) == {0.0, 1 / 16}
    # The hot positions cover the K axis (uniform over 32 positions: 192 rows miss one with odds ~ 1e-2).
    assert len(np.unique(np.argmax(a, axis=-1))) >= 28
    b = (2.0 * rng.integers(0, 2, (2, 3, 32, 16)) - 1.0) / 16
    product = ot.peak_reference(a, b, 1)
    assert set(np.unique(np.abs(product))) == {1 / 256}
    # The product picks row k_hot of B: C[c, w, i, :] = B[c, w, k_hot(w, i), :] / 16.
    hot = np.argmax(a, axis=-1)
    for c in range(2):
        for w in range(3):
            assert np.array_equal(product[c, w], b[c, w, hot[w]] / 16)


def test_product_fp8_peak_operands_are_one_hot_rows():
    """bench_tensor.peak_inputs builds the reference's FP8 operands with torch: its A must satisfy the same
    one-hot invariant as oracle.tensor.one_hot_rows, and its B be +-1/16, so the exact reference is +-1/256."""
    torch = pytest.importorskip("torch")
    from triton_chip_benchmarks_amd import bench_tensor

    config = {"tile_m": 32, "tile_n": 16, "tile_k": 64, "chains": 2, "b_nk": 0}
    a, _b, _c, b_logical = bench_tensor.peak_inputs(3, config, "fp8", "cpu", seed=4)
    a_values, b_values = a.to(torch.float64).numpy(), b_logical.to(torch.float64).numpy()
    assert np.array_equal(np.count_nonzero(a_values, axis=-1), np.ones((3, 32), dtype=np.int64))
    assert set(np.unique(a_values)) == {0.0, 1 / 16}
    assert set(np.unique(b_values)) == {-1 / 16, 1 / 16}
    assert set(np.unique(np.abs(ot.peak_reference(a_values, b_values, 1)))) == {1 / 256}


def test_gemm_tolerance_is_the_reference_published_one():
    """BF16/FP16/FP32 GEMM verdicts use rtol = atol = 2e-3, the value the reference's FP16 GEMM rows were
    checked at (bench_tensor.py:292-293; results/h20_tensor.json), and the product uses the same table."""
    from triton_chip_benchmarks_amd import gemm

    published = GOLDEN["gemm_fp16_h20"]
    assert {(row["rtol"], row["atol"]) for row in published["rows"]} == {(0.002, 0.002)}
    for dtype in ("bf16", "fp16", "fp32"):
        assert ot.GEMM_TOLERANCE[dtype] == 0.002
        assert gemm.TOLERANCE[dtype] == ot.GEMM_TOLERANCE[dtype]
        assert gemm.REFERENCE_TOLERANCE[dtype] == 0.002
    assert gemm.TOLERANCE == ot.GEMM_TOLERANCE
    assert gemm.REFERENCE_SIZES == published["sizes"]
    assert [row["flops"] for row in published["rows"]] == [2 * size**3 for size in published["sizes"]]


# ---- memory oracle ----------------------------------------------------------------------------

def test_bandwidth_traffic_matches_published_rows():
    copy, read = GOLDEN["bandwidth"]["copy"], GOLDEN["bandwidth"]["read"]
    assert memory.copy_traffic_bytes(copy["buffer_bytes"]) == copy["traffic_bytes"]
    assert memory.read_traffic_bytes(read["buffer_bytes"], read["elements"], read["block_size"]) == read["traffic_bytes"]
    assert memory.gbps(copy["traffic_bytes"], copy["median_ms"]) == pytest.approx(copy["gbps"])


def test_block_sums_exact_on_integer_lattice_and_tolerance_rejects_errors():
    rng = np.random.default_rng(11)
    values = rng.integers(-8, 9, 4096 + 17).astype(np.float32)
    sums = memory.block_sums(values, 1024)
    assert sums.shape == (5,) and sums[-1] == values[4096:].sum()
    assert memory.check_read(values, sums.astype(np.float32), 1024) == 0.0
    bad = sums.copy()
    bad[2] += 1.0
    with pytest.raises(AssertionError):
        memory.check_read(values, bad, 1024)
    assert memory.cache_regime(2**30, 256 * 2**20, False) == ("larger_than_l2", True)
    assert memory.cache_regime(512 * 2**20, 256 * 2**20, False) == ("cache_sensitive", False)
    assert memory.cache_regime(2**30, 0, False) == ("unknown_l2", False)
    assert math.isclose(memory.read_tolerance(np.ones(1024), 1024)[0], 1024 * 2 * 2**-23 * 10 + 1e-6)


# ---- widened FP8/FP4 chains ------------------------------------------------------

def _nearest_by_table(y, table, codes):
    """Brute-force round to nearest over a value table; ties go to the code with mantissa bit 0."""
    best = None
    for value, code in zip(table, codes):
        if np.isnan(value):
            continue
        distance = abs(y - value)
        if best is None or distance < best[0] or (distance == best[0] and (code & 1) == 0 and (best[2] & 1)):
            best = (distance, value, code)
    return best[1]


def test_fp8_rounding_matches_torch_on_float32_inputs():
    import torch

    rng = np.random.default_rng(1)
    y = (rng.uniform(-440, 440, 100000) * np.exp(rng.uniform(-14, 0, 100000))).astype(np.float32)
    expected = torch.from_numpy(y).to(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    assert np.array_equal(ov.round_fp8_e4m3fn(y.astype(np.float64)), expected)


def test_fp8_rounding_matches_brute_force_and_ties_go_to_even():
    table, codes = ot.fp8_e4m3fn_decode(np.arange(128)), np.arange(128)
    grid = np.concatenate([np.linspace(0, 2.0**-5, 301), np.linspace(0.9, 2.1, 241), np.linspace(200, 448, 249)])
    for y in grid:
        assert ov.round_fp8_e4m3fn(y) == _nearest_by_table(y, table, codes), y
    # 1 + 1/16 lies halfway between 1 and 1.125: even mantissa (1.0) wins; 1 + 3/16 goes to 1.25.
    assert ov.round_fp8_e4m3fn([1.0625, 1.1875]).tolist() == [1.0, 1.25]


def test_e2m1_rounding_matches_brute_force_and_known_ties():
    codes = np.arange(8)
    table = ot.e2m1_decode(codes)
    for y in np.linspace(0, 6, 97):
        assert ov.round_e2m1(y) == _nearest_by_table(y, table, codes), y
        assert ov.round_e2m1(-y) == -_nearest_by_table(y, table, codes)
    assert ov.round_e2m1([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]).tolist() == [0, 1, 1, 2, 2, 4, 4]


def test_widened_codes_round_trip():
    fp8_values = ot.fp8_e4m3fn_decode(np.arange(256))
    finite = ~np.isnan(fp8_values)
    assert np.array_equal(ot.fp8_e4m3fn_decode(ov.encode_fp8_e4m3fn(fp8_values[finite])), fp8_values[finite])
    assert np.array_equal(ov.encode_e2m1(ot.e2m1_decode(np.arange(16))), np.arange(16))
    with pytest.raises(ValueError):
        ov.encode_e2m1([2.5])


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_widened_involution_is_exact(fmt):
    """a = -1: x -> b - x -> x, exactly, on the lattices the Ascend C suite uses."""
    rng = np.random.default_rng(3)
    if fmt == "fp8":
        x = rng.integers(1, 8, (8, 64)) / 8.0
        b = np.arange(1, 9) / 8.0
        encode = ov.encode_fp8_e4m3fn
    else:
        x = rng.choice([-1.0, -0.5, 0.0, 0.5, 1.0], (8, 64))
        b = np.array([-0.5, 0.0, 0.5, -0.5, 0.0, 0.5, -0.5, 0.0])
        encode = ov.encode_e2m1
    codes, coeff = encode(x), encode(np.concatenate([[-1.0], b]))
    decode = ot.fp8_e4m3fn_decode if fmt == "fp8" else ot.e2m1_decode
    assert np.array_equal(decode(ov.run_widened_chains(fmt, codes, coeff, 7)), b[:, None] - x)
    assert np.array_equal(ov.run_widened_chains(fmt, codes, coeff, 8), codes)


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_widened_contractive_chain_matches_exact_stepwise_rounding(fmt):
    from fractions import Fraction

    rng = np.random.default_rng(4)
    if fmt == "fp8":
        x = rng.integers(-15, 16, (8, 16)) / 16.0
        coefficients = np.concatenate([[0.875], rng.integers(-7, 8, 8) / 32.0])
        table, codes_all = ot.fp8_e4m3fn_decode(np.arange(128)), np.arange(128)
        encode = ov.encode_fp8_e4m3fn
    else:
        x = rng.choice([-1.5, -1.0, -0.5, 0.0, 0.5, 1.0, 1.5], (8, 16))
        coefficients = np.concatenate([[0.5], rng.choice([-1.0, -0.5, 0.5, 1.0], 8)])
        table, codes_all = ot.e2m1_decode(np.arange(8)), np.arange(8)
        encode = ov.encode_e2m1
    got = ov.run_widened_chains(fmt, encode(x), encode(coefficients), 5)
    state = x.copy()
    for _ in range(5):
        for c in range(8):
            for i in range(state.shape[1]):
                exact = Fraction(float(state[c, i])) * Fraction(float(coefficients[0])) + \
                    Fraction(float(coefficients[1 + c]))
                f32 = float(np.float32(float(exact)))  # exact in float64, one rounding to float32
                magnitude = _nearest_by_table(abs(f32), table, codes_all)
                state[c, i] = -magnitude if f32 < 0 else magnitude
    decode = ot.fp8_e4m3fn_decode if fmt == "fp8" else ot.e2m1_decode
    assert np.array_equal(np.abs(decode(got)), np.abs(state))
    assert np.array_equal(np.sign(decode(got)), np.sign(state))


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_widened_chains_keep_ieee_signed_zeros(fmt):
    """IEEE 754 (6.3): -0 + -0 is -0, an exact zero sum of opposite signs is +0
    under round-to-nearest, and a negative value that rounds to zero keeps its
    sign; the narrow codes carry the sign bit (E4M3 0x80, E2M1 0x8)."""
    encode = ov.encode_fp8_e4m3fn if fmt == "fp8" else ov.encode_e2m1
    negative_zero = 0x80 if fmt == "fp8" else 0x8
    x = np.array([[0.0, -0.0, 1.0, -0.0]] * 8)
    # a = -0.5: +0 * a = -0; -0 * a = +0; 1 * a = -0.5.
    for b, expected in ((-0.0, [negative_zero, 0, None, 0]), (0.0, [0, 0, None, 0]), (0.5, [None, None, 0, None])):
        coefficients = encode(np.array([-0.5] + [b] * 8))
        got = ov.run_widened_chains(fmt, encode(x), coefficients, 1)[0]
        for column, code in enumerate(expected):
            if code is not None:
                assert got[column] == code, (fmt, b, column, got)
    if fmt == "fp8":
        # -2^-11 is below half the subnormal quantum 2^-9 / 2: rounds to -0.
        tiny = encode(np.array([[-2.0**-9] * 4] * 8))
        got = ov.run_widened_chains(fmt, tiny, encode(np.array([0.125] + [0.0] * 8)), 1)
        assert (got == negative_zero).all()
    else:
        got = ov.run_widened_chains(fmt, encode(np.array([[-0.5] * 4] * 8)), encode(np.array([0.5] + [0.0] * 8)), 1)
        assert (got == negative_zero).all()  # -0.25 ties to the even -0
