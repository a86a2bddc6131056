"""GPU parity of the vector chain kernels (mb_vector_chains) against oracle.vector.

The oracle emulates every update with exactly the kernels' rounding (one
rounding for fp32/fp64/fp16 FMA; bf16 states rounded from the fp32 result),
so outputs are compared bit for bit, on the reference's operands, on
the headline workload's operands and on random operands that exercise rounding.
"""

import zlib

import numpy as np
import pytest

from oracle import tensor as ot
from oracle import vector as ov

pytestmark = pytest.mark.gpu

KIND_DTYPE = {"fp32": "fp32", "fp64": "fp64", "fp16": "fp16", "bf16_dot2": "bf16", "bf16_fma": "bf16",
              "int8": "int8"}


def _device(torch, values, dtype):
    values = np.ascontiguousarray(values)
    if dtype == "fp32":
        return torch.from_numpy(values.astype(np.float32)).cuda()
    if dtype == "fp64":
        return torch.from_numpy(values.astype(np.float64)).cuda()
    if dtype == "fp16":
        return torch.from_numpy(values.astype(np.float16)).cuda()
    if dtype == "bf16":
        return torch.from_numpy(ot.bf16_bits(values).view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(values.astype(np.int32)).cuda()


def _host(tensor, dtype):
    import torch

    if dtype == "bf16":
        return tensor.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16
    return tensor.cpu().numpy()


def _as_bits(values, dtype):
    """Comparable bit patterns (so -0.0 vs 0.0 or NaN payloads would show)."""
    values = np.asarray(values)
    if dtype == "bf16":
        return np.asarray(values, dtype=np.float32).view(np.uint32) >> 16
    if dtype == "fp16":
        return np.asarray(values, dtype=np.float16).view(np.uint16)
    if dtype == "fp32":
        return np.asarray(values, dtype=np.float32).view(np.uint32)
    if dtype == "fp64":
        return np.asarray(values, dtype=np.float64).view(np.uint64)
    return np.asarray(values, dtype=np.int32)


def _run(kind, inputs, coefficients, iterations, unroll, block=256):
    import torch

    from triton_chip_benchmarks_amd import bench_vector

    dtype = KIND_DTYPE[kind]
    x = _device(torch, inputs, dtype)
    c = _device(torch, coefficients, dtype)
    out = torch.empty_like(x)
    out.fill_(-7)
    bench_vector.launch_vector(kind, x, out, c, iterations, unroll, block)
    torch.cuda.synchronize()
    return x, out, c


def _check_against_oracle(kind, inputs, coefficients, iterations, unroll, block=256):
    dtype = KIND_DTYPE[kind]
    _x, out, _c = _run(kind, inputs, coefficients, iterations, unroll, block)
    expected = ov.run_chains(dtype, inputs, coefficients, iterations, widened=dtype == "bf16")
    got = _host(out, dtype)
    if dtype == "bf16":
        assert np.array_equal(got >> 16, _as_bits(expected, "bf16")), kind
    else:
        assert np.array_equal(_as_bits(got, dtype), _as_bits(expected, dtype)), kind
    return out


@pytest.mark.parametrize("kind", list(KIND_DTYPE))
@pytest.mark.parametrize("inputs_kind", ["reference", "baseline"])
def test_vector_chains_bit_exact_against_oracle(gpu, kind, inputs_kind):
    dtype = KIND_DTYPE[kind]
    rng = np.random.default_rng(zlib.crc32(f"{kind}/{inputs_kind}".encode()))
    maker = ov.reference_inputs if inputs_kind == "reference" else ov.baseline_inputs
    inputs, coefficients = maker(dtype, 512, rng)
    for iterations, unroll in ((4096, 16), (4096, 1), (33, 1)):
        print(f"vector {kind} {inputs_kind} iterations={iterations} unroll={unroll}", flush=True)
        _check_against_oracle(kind, inputs, coefficients, iterations, unroll)


@pytest.mark.parametrize("kind", ["fp16", "bf16_dot2", "bf16_fma", "fp32"])
def test_vector_rounding_on_random_operands(gpu, kind):
    """Non-lattice operands: every update rounds, and must round like the oracle."""
    dtype = KIND_DTYPE[kind]
    rng = np.random.default_rng(42)
    inputs = rng.uniform(-2.0, 2.0, (8, 1024))
    coefficients = np.concatenate([[0.7071], rng.uniform(-0.05, 0.05, 8)])
    if dtype in ("fp16", "bf16"):
        inputs, coefficients = ov.round_narrow(inputs, dtype), ov.round_narrow(coefficients, dtype)
    else:
        inputs = inputs.astype(np.float32).astype(np.float64)
        coefficients = coefficients.astype(np.float32).astype(np.float64)
    print(f"vector rounding {kind}", flush=True)
    _check_against_oracle(kind, inputs, coefficients, 257, 1, block=512)


def test_product_validators_accept_kernel_output_and_agree_with_oracle(gpu):
    """bench_vector's own checks pass on real output; the oracle's closed form agrees."""
    import torch

    from triton_chip_benchmarks_amd import bench_vector

    for dtype in ("fp32", "fp64", "fp16", "bf16", "int8"):
        kind = "bf16_dot2" if dtype == "bf16" else dtype
        inputs, coefficients = bench_vector.make_inputs(dtype, 2048, "cuda")
        output = torch.empty_like(inputs)
        bench_vector.launch_vector(kind, inputs, output, coefficients, 4096, 8, 1024)
        torch.cuda.synchronize()
        if dtype == "int8":
            bench_vector.check_int8_output(inputs, output, coefficients, 4096)
            ov.int8_transition_check(inputs.cpu().numpy(), output.cpu().numpy(), coefficients.cpu().numpy(), 4096)
        else:
            result = bench_vector.check_output(inputs, output, coefficients, 4096)
            oracle = ov.closed_form_check(inputs.double().cpu().numpy(), output.double().cpu().numpy(),
                                          coefficients.double().cpu().numpy(), 4096, dtype)
            assert result["max_abs_tolerance"] == pytest.approx(oracle["max_abs_tolerance"])
            assert result["max_abs_error"] == pytest.approx(oracle["max_abs_error"])
        if dtype in ("fp16", "bf16"):
            bench_vector.check_narrow_steps(inputs, output, coefficients, 4096, dtype, lanes=512)



# ---- widened (converted) FP8 / FP4 chains -------------------------------------

def _run_widened(kind, codes, coefficient_codes, iterations, unroll, block=256):
    import torch

    from triton_chip_benchmarks_amd import bench_vector

    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    assert codes.shape[0] == 8 and codes.shape[1] % block == 0 and len(coefficient_codes) == 9
    x = torch.from_numpy(codes).cuda()
    c = torch.from_numpy(np.ascontiguousarray(coefficient_codes, dtype=np.uint8)).cuda()
    out = torch.full_like(x, 0x7F)
    bench_vector.launch_vector(kind, x, out, c, iterations, unroll, block)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
@pytest.mark.parametrize("iterations,unroll", [(7, 1), (8, 4), (32, 16)])
def test_widened_involution_matches_oracle(gpu, fmt, iterations, unroll):
    from triton_chip_benchmarks_amd import bench_vector

    codes, coefficients = bench_vector.widened_inputs(fmt, 1024, "cpu", seed=iterations)
    codes, coefficients = codes.numpy(), coefficients.numpy()
    got = _run_widened(f"{fmt}_widened", codes, coefficients, iterations, unroll)
    expected = ov.run_widened_chains(fmt, codes, coefficients, iterations)
    assert np.array_equal(got, expected)
    assert np.array_equal(got, codes if iterations % 2 == 0 else expected)


def _finite_fp8_codes(rng, shape, max_magnitude):
    values = ot.fp8_e4m3fn_decode(np.arange(256))
    allowed = np.flatnonzero(~np.isnan(values) & (np.abs(values) <= max_magnitude))
    return rng.choice(allowed, shape).astype(np.uint8)


@pytest.mark.parametrize("iterations,unroll", [(1, 1), (3, 1), (24, 8)])
@pytest.mark.parametrize("a", [0.875, -0.5, 0.9375, -0.0625])
def test_widened_fp8_rounds_every_step_like_the_oracle(gpu, a, iterations, unroll):
    """Contractive chains over every finite E4M3 code (subnormals, signed zeros,
    up to 448): |x a + b| stays within 448, so each of the 24 steps rounds twice
    (FP32, then E4M3) and the codes must agree bit for bit; short chains keep
    the start codes' variety, long ones reach the fixed points."""
    rng = np.random.default_rng(int(abs(a) * 1e4))
    codes = _finite_fp8_codes(rng, (8, 2048), 448.0)
    coefficients = np.concatenate([ov.encode_fp8_e4m3fn(np.array([a])), _finite_fp8_codes(rng, 8, 8.0)])
    got = _run_widened("fp8_widened", codes, coefficients, iterations, unroll)
    assert np.array_equal(got, ov.run_widened_chains("fp8", codes, coefficients, iterations))


@pytest.mark.parametrize("iterations,unroll", [(1, 1), (16, 4)])
@pytest.mark.parametrize("a", [0.5, -0.5, -1.0])
def test_widened_fp4_rounds_every_step_like_the_oracle(gpu, a, iterations, unroll):
    """Every E2M1 code as a start value; |b| <= 3 keeps |x a + b| <= 6 (for
    a = -1, |x| <= 3 as well), so no step leaves the format's range."""
    rng = np.random.default_rng(int(abs(a) * 10))
    limit = 3.0 if a == -1.0 else 6.0
    values = ot.e2m1_decode(np.arange(16))
    codes = rng.choice(np.flatnonzero(np.abs(values) <= limit), (8, 1024)).astype(np.uint8)
    b_codes = rng.choice(np.flatnonzero(np.abs(values) <= 3.0), 8).astype(np.uint8)
    coefficients = np.concatenate([ov.encode_e2m1(np.array([a])), b_codes])
    got = _run_widened("fp4_widened", codes, coefficients, iterations, unroll)
    assert np.array_equal(got, ov.run_widened_chains("fp4", codes, coefficients, iterations))


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
def test_widened_flag_keeps_the_row_status_and_reports_details(gpu, tmp_path, fmt):
    import json

    from triton_chip_benchmarks_amd import bench_vector

    output = tmp_path / f"vector_{fmt}.json"
    bench_vector.main(["--dtype", fmt, "--widened", "--quick", "--output", str(output)])
    document = json.loads(output.read_text())
    assert document["status"] == ("not_implemented" if fmt == "fp8" else "unsupported")
    widened = document["details"]["widened"]
    assert widened["peak_tflops"] > 0 and widened["arithmetic_kind"].startswith("converted_fp32_fma")
    row = document["details"]["widened_rows"][0]
    assert row["native_arithmetic_verified"] is False and row["max_abs_error"] == 0.0
