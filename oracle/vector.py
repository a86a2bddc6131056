"""Oracle for the vector rows: exact chain emulation and the reference's validators.

Follows bench_vector.py (reference):
  recurrences              87-179 (FMA, widened FMA, DP4A feedback form)
  closed-form check        322-372 (check_output)
  INT8 exact check         375-421 (_signed_bytes, _dot4_reference, check_int8_output)
  operation count          1271-1280 (throughput_fields)
  inputs                   1191-1216 (_make_inputs)
The step-by-step emulation is C (oracle/c/vector_ref.c); the closed forms are
numpy restatements, so each side can check the other.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np

from . import cbuild

CHAINS = 8
DEFAULT_ITERATIONS = 4096

_lib = None


def _library():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(str(cbuild.library_path()))
        double_p = ctypes.POINTER(ctypes.c_double)
        _lib.oracle_chain_f32.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_long, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_long]
        _lib.oracle_chain_f64.argtypes = [double_p, ctypes.c_long, ctypes.c_double, ctypes.c_double, ctypes.c_long]
        _lib.oracle_chain_narrow.argtypes = [double_p, ctypes.c_long, ctypes.c_double, ctypes.c_double,
                                             ctypes.c_long, ctypes.c_int, ctypes.c_int]
        _lib.oracle_round_narrow.argtypes = [double_p, ctypes.c_long, ctypes.c_int]
        _lib.oracle_chain_dot4.argtypes = [ctypes.POINTER(ctypes.c_int32), ctypes.c_long, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_long]
    return _lib


def round_narrow(values, dtype: str) -> np.ndarray:
    """Correctly rounded fp16/bf16 values (as float64) of float64 inputs."""
    out = np.ascontiguousarray(values, dtype=np.float64).copy()
    _library().oracle_round_narrow(out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), out.size,
                                   1 if dtype == "bf16" else 0)
    return out


def run_chains(dtype: str, inputs: np.ndarray, coefficients: np.ndarray, iterations: int,
               widened: bool = True) -> np.ndarray:
    """Emulate all chains: inputs [8, n] and coefficients [9] (a, b_0..b_7).

    fp32/fp64 use a fused multiply-add; fp16/bf16 states round once per
    update, either straight from the exact value (widened=False) or through
    fp32 first (widened=True, the gfx950 kernels' arithmetic); int8 is the
    DP4A feedback recurrence on int32 states with packed int8 weights.
    """
    lib = _library()
    inputs = np.asarray(inputs)
    out = []
    for chain in range(inputs.shape[0]):
        if dtype == "fp32":
            x = np.ascontiguousarray(inputs[chain], dtype=np.float32).copy()
            lib.oracle_chain_f32(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size,
                                 float(np.float32(coefficients[0])), float(np.float32(coefficients[1 + chain])),
                                 iterations)
        elif dtype == "fp64":
            x = np.ascontiguousarray(inputs[chain], dtype=np.float64).copy()
            lib.oracle_chain_f64(x.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), x.size,
                                 float(coefficients[0]), float(coefficients[1 + chain]), iterations)
        elif dtype in ("fp16", "bf16"):
            x = np.ascontiguousarray(inputs[chain], dtype=np.float64).copy()
            lib.oracle_chain_narrow(x.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), x.size,
                                    float(coefficients[0]), float(coefficients[1 + chain]), iterations,
                                    1 if dtype == "bf16" else 0, 1 if widened else 0)
        elif dtype == "int8":
            x = np.ascontiguousarray(inputs[chain], dtype=np.int32).copy()
            lib.oracle_chain_dot4(x.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), x.size,
                                  int(np.int32(coefficients[0])), int(np.int32(coefficients[1 + chain])), iterations)
        else:
            raise ValueError(dtype)
        out.append(x)
    return np.stack(out)


def operation_count(dtype: str, elements: int, iterations: int) -> int:
    """(8 for DP4A, else 2) * 8 chains * elements * iterations (bench_vector.py:1271-1273)."""
    return (8 if dtype == "int8" else 2) * CHAINS * elements * iterations


def closed_form_check(inputs, output, coefficients, iterations, dtype: str, explicit_fma: bool = True) -> dict:
    """Restatement of check_output (bench_vector.py:322-372) in numpy float64.

    a == -1 is the exact two-cycle (zero tolerance); otherwise the contractive
    affine recurrence x_n = a^n x_0 + b (1 - a^n) / (1 - a) with the bound
    r * u * max(|x0|, |b/(1-a)|) * sum a^i + 16u, r = 2 (FMA) or 4.
    """
    coefficients = np.asarray(coefficients, dtype=np.float64)
    a = float(coefficients[0])
    b = coefficients[1:, None]
    initial = np.asarray(inputs, dtype=np.float64)
    actual = np.asarray(output, dtype=np.float64)
    if a == -1.0:
        reference = b - initial if iterations % 2 else initial
        tolerance = np.zeros_like(reference)
    else:
        decay = math.exp(iterations * math.log(a))
        geometric = -math.expm1(iterations * math.log(a)) / (1.0 - a)
        reference = decay * initial + b * geometric
        magnitude = np.maximum(np.abs(initial), np.abs(b / (1.0 - a)))
        unit = 2.0 ** (-53 if dtype == "fp64" else -24)
        tolerance = (2.0 if explicit_fma else 4.0) * unit * magnitude * geometric + 16 * unit
    error = np.abs(actual - reference)
    if not np.all(error <= tolerance):
        raise AssertionError(f"vector output outside the closed-form bound: max error {np.nanmax(error):.6g}")
    return {"max_abs_error": float(error.max()), "max_abs_tolerance": float(tolerance.max())}


def signed_bytes(word: int) -> list[int]:
    """Four signed bytes of an int32, low byte first (bench_vector.py:375-378)."""
    return [((int(word) >> shift) & 255) - (256 if ((int(word) >> shift) & 255) >= 128 else 0)
            for shift in (0, 8, 16, 24)]


def pack_bytes(values) -> int:
    """Pack four signed bytes into an int32 (bench_vector.py:1198-1201)."""
    packed = sum((int(v) & 255) << shift for v, shift in zip(values, (0, 8, 16, 24)))
    return packed - 2**32 if packed >= 2**31 else packed


def dot4_reference(words: np.ndarray, weights) -> np.ndarray:
    words = np.asarray(words, dtype=np.int64)
    result = np.zeros_like(words)
    for shift, weight in zip((0, 8, 16, 24), weights):
        lane = (words >> shift) & 255
        result += np.where(lane >= 128, lane - 256, lane) * weight
    return result


def int8_transition_check(inputs, output, coefficients, iterations) -> None:
    """Restatement of check_int8_output (bench_vector.py:390-421).

    After one update the state lies in [-bound, bound]; the iterated map on
    that range is composed by binary lifting instead of looping per lane.
    Valid while every post-update state stays in int32 without wrapping.
    """
    coefficients = np.asarray(coefficients, dtype=np.int64)
    weights = signed_bytes(coefficients[0])
    bias = coefficients[1:, None]
    bound = 128 * sum(abs(w) for w in weights) + int(np.abs(bias).max())
    states = np.broadcast_to(np.arange(-bound, bound + 1), (CHAINS, 2 * bound + 1))
    power = dot4_reference(states, weights) + bias + bound
    composed = np.broadcast_to(np.arange(2 * bound + 1), (CHAINS, 2 * bound + 1)).copy()
    remaining = iterations - 1
    while remaining:
        if remaining & 1:
            composed = np.take_along_axis(power, composed, axis=1)
        remaining >>= 1
        if remaining:
            power = np.take_along_axis(power, power, axis=1)
    first = dot4_reference(np.asarray(inputs, dtype=np.int64), weights) + bias
    reference = np.take_along_axis(composed, first + bound, axis=1) - bound
    if not np.array_equal(np.asarray(output, dtype=np.int64), reference):
        raise AssertionError("INT8 dot4 output differs from the exact transition-table reference")


def reference_inputs(dtype: str, elements: int, rng: np.random.Generator):
    """The reference's default operands (bench_vector.py:1191-1216), numpy-drawn.

    Returns (inputs [8, elements], coefficients [9]) as exact values in the
    storage format (float64 for the floats, int32 words for int8).
    """
    if dtype == "int8":
        inputs = rng.integers(-(2**31), 2**31, size=(CHAINS, elements), dtype=np.int64).astype(np.int32)
        coefficients = np.array([pack_bytes((3, -2, 1, -1))] + list(range(1, CHAINS + 1)), dtype=np.int32)
    elif dtype in ("fp16", "bf16"):
        inputs = rng.integers(1, 8, size=(CHAINS, elements)) / 8.0
        coefficients = np.array([-1.0] + [(i + 1) / 8 for i in range(CHAINS)])
    else:
        inputs = rng.uniform(0.125, 1.0, size=(CHAINS, elements))
        if dtype == "fp32":
            inputs = inputs.astype(np.float32).astype(np.float64)
        coefficients = np.array([1.0 - 2.0**-14] + [(c + 1) * 2.0**-16 for c in range(CHAINS)])
    return inputs, coefficients


def baseline_inputs(dtype: str, elements: int, rng: np.random.Generator):
    """The headline vector workload: a0 ~ U[0.5, 1), b = 0.999, c = 1e-3.

    INT8: a0 in [-4, 4], weights 1 in every byte, bias 1 (wrapping int32). The
    float values are rounded to the storage format as the device sees them.
    """
    if dtype == "int8":
        inputs = rng.integers(-4, 5, size=(CHAINS, elements)).astype(np.int32)
        coefficients = np.array([pack_bytes((1, 1, 1, 1))] + [1] * CHAINS, dtype=np.int32)
        return inputs, coefficients
    inputs = rng.uniform(0.5, 1.0, size=(CHAINS, elements))
    coefficients = np.array([0.999] + [1e-3] * CHAINS)
    if dtype == "fp32":
        return inputs.astype(np.float32).astype(np.float64), coefficients.astype(np.float32).astype(np.float64)
    if dtype in ("fp16", "bf16"):
        return round_narrow(inputs, dtype), round_narrow(coefficients, dtype)
    return inputs, coefficients


# ---- widened (converted) FP8 / FP4 chains -------------------------------------
# The reference's Ascend C suite measures these rows as "converted" chains
# (ascendc/src/bench_vector.asc:335-572): the state stays in the narrow format
# and each update is x <- narrow(fma(f32(x), a, b_c)), one FP32 rounding then
# one rounding to the narrow format, both to nearest even. The Ascend C check
# uses the exact involution a = -1 (bench_vector.asc:1007-1012); the emulation
# below also covers contractive coefficients, where every step rounds.

FP8_E4M3_MAX = 448.0
E2M1_MAX = 6.0
_E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def round_fp8_e4m3fn(values) -> np.ndarray:
    """Nearest E4M3FN value (ties to even): 3 fraction bits, exponents -6..8,
    subnormal quantum 2^-9. Inputs must lie within +-448 (no saturation rule
    is assumed beyond it)."""
    y = np.asarray(values, dtype=np.float64)
    if np.any(np.abs(y) > FP8_E4M3_MAX) or np.any(np.isnan(y)):
        raise ValueError("E4M3FN rounding is only defined here for finite |x| <= 448")
    magnitude = np.abs(y)
    with np.errstate(divide="ignore"):
        exponent = np.floor(np.log2(np.where(magnitude > 0, magnitude, 1.0)))
    quantum = np.ldexp(1.0, (np.maximum(exponent, -6) - 3).astype(np.int64))
    return np.copysign(np.rint(magnitude / quantum) * quantum, y)  # -0 and underflow keep the sign


def encode_fp8_e4m3fn(values) -> np.ndarray:
    """Codes of E4M3FN-representable values (vectorised; -0 keeps its sign bit)."""
    y = np.asarray(values, dtype=np.float64)
    sign = np.signbit(y).astype(np.int64) << 7
    magnitude = np.abs(y)
    with np.errstate(divide="ignore"):
        exponent = np.floor(np.log2(np.where(magnitude > 0, magnitude, 1.0))).astype(np.int64)
    normal = (magnitude >= 2.0**-6)
    mantissa_normal = np.rint((magnitude / np.ldexp(1.0, exponent) - 1.0) * 8).astype(np.int64)
    code_normal = ((exponent + 7) << 3) | mantissa_normal
    code_sub = np.rint(magnitude / 2.0**-9).astype(np.int64)
    codes = np.where(normal, code_normal, code_sub) | sign
    if not np.array_equal(decode_fp8(codes), y):
        raise ValueError("value not representable in E4M3FN")
    return codes.astype(np.uint8)


def decode_fp8(codes) -> np.ndarray:
    from .tensor import fp8_e4m3fn_decode

    return fp8_e4m3fn_decode(codes)


def round_e2m1(values) -> np.ndarray:
    """Nearest E2M1 value (ties to even): quantum 0.5 below 2, 1 in [2, 4), 2 in [4, 6]."""
    y = np.asarray(values, dtype=np.float64)
    if np.any(np.abs(y) > E2M1_MAX) or np.any(np.isnan(y)):
        raise ValueError("E2M1 rounding is only defined here for finite |x| <= 6")
    magnitude = np.abs(y)
    quantum = np.where(magnitude < 2, 0.5, np.where(magnitude < 4, 1.0, 2.0))
    return np.copysign(np.rint(magnitude / quantum) * quantum, y)


def encode_e2m1(values) -> np.ndarray:
    """Codes of E2M1-representable values (sign bit 3; -0 keeps its sign bit)."""
    y = np.asarray(values, dtype=np.float64)
    index = np.searchsorted(_E2M1_MAGNITUDES, np.abs(y))
    if np.any(index >= 8) or not np.array_equal(_E2M1_MAGNITUDES[np.minimum(index, 7)], np.abs(y)):
        raise ValueError("value not representable in E2M1")
    return (index | (np.signbit(y).astype(np.int64) << 3)).astype(np.uint8)


def run_widened_chains(fmt: str, codes, coefficient_codes, iterations: int) -> np.ndarray:
    """Codes after `iterations` updates x <- narrow(f32(x * a + b_c)) of every chain.

    codes [8, n] (one code per element), coefficient_codes [9] (a, b_0..b_7).
    x * a + b_c is exact in float64 for these narrow operands, so casting it to
    float32 is the single rounding of v_fma_f32; the narrow rounding follows.
    """
    from .tensor import e2m1_decode

    decode = decode_fp8 if fmt == "fp8" else e2m1_decode
    narrow = round_fp8_e4m3fn if fmt == "fp8" else round_e2m1
    encode = encode_fp8_e4m3fn if fmt == "fp8" else encode_e2m1
    x = decode(np.asarray(codes))
    coefficients = decode(np.asarray(coefficient_codes))
    a, b = coefficients[0], coefficients[1:, None]
    for _ in range(iterations):
        x = narrow(np.asarray(x * a + b, dtype=np.float32).astype(np.float64))
    return encode(x)
