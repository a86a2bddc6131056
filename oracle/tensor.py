"""Oracle for the tensor rows: exact-lattice references, tolerances, formats.

Follows bench_tensor.py (reference):
  E2M1 table and packing       55-69, 603-611
  operand lattices             614-672
  reference, tolerance, check  277-346
  GEMM check (elementwise)     289-299
  op count                     1242
  FP32/FP64 precision probes   675-757
Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's CPU
leg may use it, never the product path. Pins: tests/test_oracle.py and
tests/test_gemm_check.py.
FP8 E4M3FN and E8M0 decoding restate the OCP 8-bit floating point and OCP
Microscaling v1.0 specifications bit by bit (no lookup into torch), so tests
can pin them against torch's float8_e4m3fn conversion independently.
"""

from __future__ import annotations

import numpy as np

E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float64)


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """Value of each 4-bit E2M1 code: sign bit 3, exponent bits 2-1 (bias 1), mantissa bit 0."""
    codes = np.asarray(codes, dtype=np.int64) & 15
    sign = np.where(codes & 8, -1.0, 1.0)
    exponent = (codes >> 1) & 3
    mantissa = codes & 1
    magnitude = np.where(exponent == 0, 0.5 * mantissa, (1.0 + 0.5 * mantissa) * 2.0 ** (exponent - 1))
    return sign * magnitude


def pack_e2m1(codes: np.ndarray) -> np.ndarray:
    """Two codes per byte along the last axis, element 2i in the low nibble (bench_tensor.py:603-611)."""
    codes = np.asarray(codes, dtype=np.uint8)
    return ((codes[..., 1::2] & 15) << 4 | (codes[..., 0::2] & 15)).astype(np.uint8)


def unpack_e2m1(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = packed & 15
    out[..., 1::2] = packed >> 4
    return out


def e8m0_decode(codes: np.ndarray) -> np.ndarray:
    """2**(code-127); code 255 is NaN (OCP MX v1.0 scale format)."""
    codes = np.asarray(codes, dtype=np.int64)
    return np.where(codes == 255, np.nan, np.ldexp(1.0, codes - 127))


def fp8_e4m3fn_decode(bits: np.ndarray) -> np.ndarray:
    """E4M3FN: bias 7, subnormals, no infinities, S.1111.111 is NaN."""
    bits = np.asarray(bits, dtype=np.int64) & 255
    sign = np.where(bits & 128, -1.0, 1.0)
    exponent = (bits >> 3) & 15
    mantissa = bits & 7
    value = np.where(exponent == 0, np.ldexp(mantissa / 8.0, -6),
                     np.ldexp(1.0 + mantissa / 8.0, exponent - 7))
    value = np.where((exponent == 15) & (mantissa == 7), np.nan, value)
    return sign * value


def fp8_e4m3fn_encode_exact(values: np.ndarray) -> np.ndarray:
    """Bit pattern of values that E4M3FN represents exactly (raises otherwise)."""
    table = fp8_e4m3fn_decode(np.arange(256))
    values = np.asarray(values, dtype=np.float64)
    out = np.empty(values.shape, dtype=np.uint8)
    lookup = {}
    for code in range(256):
        if not np.isnan(table[code]) and (table[code] not in lookup or code < 128):
            lookup.setdefault(float(table[code]), code)
    for index, value in np.ndenumerate(values):
        if float(value) not in lookup:
            raise ValueError(f"{value} is not exactly representable in E4M3FN")
        out[index] = lookup[float(value)]
    return out


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns of values exactly representable in bfloat16."""
    as32 = np.asarray(values, dtype=np.float32).view(np.uint32)
    if np.any(as32 & 0xFFFF):
        raise ValueError("values are not exactly representable in bfloat16")
    return (as32 >> 16).astype(np.uint16)


def peak_operation_count(m: int, n: int, k: int, iterations: int, chains: int, blocks: int) -> int:
    """2*M*N*K*ITER*chains*blocks (bench_tensor.py:1242)."""
    return 2 * m * n * k * iterations * chains * blocks


def peak_tolerance(dtype: str, block_k: int, iterations: int) -> float:
    """atol of the resident-peak check, rtol 0 (bench_tensor.py:302-325)."""
    if dtype == "int8":
        return 0.0
    if dtype == "fp4":
        return 4.0 * iterations * block_k * 2.0 ** -24
    unit_roundoff = 2.0 ** -53 if dtype == "fp64" else 2.0 ** -24
    return 4.0 * iterations * block_k / 256.0 * unit_roundoff


def peak_reference(a: np.ndarray, b: np.ndarray, iterations: int) -> np.ndarray:
    """C[c, w] = iterations * A[w] @ B[c, w] in float64 (bench_tensor.py:1220-1232).

    a: [blocks, M, K] values; b: [chains, blocks, K, N] values.
    """
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.stack([np.matmul(a, b[c]) for c in range(b.shape[0])]) * iterations


def check_peak(actual: np.ndarray, reference: np.ndarray, dtype: str, block_k: int, iterations: int) -> float:
    """Max abs error; raises past peak_tolerance (NaN fails)."""
    error = np.abs(np.asarray(actual, dtype=np.float64) - reference)
    tolerance = peak_tolerance(dtype, block_k, iterations)
    if not np.all(error <= tolerance):
        raise AssertionError(f"peak output differs: max_abs_error={np.nanmax(error):.6g} > atol {tolerance:.6g}")
    return float(error.max()) if error.size else 0.0


def ternary_lattice(rng: np.random.Generator, shape, scale: float = 1 / 16) -> np.ndarray:
    """Random {-1, 0, 1} * scale operands (bench_tensor.py:664-666)."""
    return rng.integers(-1, 2, size=shape).astype(np.float64) * scale


def one_hot_rows(rng: np.random.Generator, shape, value: float = 1 / 16) -> np.ndarray:
    """FP8 A operand: one `value` per row at a random K (bench_tensor.py:651-658)."""
    out = np.zeros(shape, dtype=np.float64)
    hot = rng.integers(0, shape[-1], size=shape[:-1])
    np.put_along_axis(out, hot[..., None], value, axis=-1)
    return out


def fp32_precision_probe() -> tuple[np.ndarray, np.ndarray]:
    """A (1+2^-12, 1+2^-9, 2^20) and B = I, 32x32 (bench_tensor.py:678-687)."""
    a = np.full((32, 32), 1.0 + 2.0 ** -12)
    a[0, 1], a[0, 2] = 1.0 + 2.0 ** -9, 2.0 ** 20
    return a, np.eye(32)


def fp64_precision_probe() -> tuple[np.ndarray, np.ndarray]:
    """A with 1+2^-40 and a per-row marker, B = eye(16, 32) (bench_tensor.py:728-735)."""
    a = np.full((32, 16), 1.0 + 2.0 ** -40)
    a[:, 0] = np.arange(1, 33)
    return a, np.eye(16, 32)


def gemm_reference(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """C = A @ B in float64 (bench_tensor.py:277-286); exact on the benchmark's operand lattices."""
    return np.matmul(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64))


# Elementwise GEMM tolerance, rtol = atol (bench_tensor.py:289-299 uses
# torch.testing.assert_close with rtol = atol). BF16, FP16 and FP32 take the
# reference's 2e-3 (bench_tensor.py:292-293; published as rtol = atol = 0.002
# on its FP16 GEMM rows), tighter than the benchmark configuration's 1e-2;
# FP64 takes the configuration's 1e-12, tighter than the reference's 1e-10;
# the FP8, INT8 and MXFP4 operand sets are exact in the accumulator, so 0.
GEMM_TOLERANCE = {"bf16": 2e-3, "fp16": 2e-3, "fp32": 2e-3, "fp64": 1e-12, "fp8": 0.0, "int8": 0.0, "fp4": 0.0}


def gemm_close(actual: np.ndarray, reference: np.ndarray, rtol: float, atol: float) -> np.ndarray:
    """Per-entry verdict |C - R| <= atol + rtol * |R| (NaN and infinities fail)."""
    actual = np.asarray(actual, dtype=np.float64)
    reference = np.asarray(reference, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        return np.isfinite(actual) & (np.abs(actual - reference) <= atol + rtol * np.abs(reference))


def check_gemm(actual: np.ndarray, reference: np.ndarray, dtype: str) -> float:
    """Max abs error; raises when any entry fails gemm_close at GEMM_TOLERANCE[dtype] (0 = bit-exact)."""
    tolerance = GEMM_TOLERANCE[dtype]
    ok = gemm_close(actual, reference, tolerance, tolerance)
    error = np.abs(np.asarray(actual, dtype=np.float64) - reference)
    if not ok.all():
        worst = np.unravel_index(np.argmax(np.where(ok, -1.0, np.nan_to_num(error, nan=np.inf))), ok.shape)
        raise AssertionError(f"GEMM output differs ({dtype}): {int((~ok).sum())} entries outside "
                             f"atol = rtol = {tolerance:g}; worst at {tuple(int(i) for i in worst)}: "
                             f"{actual[worst]!r} vs {reference[worst]!r}")
    return float(error.max()) if error.size else 0.0


def checksum_tolerance(a_values: np.ndarray, b_values: np.ndarray, dtype: str, axis: int) -> np.ndarray:
    """Bound on a row (axis=1) or column (axis=0) checksum of C implied by every entry passing gemm_close.

    With |R_ij| <= (|A| |B|)_ij, summing atol + rtol*|R_ij| over the summed axis
    gives count*atol + rtol * (|A| |B|) summed the same way. a_values is
    [M][K], b_values is [K][N].
    """
    tolerance = GEMM_TOLERANCE[dtype]
    abs_a, abs_b = np.abs(a_values), np.abs(b_values)
    if axis == 0:
        bound = gemm_reference(abs_a.sum(axis=0)[None, :], abs_b)[0]
        count = a_values.shape[0]
    else:
        bound = gemm_reference(abs_a, abs_b.sum(axis=1)[:, None])[:, 0]
        count = b_values.shape[1]
    return count * tolerance + tolerance * bound
