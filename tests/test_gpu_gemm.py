"""GPU parity of the MFMA GEMM kernels (mb_gemm) against oracle.tensor.

Small and ragged shapes are compared element by element with the float64
oracle; operands are exact lattices (or the benchmark's GEMM sets, which are exact in
fp32 accumulation), so the comparison is exact, except FP64 with N(0,1)
operands (normwise 1e-12). The benchmark's full sizes are checked through
size-independent properties: exact row and column checksums
(1^T C = (1^T A) B and C 1 = A (B 1)) plus exactly recomputed sampled rows.
"""

import numpy as np
import pytest

from oracle import tensor as ot

pytestmark = pytest.mark.gpu

FORMATS = ["bf16", "fp16", "fp32", "fp64", "int8", "fp8", "fp4"]


def _configs(dtype):
    from triton_chip_benchmarks_amd import _native

    return _native.gemm_configs(dtype)


def _operand_values(rng, dtype, rows, k):
    if dtype == "fp8":
        return rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0]), (rows, k))
    if dtype == "int8":
        return rng.integers(-8, 9, (rows, k)).astype(np.float64)
    if dtype == "fp64":
        return rng.standard_normal((rows, k))
    return ot.ternary_lattice(rng, (rows, k))


def _device_operand(torch, values, dtype):
    values = np.ascontiguousarray(values)
    if dtype == "bf16":
        return torch.from_numpy(ot.bf16_bits(values).view(np.int16)).view(torch.bfloat16).cuda()
    if dtype == "fp16":
        return torch.from_numpy(values.astype(np.float16)).cuda()
    if dtype == "fp32":
        return torch.from_numpy(values.astype(np.float32)).cuda()
    if dtype == "fp64":
        return torch.from_numpy(values).cuda()
    if dtype == "int8":
        return torch.from_numpy(values.astype(np.int8)).cuda()
    if dtype == "fp8":
        return torch.from_numpy(ot.fp8_e4m3fn_encode_exact(values)).cuda().view(torch.float8_e4m3fn)
    raise ValueError(dtype)


def _run_gemm(dtype, config, m, n, k, rng):
    """Returns (C on the host as float64, A values, B values [n][k])."""
    import torch

    from triton_chip_benchmarks_amd import _native

    scales = (None, None)
    if dtype == "fp4":
        codes_a = rng.integers(0, 16, (m, k), dtype=np.uint8)
        codes_b = rng.integers(0, 16, (n, k), dtype=np.uint8)
        a = torch.from_numpy(ot.pack_e2m1(codes_a)).cuda()
        b = torch.from_numpy(ot.pack_e2m1(codes_b)).cuda()
        scales = (torch.full((m, k // 32), 127, dtype=torch.uint8, device="cuda"),
                  torch.full((n, k // 32), 127, dtype=torch.uint8, device="cuda"))
        a_values, b_values = ot.e2m1_decode(codes_a), ot.e2m1_decode(codes_b)
    else:
        a_values, b_values = _operand_values(rng, dtype, m, k), _operand_values(rng, dtype, n, k)
        a, b = _device_operand(torch, a_values, dtype), _device_operand(torch, b_values, dtype)
    out = torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32
    c = torch.full((m, n), -3, dtype=out, device="cuda")
    _native.gemm(dtype, config, a, b, c, m, n, k, *scales)
    torch.cuda.synchronize()
    return c.cpu().numpy().astype(np.float64), a_values, b_values


def _assert_matches(dtype, got, reference):
    if dtype == "fp64":
        assert ot.gemm_relative_error(got, reference) <= 1e-12
    else:
        assert np.array_equal(got, reference), f"max error {np.abs(got - reference).max()}"


@pytest.mark.parametrize("dtype", FORMATS)
def test_gemm_matches_oracle_every_tile_and_ragged_shapes(gpu, dtype):
    rng = np.random.default_rng(7)
    for config in _configs(dtype):
        shapes = [(config["tile_m"], config["tile_n"], 2 * config["tile_k"]),
                  (2 * config["tile_m"], config["tile_n"], 4 * config["tile_k"])]
        # Ragged: M, N off the tile; K a whole number of 16-byte rows but not of tiles.
        k_ragged = {"fp4": 160, "fp8": 176, "int8": 176}.get(dtype, 88)
        shapes.append((config["tile_m"] + 37, config["tile_n"] - 5, k_ragged))
        for m, n, k in shapes:
            print(f"gemm {dtype} tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']} shape {m}x{n}x{k}",
                  flush=True)
            got, a_values, b_values = _run_gemm(dtype, config, m, n, k, rng)
            _assert_matches(dtype, got, ot.gemm_reference(a_values, b_values.T))


@pytest.mark.parametrize("dtype,size", [("bf16", 8192), ("fp8", 8192), ("int8", 8192), ("fp4", 16384),
                                        ("fp64", 4096)])
def test_gemm_baseline_size_checksums(gpu, dtype, size):
    """Benchmark sizes: exact row/column checksums and sampled rows against the oracle."""
    config = max(_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
    print(f"gemm {dtype} {size}^3 tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']}", flush=True)
    rng = np.random.default_rng(size)
    got, a_values, b_values = _run_gemm(dtype, config, size, size, size, rng)
    column_sums = ot.gemm_reference(a_values.sum(axis=0)[None, :], b_values.T)[0]   # 1^T C = (1^T A) B
    row_sums = ot.gemm_reference(a_values, b_values.sum(axis=0)[:, None])[:, 0]       # C 1 = A (B 1)
    rows = rng.choice(size, 4, replace=False)
    sampled = ot.gemm_reference(a_values[rows], b_values.T)
    if dtype == "fp64":
        scale = np.abs(sampled).max()
        assert np.abs(got[rows] - sampled).max() <= 1e-12 * scale
        assert np.abs(got.sum(axis=0) - column_sums).max() <= 1e-10 * np.abs(column_sums).max()
    else:
        assert np.array_equal(got[rows], sampled)
        assert np.array_equal(got.sum(axis=0), column_sums)
        assert np.array_equal(got.sum(axis=1), row_sums)


def test_mxfp4_gemm_applies_each_rows_group_scale(gpu):
    """E8M0 scales drawn from {126, 127, 128} per (row, 32-element group): a
    wrong row or group index, or a scale applied to the wrong operand, moves
    the result off the exact oracle. Products are multiples of 2^-4 below 145
    and K <= 1024, so every partial sum is exact in fp32 in any order."""
    import torch

    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(11)
    for config in _configs("fp4"):
        shapes = [(config["tile_m"], config["tile_n"], 2 * config["tile_k"]),
                  (2 * config["tile_m"], config["tile_n"], 4 * config["tile_k"]),
                  (config["tile_m"] + 37, config["tile_n"] - 5, 160)]
        for m, n, k in shapes:
            print(f"gemm fp4 scaled tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']} shape {m}x{n}x{k}",
                  flush=True)
            codes_a = rng.integers(0, 16, (m, k), dtype=np.uint8)
            codes_b = rng.integers(0, 16, (n, k), dtype=np.uint8)
            sa = rng.integers(126, 129, (m, k // 32), dtype=np.uint8)
            sb = rng.integers(126, 129, (n, k // 32), dtype=np.uint8)
            c = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
            _native.gemm("fp4", config, torch.from_numpy(ot.pack_e2m1(codes_a)).cuda(),
                         torch.from_numpy(ot.pack_e2m1(codes_b)).cuda(), c, m, n, k,
                         torch.from_numpy(sa).cuda(), torch.from_numpy(sb).cuda())
            torch.cuda.synchronize()
            a_values = ot.e2m1_decode(codes_a) * np.repeat(ot.e8m0_decode(sa), 32, axis=1)
            b_values = ot.e2m1_decode(codes_b) * np.repeat(ot.e8m0_decode(sb), 32, axis=1)
            expected = ot.gemm_reference(a_values, b_values.T)
            got = c.cpu().numpy().astype(np.float64)
            assert np.array_equal(got, expected), f"max error {np.abs(got - expected).max()}"
