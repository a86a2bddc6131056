"""GPU parity of the MFMA GEMM kernels (mb_gemm) against oracle.tensor.

Small and ragged shapes are compared element by element with the float64
oracle; operands are exact lattices (or the benchmark's GEMM sets, which are exact in
fp32 accumulation), so the comparison is exact. N(0,1) operands (every float
format, and FP64 throughout) are checked entry by entry with the reference's
rule |C - R| <= atol + rtol*|R|, rtol = atol = oracle.tensor.GEMM_TOLERANCE
(1e-2 BF16/FP16, 2e-3 FP32, 1e-12 FP64). The benchmark's full sizes are
checked through size-independent properties: row and column checksums
(1^T C = (1^T A) B and C 1 = A (B 1)), exact on the lattices and within the
bound every passing entry implies otherwise, plus sampled rows recomputed by
the oracle, plus the product's own full-output check against a float64
device product.
"""

import numpy as np
import pytest

from oracle import tensor as ot

pytestmark = pytest.mark.gpu

FORMATS = ["bf16", "fp16", "fp32", "fp64", "int8", "fp8", "fp4"]


def _configs(dtype):
    from triton_chip_benchmarks_amd import _native

    return _native.gemm_configs(dtype)


def _operand_values(rng, dtype, rows, k, normal=False):
    if normal:  # N(0,1) rounded to the storage format (exact for fp64)
        values = rng.standard_normal((rows, k))
        if dtype == "bf16":
            import torch

            return torch.from_numpy(values).to(torch.bfloat16).double().numpy()
        return values.astype({"fp16": np.float16, "fp32": np.float32, "fp64": np.float64}[dtype]).astype(np.float64)
    if dtype == "fp8":
        return rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0]), (rows, k))
    if dtype == "int8":
        return rng.integers(-8, 9, (rows, k)).astype(np.float64)
    if dtype == "fp64":
        return rng.standard_normal((rows, k))
    return ot.ternary_lattice(rng, (rows, k))


def _scale_blocks(scales):
    """[rows][K/32] E8M0 codes -> mb_gemm's K-step blocks [ceil(K/256)][rows][8] (padding 127)."""
    rows, groups = scales.shape
    out = np.full((-(-groups // 8), rows, 8), 127, dtype=np.uint8)
    for block in range(out.shape[0]):
        part = scales[:, 8 * block:8 * block + 8]
        out[block, :, :part.shape[1]] = part
    return out


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


def _run_gemm(dtype, config, m, n, k, rng, normal=False, keep_device=False):
    """Returns (C on the host as float64, A values, B values [n][k]) [+ device C, A, B]."""
    import torch

    from triton_chip_benchmarks_amd import _native

    scales = (None, None)
    if dtype == "fp4":
        codes_a = rng.integers(0, 16, (m, k), dtype=np.uint8)
        codes_b = rng.integers(0, 16, (n, k), dtype=np.uint8)
        a = torch.from_numpy(ot.pack_e2m1(codes_a)).cuda()
        b = torch.from_numpy(ot.pack_e2m1(codes_b)).cuda()
        scales = (torch.full((-(-k // 256), m, 8), 127, dtype=torch.uint8, device="cuda"),
                  torch.full((-(-k // 256), n, 8), 127, dtype=torch.uint8, device="cuda"))
        a_values, b_values = ot.e2m1_decode(codes_a), ot.e2m1_decode(codes_b)
    else:
        a_values = _operand_values(rng, dtype, m, k, normal or dtype == "fp64")
        b_values = _operand_values(rng, dtype, n, k, normal or dtype == "fp64")
        a, b = _device_operand(torch, a_values, dtype), _device_operand(torch, b_values, dtype)
    out = torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32
    c = torch.full((m, n), -3, dtype=out, device="cuda")
    _native.gemm(dtype, config, a, b, c, m, n, k, *scales)
    torch.cuda.synchronize()
    host = c.cpu().numpy().astype(np.float64)
    if keep_device:
        return host, a_values, b_values, (c, a, b)
    return host, a_values, b_values


def _assert_matches(dtype, got, reference, normal=False):
    if normal or dtype == "fp64":
        ot.check_gemm(got, reference, dtype)
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


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "int8", "fp8", "fp32", "fp64"])
def test_fast_path_over_step_counts(gpu, dtype):
    """The fast path (256x256 with A and B by LDS-DMA into rings of three and
    two slots; 256x128 for FP64, B through registers) at K step counts 4, 6,
    10, 12 and 14, which wrap the three-slot ring at every phase, on lattice
    operands (exact; FP64 on N(0,1) within its tolerance), with M != N so a
    transposed tile order would show."""
    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(23)
    config = max(_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
    elements_per_step = 128 * 8 // {"bf16": 16, "fp16": 16, "int8": 8, "fp8": 8, "fp32": 32, "fp64": 64}[dtype]
    for steps in (4, 6, 10, 12, 14):
        m, n, k = 512, 768, steps * elements_per_step
        launched = _native.gemm_launched_kernel(dtype, config, m, n, k)
        assert not launched.endswith("_checked"), launched
        print(f"gemm {dtype} fast path {m}x{n}x{k} ({steps} K steps) via {launched}", flush=True)
        got, a_values, b_values = _run_gemm(dtype, config, m, n, k, rng)
        _assert_matches(dtype, got, ot.gemm_reference(a_values, b_values.T))


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "int8", "fp8", "fp32", "fp64"])
def test_band_height_orders_tiles_only(gpu, dtype):
    """group_m orders the tiles and nothing else: every band height, including
    ones taller than the tile rows and values near 2^32 (clamped by mb_gemm),
    gives the same C on the fast path and on the checked path (ragged shape)."""
    import torch

    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(31)
    config = max(_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
    for m, n, k in ((768, 512, 1024), (320, 448, 2 * config["tile_k"])):
        launched = _native.gemm_launched_kernel(dtype, config, m, n, k)
        print(f"gemm {dtype} band heights {m}x{n}x{k} via {launched}", flush=True)
        got, a_values, b_values, (c, a, b) = _run_gemm(dtype, config, m, n, k, rng, keep_device=True)
        _assert_matches(dtype, got, ot.gemm_reference(a_values, b_values.T))
        for group in (1, 2, 3, 7, 64, 2**31 + 5, 2**32 - 1):
            c.fill_(-3)
            _native.gemm(dtype, config, a, b, c, m, n, k, group_m=group)
            torch.cuda.synchronize()
            assert np.array_equal(c.cpu().numpy().astype(np.float64), got), group


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
def test_gemm_normal_operands_every_tile_elementwise(gpu, dtype):
    """N(0,1) operands: every entry within rtol = atol = GEMM_TOLERANCE[dtype] of the float64 oracle."""
    rng = np.random.default_rng(17)
    for config in _configs(dtype):
        for m, n, k in [(config["tile_m"], config["tile_n"], 8 * config["tile_k"]),
                        (config["tile_m"] + 37, config["tile_n"] - 5, 1000)]:
            print(f"gemm {dtype} N(0,1) tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']} "
                  f"shape {m}x{n}x{k}", flush=True)
            got, a_values, b_values = _run_gemm(dtype, config, m, n, k, rng, normal=True)
            _assert_matches(dtype, got, ot.gemm_reference(a_values, b_values.T), normal=True)


@pytest.mark.parametrize("dtype,size,normal", [("bf16", 8192, False), ("fp16", 8192, False), ("fp8", 8192, False),
                                               ("int8", 8192, False), ("fp4", 16384, False), ("fp64", 4096, True),
                                               ("bf16", 8192, True), ("fp16", 8192, True)])
def test_gemm_baseline_size_checksums(gpu, dtype, size, normal):
    """Benchmark sizes: row/column checksums, sampled rows against the oracle, and every entry
    against the product's float64 device check. Lattice operands (normal=False) must match
    exactly; N(0,1) operands within the elementwise tolerance."""
    from triton_chip_benchmarks_amd import gemm

    config = max(_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
    print(f"gemm {dtype} {size}^3 {'N(0,1)' if normal else 'lattice'} "
          f"tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']}", flush=True)
    rng = np.random.default_rng(size + normal)
    got, a_values, b_values, (c, _a, _b) = _run_gemm(dtype, config, size, size, size, rng, normal=normal,
                                                     keep_device=True)
    b_kn = b_values.T
    column_sums = ot.gemm_reference(a_values.sum(axis=0)[None, :], b_kn)[0]   # 1^T C = (1^T A) B
    row_sums = ot.gemm_reference(a_values, b_values.sum(axis=0)[:, None])[:, 0]  # C 1 = A (B 1)
    rows = rng.choice(size, 8, replace=False)
    sampled = ot.gemm_reference(a_values[rows], b_kn)
    if normal:
        ot.check_gemm(got[rows], sampled, dtype)
        assert np.all(np.abs(got.sum(axis=0) - column_sums) <= ot.checksum_tolerance(a_values, b_kn, dtype, 0))
        assert np.all(np.abs(got.sum(axis=1) - row_sums) <= ot.checksum_tolerance(a_values, b_kn, dtype, 1))
        import torch

        device_a = torch.from_numpy(a_values).cuda()
        device_b = torch.from_numpy(b_values).cuda()
        result = gemm.validate(c, gemm.reference(device_a, device_b), dtype)
        assert result["max_error_over_allowed"] <= 1.0
        print(f"  max abs error {result['max_abs_error']:.3g}, worst error / allowed "
              f"{result['max_error_over_allowed']:.3g}", flush=True)
    else:
        assert np.array_equal(got[rows], sampled)
        assert np.array_equal(got.sum(axis=0), column_sums)
        assert np.array_equal(got.sum(axis=1), row_sums)


def test_mxfp4_gemm_applies_each_rows_group_scale(gpu):
    """E8M0 scales drawn from {126, 127, 128} per (row, 32-element group): a
    wrong row or group index, or a scale applied to the wrong operand, moves
    the result off the exact oracle. Products are multiples of 2^-4 below 145
    and K <= 4096, so every partial sum is exact in fp32 in any order. The
    scales are passed in mb_gemm's K-step block layout; shapes cover the fast
    path (>= 4 even K steps) and the checked one (2 steps, ragged M/N/K)."""
    import torch

    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(11)
    for config in _configs("fp4"):
        shapes = [(config["tile_m"], config["tile_n"], 2 * config["tile_k"]),
                  (2 * config["tile_m"], config["tile_n"], 4 * config["tile_k"]),
                  (config["tile_m"], 2 * config["tile_n"], 2048),
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
                         torch.from_numpy(_scale_blocks(sa)).cuda(), torch.from_numpy(_scale_blocks(sb)).cuda())
            torch.cuda.synchronize()
            a_values = ot.e2m1_decode(codes_a) * np.repeat(ot.e8m0_decode(sa), 32, axis=1)
            b_values = ot.e2m1_decode(codes_b) * np.repeat(ot.e8m0_decode(sb), 32, axis=1)
            expected = ot.gemm_reference(a_values, b_values.T)
            got = c.cpu().numpy().astype(np.float64)
            assert np.array_equal(got, expected), f"max error {np.abs(got - expected).max()}"


def test_mxfp4_gemm_reads_the_block_scale_layout_not_row_major(gpu):
    """The scale layout is ABI (version 2): the K-step blocks [K/256][rows][8]. Row-major [rows][K/32]
    scales have the same byte count whenever K is a multiple of 256, so the size check cannot catch a
    caller still using them; this pins what such a call computes. Passing the row-major bytes gives the
    oracle product of those bytes read as blocks (so the kernel reads exactly the documented layout), and
    differs from the correctly scaled product (so the mix-up is visible, not hidden by unit scales)."""
    import torch

    from triton_chip_benchmarks_amd import _native

    assert _native.load().mb_abi_version() == 2
    rng = np.random.default_rng(29)
    config = max(_configs("fp4"), key=lambda c: c["tile_m"] * c["tile_n"])
    m, n, k = config["tile_m"], config["tile_n"], 4 * 256
    print(f"gemm fp4 scale layout {m}x{n}x{k}", flush=True)
    codes_a = rng.integers(0, 16, (m, k), dtype=np.uint8)
    codes_b = rng.integers(0, 16, (n, k), dtype=np.uint8)
    sa = rng.integers(126, 129, (m, k // 32), dtype=np.uint8)
    sb = rng.integers(126, 129, (n, k // 32), dtype=np.uint8)
    a = torch.from_numpy(ot.pack_e2m1(codes_a)).cuda()
    b = torch.from_numpy(ot.pack_e2m1(codes_b)).cuda()

    def product(scale_a_rows, scale_b_rows):
        return ot.gemm_reference(ot.e2m1_decode(codes_a) * np.repeat(ot.e8m0_decode(scale_a_rows), 32, axis=1),
                                 (ot.e2m1_decode(codes_b) * np.repeat(ot.e8m0_decode(scale_b_rows), 32, axis=1)).T)

    def as_rows(blocks):  # bytes read as [K/256][rows][8] -> the [rows][K/32] scales they mean
        return np.ascontiguousarray(blocks.transpose(1, 0, 2)).reshape(blocks.shape[1], -1)

    c = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    _native.gemm("fp4", config, a, b, c, m, n, k, torch.from_numpy(sa).cuda(), torch.from_numpy(sb).cuda())
    torch.cuda.synchronize()
    got = c.cpu().numpy().astype(np.float64)
    misread = product(as_rows(sa.reshape(k // 256, m, 8)), as_rows(sb.reshape(k // 256, n, 8)))
    assert np.array_equal(got, misread)
    assert not np.array_equal(got, product(sa, sb))


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32", "fp64", "int8"])
def test_reference_recipe_ragged_shape_matches_oracle(gpu, dtype):
    """The reference's own operands (bench_tensor.py:249-261: N(0,1) A, N(0,1)/sqrt(K) B drawn [K][N], INT8
    {-1,0,1}) at a ragged shape on every tile, every entry against the float64 oracle at the reference's
    tolerance (bench_tensor.py:289-299: 2e-3, 1e-10 FP64, exact INT8)."""
    import torch

    from triton_chip_benchmarks_amd import _native, gemm

    m, n, k = 1000, 744, {"int8": 1008, "fp64": 1000, "fp32": 1000}.get(dtype, 1000)
    for config in _configs(dtype):
        print(f"gemm {dtype} reference recipe tile {config['tile_m']}x{config['tile_n']}x{config['tile_k']} "
              f"shape {m}x{n}x{k}", flush=True)
        a, b, c, _scales, a_values, b_values = gemm.gemm_inputs(dtype, m, n, k, "cuda", 9, inputs="reference")
        c.fill_(-3)
        _native.gemm(dtype, config, a, b, c, m, n, k)
        torch.cuda.synchronize()
        got = c.cpu().numpy().astype(np.float64)
        expected = ot.gemm_reference(a_values.cpu().numpy(), b_values.cpu().numpy().T)
        tolerance = gemm.REFERENCE_TOLERANCE[dtype]
        if tolerance == 0.0:
            assert np.array_equal(got, expected)
        else:
            assert np.all(ot.gemm_close(got, expected, tolerance, tolerance)), np.abs(got - expected).max()


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_reference_recipe_8192_diffs_against_the_published_row(gpu, dtype):
    """8192^3 on the reference recipe, the size of its published FP16 row (results/h20_tensor.json,
    max abs error 7.49e-5 at rtol = atol = 2e-3): sampled rows against the oracle, both checksums, and every
    entry through the product's float64 device check at the reference's tolerance."""
    import json
    from pathlib import Path

    import torch

    from triton_chip_benchmarks_amd import _native, gemm

    size = 8192
    published = {row["m"]: row for row in
                 json.loads((Path(__file__).parent / "golden" / "reference_published.json").read_text())
                 ["gemm_fp16_h20"]["rows"]}[size]
    config = max(_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
    print(f"gemm {dtype} reference recipe {size}^3 tile {config['tile_m']}x{config['tile_n']}", flush=True)
    a, b, c, _scales, a_values, b_values = gemm.gemm_inputs(dtype, size, size, size, "cuda", 0, inputs="reference")
    c.fill_(float("nan"))
    _native.gemm(dtype, config, a, b, c, size, size, size)
    torch.cuda.synchronize()
    result = gemm.validate(c, gemm.reference(a_values, b_values), dtype, tolerance=gemm.REFERENCE_TOLERANCE[dtype])
    assert result["rtol"] == published["rtol"] and result["atol"] == published["atol"]
    print(f"  max abs error {result['max_abs_error']:.3g} (published H20 FP16 row: {published['max_abs_error']:.3g})",
          flush=True)
    # |C| ~ N(0,1) entries from an fp32 accumulation of 8192 products: errors of order 1e-4, as published.
    assert result["max_abs_error"] < 20 * published["max_abs_error"]
    host_a, host_b = a_values.cpu().numpy(), b_values.cpu().numpy()
    got = c.cpu().numpy().astype(np.float64)
    rng = np.random.default_rng(8)
    rows = rng.choice(size, 8, replace=False)
    sampled = ot.gemm_reference(host_a[rows], host_b.T)
    assert np.all(ot.gemm_close(got[rows], sampled, 2e-3, 2e-3))
    b_kn = host_b.T
    column_sums = ot.gemm_reference(host_a.sum(axis=0)[None, :], b_kn)[0]
    row_sums = ot.gemm_reference(host_a, host_b.sum(axis=0)[:, None])[:, 0]
    assert np.all(np.abs(got.sum(axis=0) - column_sums) <= ot.checksum_tolerance(host_a, b_kn, dtype, 0))
    assert np.all(np.abs(got.sum(axis=1) - row_sums) <= ot.checksum_tolerance(host_a, b_kn, dtype, 1))
