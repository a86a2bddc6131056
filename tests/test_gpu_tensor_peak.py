"""GPU parity of the resident-operand MFMA peak kernels against oracle.tensor.

Inputs are built with numpy on exact lattices (so any summation order gives
the same float32/float64 result), encoded bit-exactly, run through
mb_tensor_peak for every compiled tile and both B layouts, and compared with
the float64 oracle under the reference's tolerance (bench_tensor.py:302-346;
zero for INT8, exact for the FP8/FP4 product sets).
"""

import numpy as np
import pytest

from oracle import tensor as ot

pytestmark = pytest.mark.gpu

FORMATS = ["bf16", "fp16", "fp32", "int8", "fp64", "fp8", "fp4"]


def _configs(dtype):
    from triton_chip_benchmarks_amd import _native

    return _native.peak_configs(dtype)


def _encode(torch, values, dtype):
    """Device tensor holding `values` in the kernel's storage format (bit-exact)."""
    values = np.ascontiguousarray(values)
    if dtype == "bf16":
        return torch.from_numpy(ot.bf16_bits(values).view(np.int16)).view(torch.bfloat16).cuda()
    if dtype == "fp16":
        encoded = values.astype(np.float16)
        assert np.array_equal(encoded.astype(np.float64), values)
        return torch.from_numpy(encoded).cuda()
    if dtype == "fp32":
        return torch.from_numpy(values.astype(np.float32)).cuda()
    if dtype == "fp64":
        return torch.from_numpy(values.astype(np.float64)).cuda()
    if dtype == "int8":
        return torch.from_numpy(values.astype(np.int8)).cuda()
    if dtype == "fp8":
        return torch.from_numpy(ot.fp8_e4m3fn_encode_exact(values)).cuda().view(torch.float8_e4m3fn)
    raise ValueError(dtype)


def _operands(rng, dtype, blocks, m, n, k, chains):
    if dtype == "fp8":
        palette = np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0])  # FP8 GEMM set: products exact in fp32
        return palette[rng.integers(0, 6, (blocks, m, k))], palette[rng.integers(0, 6, (chains, blocks, k, n))]
    if dtype == "int8":
        return (rng.integers(-8, 9, (blocks, m, k)).astype(np.float64),
                rng.integers(-8, 9, (chains, blocks, k, n)).astype(np.float64))
    return ot.ternary_lattice(rng, (blocks, m, k)), ot.ternary_lattice(rng, (chains, blocks, k, n))


def _out_dtype(torch, dtype):
    return torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32


def _tolerance(dtype, k, iterations, a, b):
    # The int8/fp8 sets here are not the reference's ternary lattice; every
    # partial sum is still exactly representable, so the check is exact.
    return 0.0 if dtype in ("int8", "fp8") else ot.peak_tolerance(dtype, k, iterations)


@pytest.mark.parametrize("dtype", [d for d in FORMATS if d != "fp4"])
@pytest.mark.parametrize("iterations", [1, 7])
def test_peak_matches_oracle_every_tile(gpu, dtype, iterations):
    import torch

    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(1000 + iterations)
    for config in _configs(dtype):
        m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
        blocks = 3
        print(f"peak {dtype} {m}x{n}x{k} c{chains} nk={config['b_nk']} iterations={iterations}", flush=True)
        a_values, b_values = _operands(rng, dtype, blocks, m, n, k, chains)
        a = _encode(torch, a_values, dtype)
        b_stored = np.swapaxes(b_values, -1, -2) if config["b_nk"] else b_values
        b = _encode(torch, b_stored, dtype)
        c = torch.full((chains, blocks, m, n), -7, dtype=_out_dtype(torch, dtype), device="cuda")
        _native.tensor_peak(dtype, config, a, b, c, blocks, iterations)
        torch.cuda.synchronize()
        reference = ot.peak_reference(a_values, b_values, iterations)
        error = np.abs(c.cpu().numpy().astype(np.float64) - reference)
        assert np.all(error <= _tolerance(dtype, k, iterations, a_values, b_values)), (
            f"{dtype} {config}: max error {np.nanmax(error)}")


@pytest.mark.parametrize("b_nk", [0, 1])
def test_specification_resident_bf16_tile_at_1024_iterations(gpu, b_nk):
    """The headline resident BF16 configuration: a 256x256x64 tile looped 1024 times per workgroup.

    The 16x16 in-place kernel (bench.py's peak_bf16 row) on the reference's ternary/16 lattice
    (bench_tensor.py:651-672), against oracle.tensor.peak_reference under the reference's tolerance
    (bench_tensor.py:302-346), with 64 workgroups so that every wave position of the tile is covered many times.
    """
    import torch

    from triton_chip_benchmarks_amd import _native

    config = next(c for c in _native.peak_configs("bf16") if (c["tile_m"], c["tile_n"], c["tile_k"]) == (256, 256, 64)
                  and c["mfma_m"] == 16 and c["chains"] == 1 and c["b_nk"] == b_nk)
    assert _native.peak_kernel_name("bf16", config) == f"tensor_peak_bf16_256x256x64_c1_mfma16_{'nk' if b_nk else 'kn'}"
    rng = np.random.default_rng(256 + b_nk)
    blocks, iterations = 64, 1024
    print(f"peak bf16 256x256x64 c1 mfma16 nk={b_nk} blocks={blocks} iterations={iterations}", flush=True)
    a_values = ot.ternary_lattice(rng, (blocks, 256, 64))
    b_values = ot.ternary_lattice(rng, (1, blocks, 64, 256))
    a = _encode(torch, a_values, "bf16")
    b = _encode(torch, np.swapaxes(b_values, -1, -2) if b_nk else b_values, "bf16")
    c = torch.full((1, blocks, 256, 256), float("nan"), dtype=torch.float32, device="cuda")
    _native.tensor_peak("bf16", config, a, b, c, blocks, iterations)
    torch.cuda.synchronize()
    reference = ot.peak_reference(a_values, b_values, iterations)
    error = np.abs(c.cpu().numpy().astype(np.float64) - reference)
    assert np.all(error <= ot.peak_tolerance("bf16", 64, iterations)), f"max error {np.nanmax(error)}"
    assert np.count_nonzero(reference) > reference.size // 2  # the lattice is not a trivial product


@pytest.mark.parametrize("iterations", [1, 5])
def test_mxfp4_all_codes_and_scales_match_oracle(gpu, iterations):
    """All 16 E2M1 codes, packed two per byte; E8M0 scales 126..128 per 32-K group."""
    import torch

    from triton_chip_benchmarks_amd import _native

    rng = np.random.default_rng(77 + iterations)
    for config in _configs("fp4"):
        m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
        blocks = 2
        print(f"peak mxfp4 {m}x{n}x{k} c{chains} nk={config['b_nk']} iterations={iterations}", flush=True)
        codes_a = rng.integers(0, 16, (blocks, m, k), dtype=np.uint8)
        codes_b = rng.integers(0, 16, (chains, blocks, k, n), dtype=np.uint8)
        scales_a = rng.integers(126, 129, (blocks, m, k // 32), dtype=np.uint8)
        scales_b = rng.integers(126, 129, (blocks, n, k // 32), dtype=np.uint8)
        a = torch.from_numpy(ot.pack_e2m1(codes_a)).cuda()
        b_nk = ot.pack_e2m1(np.swapaxes(codes_b, -1, -2))  # [chains, blocks, N, K/2]
        b = torch.from_numpy(np.ascontiguousarray(b_nk if config["b_nk"] else np.swapaxes(b_nk, -1, -2))).cuda()
        c = torch.full((chains, blocks, m, n), float("nan"), device="cuda")
        _native.tensor_peak("fp4", config, a, b, c, blocks, iterations,
                            torch.from_numpy(scales_a).cuda(), torch.from_numpy(scales_b).cuda())
        torch.cuda.synchronize()
        group = np.arange(k) // 32
        a_values = ot.e2m1_decode(codes_a) * ot.e8m0_decode(scales_a)[:, :, group]
        b_values = ot.e2m1_decode(codes_b) * np.swapaxes(ot.e8m0_decode(scales_b)[:, :, group], -1, -2)[None]
        reference = ot.peak_reference(a_values, b_values, iterations)
        assert np.array_equal(c.cpu().numpy().astype(np.float64), reference), f"mxfp4 {config}"


def test_mxfp4_scale_doubling_probe(gpu):
    """Raising A's E8M0 scale from 127 to 128 doubles every output (bench_tensor.py:859-868)."""
    import torch

    from triton_chip_benchmarks_amd import _native

    config = min(_configs("fp4"), key=lambda c: c["tile_m"] * c["tile_n"])
    m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
    rng = np.random.default_rng(5)
    codes_a = rng.choice(np.array([1, 2, 9, 10], dtype=np.uint8), (1, m, k))
    codes_b = rng.choice(np.array([1, 2, 9, 10], dtype=np.uint8), (chains, 1, k, n))
    a = torch.from_numpy(ot.pack_e2m1(codes_a)).cuda()
    b_nk = ot.pack_e2m1(np.swapaxes(codes_b, -1, -2))
    b = torch.from_numpy(np.ascontiguousarray(b_nk if config["b_nk"] else np.swapaxes(b_nk, -1, -2))).cuda()
    outputs = []
    for scale in (127, 128):
        c = torch.empty((chains, 1, m, n), device="cuda")
        _native.tensor_peak("fp4", config, a, b, c, 1, 1,
                            torch.full((1, m, k // 32), scale, dtype=torch.uint8, device="cuda"),
                            torch.full((1, n, k // 32), 127, dtype=torch.uint8, device="cuda"))
        torch.cuda.synchronize()
        outputs.append(c.cpu().numpy().astype(np.float64))
    reference = ot.peak_reference(ot.e2m1_decode(codes_a), ot.e2m1_decode(codes_b), 1)
    assert np.array_equal(outputs[0], reference)
    assert np.array_equal(outputs[1], 2 * reference)


def test_fp32_and_fp64_precision_probes(gpu):
    """IEEE fp32 and fp64 survive their precision probes (bench_tensor.py:675-757)."""
    import torch

    from triton_chip_benchmarks_amd import _native

    for dtype, (probe_a, probe_b) in (("fp32", ot.fp32_precision_probe()), ("fp64", ot.fp64_precision_probe())):
        config = min((c for c in _configs(dtype) if not c["b_nk"]), key=lambda c: c["tile_m"] * c["tile_n"])
        m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
        a = np.zeros((1, m, k))
        a[0, :probe_a.shape[0], :probe_a.shape[1]] = probe_a
        b = np.zeros((chains, 1, k, n))
        b[:, 0, :probe_b.shape[0], :probe_b.shape[1]] = probe_b
        c = torch.empty((chains, 1, m, n), dtype=_out_dtype(torch, dtype), device="cuda")
        _native.tensor_peak(dtype, config, _encode(torch, a, dtype), _encode(torch, b, dtype), c, 1, 1)
        torch.cuda.synchronize()
        assert np.array_equal(c.cpu().numpy().astype(np.float64), ot.peak_reference(a, b, 1)), dtype


def test_bench_tensor_peak_validation_matches_oracle(gpu):
    """The product's own operand builder and validator agree with the oracle."""
    import torch

    from triton_chip_benchmarks_amd import bench_tensor

    for dtype in ("bf16", "int8", "fp8", "fp4"):
        config = [c for c in _configs(dtype) if not c["b_nk"]][0]
        if dtype == "fp4":
            a, b, c, scales, (va, vb) = bench_tensor.fp4_peak_inputs(4, config, "cuda", seed=3)
        else:
            a, b, c, vb = bench_tensor.peak_inputs(4, config, dtype, "cuda", seed=3)
            va, scales = a, None
        bench_tensor.launch_peak(dtype, config, a, b, c, 9, scales)
        torch.cuda.synchronize()
        reference = ot.peak_reference(va.double().cpu().numpy(), vb.double().cpu().numpy(), 9)
        ot.check_peak(c.cpu().numpy(), reference, dtype, config["tile_k"], 9)
