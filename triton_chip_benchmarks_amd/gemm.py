"""Dense GEMM mode of the tensor benchmark (bench_tensor.py --mode gemm).

Follows the reference's run_gemm (bench_tensor.py:1509-1595): per size and
tile, validate C against a full-precision reference, then time the kernel and
report 2*M*N*K operations. Two operand recipes (--inputs):

baseline (default), the benchmark configuration's GEMM sets:
  bf16/fp16/fp32/fp64  N(0, 1) from the seed; elementwise |C - R| <= atol +
                       rtol*|R| with rtol = atol: the reference's 2e-3 for
                       bf16/fp16/fp32 (bench_tensor.py:292-293; the
                       configuration states 1e-2, reported beside it), 1e-12
                       for fp64 (the configuration's, stricter than the
                       reference's 1e-10)
  fp8 (E4M3FN)         values from {+-0.5, +-1, +-2}; every product and partial
                       sum is exact in fp32, so C must match bit for bit
  int8                 uniform integers in [-8, 8]; exact int32
  fp4 (MXFP4)          E2M1 codes uniform over all 16 values, E8M0 scale 127
                       for every 32-element group; exact in fp32

reference, the reference's own _inputs (bench_tensor.py:249-261), so a row
diffs against its published GEMM rows on the same recipe:
  A [M][K] ~ N(0, 1) and B generated row-major [K][N] ~ N(0, 1) / sqrt(K), both
  drawn in fp32 (fp64 for fp64) and rounded to the format; INT8 from
  {-1, 0, 1}; B is then transposed to [N][K] once, outside any timing. The
  check is the reference's: rtol = atol = 2e-3, 1e-10 for fp64, exact for
  int8 (bench_tensor.py:289-299). FP8 and FP4 are refused in this recipe, as
  the reference refuses them in GEMM mode (bench_tensor.py:1404-1407).

B is stored column-major ([N][K]), both operands K-contiguous. The reference
is a float64 torch.matmul on the device, exact on the integer-valued sets.
"""

from __future__ import annotations

import math

from . import _native, audit, formats, roofline
from .common import available_memory_bytes, emit_unsupported, measure

DEFAULT_SIZES = {"bf16": [8192], "fp16": [8192], "fp32": [8192], "fp8": [8192], "int8": [8192], "fp64": [4096],
                 "fp4": [16384]}
# rtol = atol per format; 0 means bit-exact (the operand sets are exact in the accumulator).
TOLERANCE = {"bf16": 2e-3, "fp16": 2e-3, "fp32": 2e-3, "fp64": 1e-12, "fp8": 0.0, "int8": 0.0, "fp4": 0.0}
# The benchmark configuration's stated BF16/FP16 bound, looser than the check above; rows report their worst
# error against it too.
STATED_TOLERANCE = {"bf16": 1e-2, "fp16": 1e-2}
# The reference's own rule for its own operands (bench_tensor.py:291-293): 0 for int32 output, 1e-10 for
# fp64, 2e-3 otherwise (IEEE dot precision).
REFERENCE_TOLERANCE = {"bf16": 2e-3, "fp16": 2e-3, "fp32": 2e-3, "fp64": 1e-10, "int8": 0.0}
REFERENCE_SIZES = [2048, 4096, 8192]  # bench_tensor.py:1319
REFERENCE_REFUSAL = {"fp8": "This benchmark implements FP8 E4M3FN in --mode peak only",
                     "fp4": "This benchmark implements MX FP4 (E2M1) in --mode peak only"}  # bench_tensor.py:1404-1407
REFERENCE_PATTERN = {"bf16": "A ~ N(0,1), B ~ N(0,1)/sqrt(K) drawn [K][N] in fp32, rounded to bf16",
                     "fp16": "A ~ N(0,1), B ~ N(0,1)/sqrt(K) drawn [K][N] in fp32, rounded to fp16",
                     "fp32": "A ~ N(0,1), B ~ N(0,1)/sqrt(K) drawn [K][N] in fp32",
                     "fp64": "A ~ N(0,1), B ~ N(0,1)/sqrt(K) drawn [K][N] in fp64",
                     "int8": "A, B uniform over {-1, 0, 1}, B drawn [K][N]"}
INPUT_PATTERN = {
    "bf16": "N(0,1) values rounded to bf16", "fp16": "N(0,1) values rounded to fp16", "fp32": "N(0,1)",
    "fp64": "N(0,1)", "fp8": "uniform over {+-0.5, +-1, +-2} (E4M3FN exact)", "int8": "uniform integers in [-8, 8]",
    "fp4": "E2M1 codes uniform over all 16 values, E8M0 scale 127 (2^0) per 32 K elements"}


def _torch():
    import torch

    return torch


def gemm_inputs(dtype: str, m: int, n: int, k: int, device, seed: int = 0, inputs: str = "baseline"):
    """(a, b, c, scales, a_values, b_values): b stored [n][k]; *_values are float64 [.., k] views."""
    torch = _torch()
    generator = torch.Generator(device=device).manual_seed(seed)
    if inputs == "reference":
        return _reference_inputs(dtype, m, n, k, device, generator)
    if inputs != "baseline":
        raise ValueError(f"unknown operand recipe {inputs!r}")
    scales = None
    if dtype == "fp4":
        codes_a = torch.randint(0, 16, (m, k), device=device, generator=generator, dtype=torch.uint8)
        codes_b = torch.randint(0, 16, (n, k), device=device, generator=generator, dtype=torch.uint8)
        a, b = formats.pack_e2m1_pairs(codes_a), formats.pack_e2m1_pairs(codes_b)
        blocks = -(-k // 256)  # K-step scale blocks [ceil(K/256)][rows][8] (mb_gemm's layout)
        scales = (torch.full((blocks, m, 8), formats.E8M0_UNIT_SCALE, dtype=torch.uint8, device=device),
                  torch.full((blocks, n, 8), formats.E8M0_UNIT_SCALE, dtype=torch.uint8, device=device))
        a_values, b_values = formats.e2m1_decode(codes_a), formats.e2m1_decode(codes_b)
        del codes_a, codes_b
    elif dtype == "fp8":
        palette = torch.tensor([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], device=device)
        a = palette[torch.randint(0, 6, (m, k), device=device, generator=generator)].to(torch.float8_e4m3fn)
        b = palette[torch.randint(0, 6, (n, k), device=device, generator=generator)].to(torch.float8_e4m3fn)
        a_values, b_values = a.double(), b.double()
    elif dtype == "int8":
        a = torch.randint(-8, 9, (m, k), device=device, generator=generator, dtype=torch.int8)
        b = torch.randint(-8, 9, (n, k), device=device, generator=generator, dtype=torch.int8)
        a_values, b_values = a.double(), b.double()
    else:
        store = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32, "fp64": torch.float64}[dtype]
        a = torch.randn((m, k), device=device, generator=generator, dtype=torch.float64).to(store)
        b = torch.randn((n, k), device=device, generator=generator, dtype=torch.float64).to(store)
        a_values, b_values = a.double(), b.double()
    out = torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32
    c = torch.empty((m, n), dtype=out, device=device)
    return a, b, c, scales, a_values, b_values


def _reference_inputs(dtype: str, m: int, n: int, k: int, device, generator):
    """The reference's _inputs (bench_tensor.py:249-261), with B transposed to [N][K] once."""
    torch = _torch()
    if dtype in REFERENCE_REFUSAL:
        raise ValueError(REFERENCE_REFUSAL[dtype])
    if dtype == "int8":
        a = torch.randint(-1, 2, (m, k), device=device, generator=generator, dtype=torch.int8)
        b_kn = torch.randint(-1, 2, (k, n), device=device, generator=generator, dtype=torch.int8)
    else:
        store = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32, "fp64": torch.float64}[dtype]
        drawn = torch.float64 if dtype == "fp64" else torch.float32
        a = torch.randn((m, k), device=device, generator=generator, dtype=drawn).to(store)
        b_kn = (torch.randn((k, n), device=device, generator=generator, dtype=drawn) * (1.0 / math.sqrt(k))).to(store)
    b = b_kn.t().contiguous()
    del b_kn
    out = torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32
    c = torch.empty((m, n), dtype=out, device=device)
    return a, b, c, None, a.double(), b.double()


def reference(a_values, b_values):
    """C = A . B in float64 (B given [n][k])."""
    return _torch().matmul(a_values, b_values.t().contiguous())


def validate(c, ref, dtype: str, rows_per_chunk: int = 2048, tolerance: float | None = None) -> dict:
    """Every entry of C against the float64 reference R (bench_tensor.py:289-299).

    Passes when |C - R| <= atol + rtol * |R| holds for every entry, with
    rtol = atol = TOLERANCE[dtype], as torch.testing.assert_close applies it;
    a tolerance of 0 demands bit equality. NaN or infinite entries fail.
    Rows are checked in chunks so the float64 temporaries stay small.
    `tolerance` overrides TOLERANCE[dtype] (the reference recipe's own rule).
    """
    torch = _torch()
    tolerance = TOLERANCE[dtype] if tolerance is None else tolerance
    max_error, max_ratio, failures, worst = 0.0, 0.0, 0, None
    for start in range(0, c.shape[0], rows_per_chunk):
        got = c[start:start + rows_per_chunk].double()
        expected = ref[start:start + rows_per_chunk]
        error = (got - expected).abs()
        allowed = tolerance + tolerance * expected.abs()
        bad = ~(torch.isfinite(got) & (error <= allowed))
        count = int(bad.sum().item())
        if count:
            failures += count
            if worst is None:
                index = tuple(int(i) for i in torch.nonzero(bad)[0].tolist())
                worst = ((start + index[0],) + index[1:], got[index].item(), expected[index].item())
        finite = torch.isfinite(error)
        if finite.any():
            max_error = max(max_error, error[finite].max().item())
            if tolerance:
                max_ratio = max(max_ratio, (error[finite] / allowed[finite]).max().item())
    if failures:
        where, got_value, expected_value = worst
        raise RuntimeError(f"GEMM correctness failed ({dtype}): {failures} entries outside rtol = atol = "
                           f"{tolerance:g}; first at {list(where)}: {got_value!r} vs {expected_value!r}")
    stated = STATED_TOLERANCE.get(dtype)
    return {"passed": True, "max_abs_error": max_error, "rtol": tolerance, "atol": tolerance,
            "max_error_over_allowed": max_ratio if tolerance else 0.0,
            **({"stated_tolerance": stated,
                "max_error_over_stated": max_ratio * tolerance / stated} if stated and tolerance else {}),
            "tolerance_kind": "exact" if not tolerance else "elementwise |C-R| <= atol + rtol*|R|",
            "reference": "FP64 torch.matmul on the device (exact for the integer-valued operand sets)"}


def run_gemm(args, metadata: dict, device) -> None:
    from .bench_tensor import accumulator_name, precision_descriptor, rates

    torch = _torch()
    dtype = args.dtype
    if args.input_precision == "tf32":
        emit_unsupported("tensor", metadata, args, "gfx950 has no TF32 matrix instruction")
        return
    inputs = getattr(args, "inputs", "baseline")
    if inputs == "reference" and dtype in REFERENCE_REFUSAL:
        emit_unsupported("tensor", metadata, args, REFERENCE_REFUSAL[dtype])
        return
    pattern = (REFERENCE_PATTERN if inputs == "reference" else INPUT_PATTERN)[dtype]
    tolerance = REFERENCE_TOLERANCE[dtype] if inputs == "reference" else TOLERANCE[dtype]
    sizes = (args.sizes if getattr(args, "sizes_given", False)
             else REFERENCE_SIZES if inputs == "reference" else DEFAULT_SIZES[dtype])
    if args.quick:
        sizes = [256, 512]
    candidates = _native.gemm_configs(dtype)
    if args.tiles:
        wanted = {tuple(int(x) for x in tile.split("x")) for tile in args.tiles}
        candidates = [c for c in candidates if (c["tile_m"], c["tile_n"], c["tile_k"]) in wanted]
    if args.quick:
        candidates = candidates[:1]
    unit = "TOPS" if dtype == "int8" else "TFLOP/s"
    peak_value = roofline.PEAKS[f"tensor_{dtype}"][0]
    print(f"\nMatrix GEMM: {dtype} inputs ({inputs} recipe: {pattern}), {accumulator_name(dtype).upper()} "
          "accumulate/output, B column-major; 2*M*N*K operations")
    print(f"  N        tile M/N/K   median ms  median {unit}  peak {unit}  % peak   error")
    rows = []
    for size in sizes:
        free = available_memory_bytes()
        required = size * size * 48
        if free is not None and required > 0.8 * free:
            raise RuntimeError(f"N={size} needs about {required / 2**30:.1f} GiB; reduce --sizes")
        a, b, c, scales, a_values, b_values = gemm_inputs(dtype, size, size, size, device, args.seed, inputs)
        ref = reference(a_values, b_values)
        del a_values, b_values
        for config in candidates:
            # The kernel this shape actually launches (a ragged shape runs the tile's checked variant).
            kernel = _native.gemm_launched_kernel(dtype, config, size, size, size, *(scales or (None, None)))
            c.fill_(-2**31 if dtype == "int8" else float("nan"))

            def run(config=config):
                _native.gemm(dtype, config, a, b, c, size, size, size, *(scales or (None, None)))

            run()
            torch.cuda.synchronize()
            correctness = validate(c, ref, dtype, tolerance=tolerance)
            info = dict(audit.resources(kernel))
            info.update(audit.audit_tensor(audit.instructions(kernel), dtype, args.input_precision))
            if info.get("register_spills"):
                rows.append({"mode": "gemm", "m": size, "n": size, "k": size, "dtype": dtype, "config": config,
                             "status": "skipped", "reason": "configuration spills registers"})
                continue
            timing = measure(run, args)
            row_rates = rates(2 * size**3, timing, dtype)
            descriptor = precision_descriptor(dtype, args.input_precision)
            row = {"mode": "gemm", "m": size, "n": size, "k": size, "dtype": dtype,
                   "measurement_kind": f"{descriptor['math_mode']}_gemm" if dtype in ("fp32", "fp64")
                   else "dense_tensor_gemm",
                   "execution_kind": info["execution_kind"],
                   "precision_verified": info["instruction_precision_verified"],
                   "accumulator_dtype": accumulator_name(dtype), "output_dtype": accumulator_name(dtype),
                   "layout": "A row-major, B column-major (both K-contiguous)", "inputs": inputs, "input_pattern": pattern,
                   **descriptor, **row_rates,
                   "config": {"block_m": config["tile_m"], "block_n": config["tile_n"], "block_k": config["tile_k"],
                              "threads": config["threads"]},
                   "kernel": kernel, "status": "ok", "correctness": correctness, "compiled": info,
                   "roofline": roofline.describe(f"tensor_{dtype}", row_rates["peak_teraops_per_second"]),
                   **timing}
            rows.append(row)
            print(f"{size:5d}   {config['tile_m']:>4}/{config['tile_n']}/{config['tile_k']:<4} "
                  f"{timing['median_ms']:10.4f} {row_rates['median_teraops_per_second']:12.2f} "
                  f"{row_rates['peak_teraops_per_second']:10.2f} "
                  f"{100 * row_rates['peak_teraops_per_second'] / peak_value:7.1f}   "
                  f"{correctness['max_abs_error']:.3g}", flush=True)
        del a, b, c, ref
    from .bench_tensor import emit_tensor_results

    emit_tensor_results(metadata, args, rows)
