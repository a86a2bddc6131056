#!/usr/bin/env python3
"""Matrix-core peak (resident operands) and dense GEMM throughput on one MI355X.

Mirrors the reference's bench_tensor.py CLI, operand lattices, validation and
row fields (bench_tensor.py:84-403, 1149-1599). The kernels are gfx950 MFMA
kernels of libmi355x_bench.so:
  peak: mb_tensor_peak - each workgroup stages A and two B tiles through LDS,
        keeps its MFMA fragments in registers and repeats v_mfma over two
        independent accumulator chains `iterations` times;
  gemm: mb_gemm - LDS double-buffered MFMA GEMM.
FP16/BF16/FP8/MXFP4/FP32 accumulate in fp32, FP64 in fp64 and INT8 in int32.
TF32 has no gfx950 instruction and is reported unsupported.
"""

from __future__ import annotations

import argparse
from pathlib import Path
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd import _native, audit, cpu_baseline, formats, roofline
    from triton_chip_benchmarks_amd.common import (add_common_arguments, available_memory_bytes, emit_results,
                                                   emit_unsupported, get_device, measure, setup_device)
else:
    from . import _native, audit, cpu_baseline, formats, roofline
    from .common import (add_common_arguments, available_memory_bytes, emit_results, emit_unsupported,
                         get_device, measure, setup_device)

DTYPES = ("fp16", "bf16", "fp8", "fp4", "fp32", "tf32", "int8", "fp64")
TF32_REASON = ("gfx950 (CDNA4) has no xf32/TF32 matrix instruction: v_mfma_f32_*_xf32 exists only up to "
               "gfx942, so no TF32 matrix rate can be measured on MI355X. IEEE FP32 is the tensor_fp32 row")


class TensorUnsupportedError(RuntimeError):
    """The requested format or its required execution precision is unavailable."""


def _torch():
    import torch

    return torch


def storage_dtype(dtype: str):
    torch = _torch()
    return {"fp16": torch.float16, "bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "fp4": torch.uint8,
            "fp32": torch.float32, "tf32": torch.float32, "int8": torch.int8, "fp64": torch.float64}[dtype]


def output_dtype(dtype: str):
    torch = _torch()
    return torch.int32 if dtype == "int8" else torch.float64 if dtype == "fp64" else torch.float32


def accumulator_name(dtype: str) -> str:
    return "int32" if dtype == "int8" else "fp64" if dtype == "fp64" else "fp32"


def rates(operation_count: int, timing: dict, dtype: str) -> dict:
    """Rate fields of one row (bench_tensor.py:84-93)."""
    median = operation_count / (timing["median_ms"] * 1e9)
    peak = operation_count / (timing.get("min_ms", timing["median_ms"]) * 1e9)
    integer = dtype == "int8"
    return {"operation_count": operation_count,
            "operation_type": "integer" if integer else "floating_point",
            "throughput_unit": "TOPS" if integer else "TFLOP/s",
            "median_teraops_per_second": median, "peak_teraops_per_second": peak,
            **({"integer_ops": operation_count, "tops": median, "peak_tops": peak} if integer else
               {"flops": operation_count, "tflops": median, "peak_tflops": peak})}


def peak_tolerance(dtype: str, block_k: int, iterations: int) -> float:
    """Bound on accumulated rounding of the resident recurrence (bench_tensor.py:302-325).

    Lattice operands make every exact dot a multiple of 1/256 (of 0.25 for
    FP4); the accumulator rounds once per dot, adding at most
    iterations * block_k * step * unit roundoff, with a factor 4 of headroom -
    still far below one lattice step, which a skipped dot would change.
    """
    if dtype == "int8":
        return 0.0
    if dtype == "fp4":
        return 4.0 * iterations * block_k * 1.0 * 2.0**-24
    unit_roundoff = 2.0**-53 if dtype == "fp64" else 2.0**-24
    return 4.0 * iterations * block_k * (1.0 / 256.0) * unit_roundoff


def validate_peak(c, reference, dtype: str, block_k: int, iterations: int) -> dict:
    """Every output against the exact scaled dot (bench_tensor.py:328-346)."""
    torch = _torch()
    tolerance = peak_tolerance(dtype, block_k, iterations)
    torch.testing.assert_close(c, reference, rtol=0, atol=tolerance)
    return {"passed": True, "max_abs_error": (c.double() - reference.double()).abs().max().item(),
            "rtol": 0, "atol": tolerance,
            "reference": f"exact {accumulator_name(dtype).upper()} dot * iterations",
            "tolerance_basis": ("exact INT32 equality" if dtype == "int8" else
                                "accumulated accumulator unit roundoff over all iterations, "
                                "far below the 1/256 exact-operand lattice step")}


def precision_descriptor(dtype: str, dot_input_precision: str | None) -> dict:
    """Format description fields (bench_tensor.py:381-403)."""
    storage = "fp32" if dtype == "fp32" else ("e4m3fn" if dtype == "fp8" else "e2m1" if dtype == "fp4" else dtype)
    if dtype == "fp32":
        math_mode = "tf32" if dot_input_precision == "tf32" else "ieee_fp32"
    elif dtype == "fp4":
        math_mode = "mxfp4_e2m1"
    else:
        math_mode = dtype
    descriptor = {"input_format": storage, "input_storage_dtype": storage,
                  "dot_input_precision": dot_input_precision, "math_mode": math_mode}
    if dtype == "fp4":
        descriptor.update({"container_dtype": "uint8", "elements_per_container": formats.FP4_PACKING_FACTOR,
                           "scale_format": "e8m0", "scale_group_size": formats.MX_GROUP_SIZE,
                           "scale_value": "2**0 (E8M0 code 127) for every group", "microscaled": True,
                           "dot_operation": "v_mfma_scale_f32_32x32x64_f8f6f4 (cbsz:4 blgp:4)"})
    return descriptor


def _generator(device, seed):
    torch = _torch()
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    return generator


FP8_DENSE_SET = (-2.0, -1.0, -0.5, 0.5, 1.0, 2.0)


def peak_inputs(blocks: int, config: dict, dtype: str, device, seed: int = 0, operands: str = "lattice"):
    """Exact-lattice operands (bench_tensor.py:647-672) in the kernel's layouts.

    Returns (a, b, c, b_logical): b is stored [chains, blocks, K, N] or, for
    b_nk configurations, [chains, blocks, N, K]; b_logical is always the
    [chains, blocks, K, N] view used by the reference. operands="dense"
    (FP8 only) draws every A and B entry from {+-0.5, +-1, +-2} instead of
    the reference's one-hot A: each dot entry is a multiple of 1/4 of
    magnitude at most 4*K, so 1024 accumulations stay exact in fp32 for K <= 2048.
    """
    torch = _torch()
    m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
    generator = _generator(device, seed)
    store = storage_dtype(dtype)
    if operands not in ("lattice", "dense") or (operands == "dense" and dtype != "fp8"):
        raise ValueError(f"operand set {operands!r} is not defined for {dtype}")
    if operands == "dense":
        palette = torch.tensor(FP8_DENSE_SET, device=device)
        a = palette[torch.randint(len(FP8_DENSE_SET), (blocks, m, k), device=device, generator=generator)].to(store)
        b = palette[torch.randint(len(FP8_DENSE_SET), (chains, blocks, k, n), device=device,
                                  generator=generator)].to(store)
    elif dtype == "fp8":
        # One-hot rows of 1/16 in A and signs/16 in B: every dot is +-1/256.
        a = torch.zeros((blocks, m, k), device=device)
        hot = torch.randint(k, (blocks, m, 1), device=device, generator=generator)
        a.scatter_(2, hot, 1 / 16)
        a = a.to(store)
        b = torch.randint(0, 2, (chains, blocks, k, n), device=device, generator=generator).float()
        b = b.mul_(2).sub_(1).mul_(1 / 16).to(store)
    elif dtype == "int8":
        a = torch.randint(-1, 2, (blocks, m, k), device=device, dtype=torch.int8, generator=generator)
        b = torch.randint(-1, 2, (chains, blocks, k, n), device=device, dtype=torch.int8, generator=generator)
    else:
        a = torch.randint(-1, 2, (blocks, m, k), device=device, generator=generator).double().mul_(1 / 16).to(store)
        b = torch.randint(-1, 2, (chains, blocks, k, n), device=device, generator=generator).double()
        b = b.mul_(1 / 16).to(store)
    b_logical = b
    if config.get("b_nk"):
        b = b.transpose(-1, -2).contiguous()
    c = torch.empty((chains, blocks, m, n), dtype=output_dtype(dtype), device=device)
    return a, b, c, b_logical


def fp4_peak_inputs(blocks: int, config: dict, device, seed: int = 0, palette=(1, 2, 9, 10)):
    """Packed MX FP4 operands, unit scales and their exact values (bench_tensor.py:614-644).

    The default palette holds the codes of +-0.5 and +-1.0; any subset of the
    16 codes may be passed (the MXFP4 GEMM configuration uses all 16).
    """
    torch = _torch()
    m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
    generator = _generator(device, seed)
    choices = torch.tensor(palette, dtype=torch.uint8, device=device)
    codes_a = choices[torch.randint(len(palette), (blocks, m, k), device=device, generator=generator)]
    codes_b = choices[torch.randint(len(palette), (chains, blocks, k, n), device=device, generator=generator)]
    a = formats.pack_e2m1_pairs(codes_a)
    if config.get("b_nk"):
        b = formats.pack_e2m1_pairs(codes_b.transpose(-1, -2).contiguous())          # [.., N, K/2]
    else:
        b = formats.pack_e2m1_pairs(codes_b.transpose(-1, -2).contiguous())
        b = b.transpose(-1, -2).contiguous()                                           # [.., K/2, N]
    groups = k // formats.MX_GROUP_SIZE
    scale_a = torch.full((blocks, m, groups), formats.E8M0_UNIT_SCALE, dtype=torch.uint8, device=device)
    scale_b = torch.full((blocks, n, groups), formats.E8M0_UNIT_SCALE, dtype=torch.uint8, device=device)
    c = torch.empty((chains, blocks, m, n), dtype=torch.float32, device=device)
    return a, b, c, (scale_a, scale_b), (formats.e2m1_decode(codes_a), formats.e2m1_decode(codes_b))


def exact_reference(a_values, b_values, iterations: int, out_dtype):
    """iterations * (A . B_c) for every chain, exact in float64 on the lattice."""
    torch = _torch()
    a64 = a_values.double()
    product = torch.stack([torch.matmul(a64, b_values[c].double().contiguous()) for c in range(b_values.shape[0])])
    return (product * iterations).to(out_dtype)


def launch_peak(dtype, config, a, b, c, iterations, scales=None):
    blocks = a.shape[0]
    scale_a, scale_b = scales if scales is not None else (None, None)
    _native.tensor_peak(dtype, config, a, b, c, blocks, iterations, scale_a, scale_b)


def _smallest(configs):
    return min(configs, key=lambda config: config["tile_m"] * config["tile_n"] * config["tile_k"])


def fp32_probe_matrix(size: int = 32):
    """A of the FP32 probe: 1+2^-12 everywhere (lost by TF32, BF16 and FP16 rounding), 1+2^-9 at
    [0, 1] (lost by BF16) and 2^20 at [0, 2] (beyond FP16's range) (bench_tensor.py:678-687)."""
    torch = _torch()
    probe = torch.full((size, size), 1.0 + 2.0**-12, dtype=torch.float32)
    probe[0, 1], probe[0, 2] = 1.0 + 2.0**-9, 2.0**20
    return probe


def fp64_probe_matrix(size: int = 32, inner: int = 16):
    """A of the FP64 probe: 1+2^-40 (lost by any FP32 rounding) with row r's column 0 set to r+1,
    so a permuted output row is visible (bench_tensor.py:728-735)."""
    torch = _torch()
    probe = torch.full((size, inner), 1.0 + 2.0**-40, dtype=torch.float64)
    probe[:, 0] = torch.arange(1, size + 1, dtype=torch.float64)
    return probe


def validate_fp32_precision(device, configs) -> dict:
    """IEEE vs TF32/BF16/FP16 probe through the peak kernel (bench_tensor.py:675-714).

    A holds 1+2^-12, 1+2^-9 and 2^20, B is the identity; only an IEEE fp32
    multiply returns A exactly.
    """
    torch = _torch()
    config = _smallest([c for c in configs if not c["b_nk"]])
    m, n, k = config["tile_m"], config["tile_n"], config["tile_k"]
    size = 32
    probe = fp32_probe_matrix(size)
    a = torch.zeros((1, m, k), dtype=torch.float32)
    a[0, :size, :size] = probe
    b = torch.zeros((config["chains"], 1, k, n), dtype=torch.float32)
    b[:, 0, :size, :size] = torch.eye(size)
    c = torch.empty((config["chains"], 1, m, n), dtype=torch.float32, device=device)
    launch_peak("fp32", config, a.to(device), b.to(device), c, 1)
    torch.cuda.synchronize()
    expected = torch.zeros((m, n), dtype=torch.float32)
    expected[:size, :size] = probe
    error = max((c[chain, 0].cpu() - expected).abs().max().item() for chain in range(config["chains"]))
    if error != 0.0:
        raise TensorUnsupportedError("The kernel did not compute IEEE FP32: precision probe max absolute "
                                     f"error {error}")
    return {"passed": True, "max_abs_error": error, "probe_values": [1.0 + 2.0**-12, 1.0 + 2.0**-9, 2.0**20],
            "kernel_mode": "peak", "probed_tile": f"{m}x{n}x{k}",
            "description": "A contains 1+2^-12, 1+2^-9, and 2^20; B=identity; distinguishes IEEE, TF32, BF16, "
                           "and FP16"}


def validate_fp64_precision(device, configs) -> dict:
    """FP64 probe with a per-row marker (bench_tensor.py:717-757)."""
    torch = _torch()
    config = _smallest([c for c in configs if not c["b_nk"]])
    m, n, k = config["tile_m"], config["tile_n"], config["tile_k"]
    size, inner = 32, 16
    a = torch.zeros((1, m, k), dtype=torch.float64)
    a[0, :size, :inner] = fp64_probe_matrix(size, inner)
    b = torch.zeros((config["chains"], 1, k, n), dtype=torch.float64)
    b[:, 0, :inner, :size] = torch.eye(inner, size, dtype=torch.float64)
    c = torch.empty((config["chains"], 1, m, n), dtype=torch.float64, device=device)
    launch_peak("fp64", config, a.to(device), b.to(device), c, 1)
    torch.cuda.synchronize()
    expected = torch.zeros((m, n), dtype=torch.float64)
    expected[:size, :inner] = a[0, :size, :inner]
    error = max((c[chain, 0].cpu() - expected).abs().max().item() for chain in range(config["chains"]))
    if error != 0.0:
        rows_match = sorted(map(tuple, c[0, 0].cpu().tolist())) == sorted(map(tuple, expected.tolist()))
        detail = ("the returned rows are a permutation of the correct rows" if rows_match
                  else f"probe error={error}")
        raise TensorUnsupportedError(f"The kernel did not compute FP64 correctly: {detail}")
    return {"passed": True, "max_abs_error": error, "kernel_mode": "peak", "probed_tile": f"{m}x{n}x{k}",
            "description": "FP64 (1+2^-40) with a per-row marker times identity; rejects FP32 fallback and "
                           "permuted output rows"}


def validate_fp8_storage(device) -> dict:
    """FP8 E4M3FN round trip of exactly representable values (bench_tensor.py:760-779)."""
    torch = _torch()
    probe = torch.tensor([1 / 16, -1 / 16, 1.0], dtype=torch.float32, device=device)
    restored = probe.to(torch.float8_e4m3fn).float()
    error = (restored - probe).abs().max().item()
    if error != 0.0:
        raise TensorUnsupportedError(f"FP8 E4M3FN storage did not round-trip; error={error}")
    return {"passed": True, "max_abs_error": error, "probe_values": [1 / 16, -1 / 16, 1.0],
            "description": "FP8 E4M3FN storage round-trip of exactly representable values"}


def validate_fp4_arithmetic(device, configs) -> dict:
    """Exact E2M1 products, then E8M0 scale 127 -> 128 must double C (bench_tensor.py:829-886)."""
    torch = _torch()
    config = _smallest([c for c in configs if not c["b_nk"]])
    a, b, c, scales, values = fp4_peak_inputs(1, config, device, seed=0)
    launch_peak("fp4", config, a, b, c, 1, scales)
    torch.cuda.synchronize()
    reference = exact_reference(values[0], values[1], 1, torch.float64)
    error = (c.double() - reference).abs().max().item()
    if error != 0.0:
        raise TensorUnsupportedError(f"MX FP4 products are not exact: max_abs_error={error}")
    doubled = torch.empty_like(c)
    launch_peak("fp4", config, a, b, doubled, 1, (torch.full_like(scales[0], formats.E8M0_UNIT_SCALE + 1),
                                                   scales[1]))
    torch.cuda.synchronize()
    scale_error = (doubled.double() - 2.0 * reference).abs().max().item()
    if scale_error != 0.0:
        raise TensorUnsupportedError("The kernel did not apply the E8M0 scale: raising A's scale from 2**0 to "
                                     f"2**1 left max_abs_error={scale_error} against the doubled reference")
    m, n, k = config["tile_m"], config["tile_n"], config["tile_k"]
    return {"passed": True, "kernel_mode": "peak", "probed_tile": f"{m}x{n}x{k}", "max_abs_error": 0.0,
            "scale_sensitivity_verified": True,
            "description": "MX FP4 (E2M1 packed two per uint8, E8M0 unit scales) exact-product and "
                           "scale-application probe"}


def compiled_info(kernel: str, dtype: str, input_precision: str | None) -> dict:
    """Instruction audit plus resource figures of one kernel."""
    info = dict(audit.resources(kernel))
    info["spill_count"] = info.get("register_spills")
    info["kernel"] = kernel
    try:
        info.update(audit.audit_tensor(audit.instructions(kernel), dtype, input_precision))
    except audit.TensorAuditError as exc:
        raise TensorUnsupportedError(str(exc)) from exc
    info.update(audit.loop_summary(kernel))
    return info


def peak_configs(dtype: str, b_layout: str) -> list[dict]:
    configs = _native.peak_configs(dtype)
    wanted = {"kn": [0], "nk": [1], "both": [0, 1]}[b_layout]
    return [config for config in configs if config["b_nk"] in wanted]


def run_peak(args, metadata: dict, device) -> None:
    torch = _torch()
    if not metadata.get("sm_count"):
        raise RuntimeError("The runtime did not report the compute-unit count; provide --compute-units")
    candidates = peak_configs(args.dtype, args.b_layout)
    if args.tiles:
        wanted = {tuple(int(x) for x in tile.split("x")) for tile in args.tiles}
        candidates = [c for c in candidates if (c["tile_m"], c["tile_n"], c["tile_k"]) in wanted]
    blocks_per_sm_values = list(args.blocks_per_sm)
    if args.quick:
        candidates = candidates[:1]
        blocks_per_sm_values = [1]
        args.iterations = min(args.iterations, 64)
    accumulator = accumulator_name(args.dtype)
    unit = "TOPS" if args.dtype == "int8" else "TFLOP/s"
    peak_value = roofline.PEAKS[f"tensor_{args.dtype}"][0]
    text = (f"FP32 storage, {args.input_precision.upper()} dot precision" if args.dtype == "fp32" else
            "MX FP4 (E2M1) operands with E8M0 group scales" if args.dtype == "fp4" else f"{args.dtype} operands")
    print(f"\nMatrix peak: resident {text}, independent {accumulator.upper()} accumulator chains (v_mfma)")
    print(f"Iterations={args.iterations}; operations=2*tile_M*tile_N*tile_K*iterations*chains*blocks")
    print(f" tile M/N/K     mfma  chains  blocks/CU  median ms    min ms  median {unit}  peak {unit}  % peak  regs")
    rows = []
    for config in candidates:
        m, n, k, chains = config["tile_m"], config["tile_n"], config["tile_k"], config["chains"]
        kernel = _native.peak_kernel_name(args.dtype, config)
        for blocks_per_sm in blocks_per_sm_values:
            blocks = blocks_per_sm * metadata["sm_count"]
            free_bytes = available_memory_bytes()
            if free_bytes is not None and blocks * (m * k + chains * k * n + 8 * chains * m * n) * 8 > 0.8 * free_bytes:
                raise RuntimeError("Peak validation exceeds available memory; reduce --blocks-per-sm")
            try:
                scales = None
                if args.dtype == "fp4":
                    a, b, c, scales, (values_a, values_b) = fp4_peak_inputs(blocks, config, device, args.seed)
                else:
                    a, b, c, b_logical = peak_inputs(blocks, config, args.dtype, device, args.seed)
                    values_a, values_b = a, b_logical
                c.fill_(-2**31 if args.dtype == "int8" else float("nan"))
                launch_peak(args.dtype, config, a, b, c, args.iterations, scales)
                info = compiled_info(kernel, args.dtype, args.input_precision)
            except TensorUnsupportedError as exc:
                rows.append({"mode": "peak", "dtype": args.dtype, "config": config, "blocks_per_sm": blocks_per_sm,
                             "status": "unsupported", "reason": str(exc)})
                print(f"  config={config}: unsupported ({exc})")
                continue
            reference = exact_reference(values_a, values_b, args.iterations, output_dtype(args.dtype))
            torch.cuda.synchronize()
            correctness = validate_peak(c, reference, args.dtype, k, args.iterations)
            del reference
            if info["spill_count"]:
                rows.append({"mode": "peak", "dtype": args.dtype, "config": config, "blocks_per_sm": blocks_per_sm,
                             "status": "skipped", "reason": "configuration spills registers"})
                continue
            timing = measure(lambda: launch_peak(args.dtype, config, a, b, c, args.iterations, scales), args)
            operations = 2 * m * n * k * args.iterations * chains * blocks
            row_rates = rates(operations, timing, args.dtype)
            descriptor = precision_descriptor(args.dtype, args.input_precision)
            if args.dtype in ("fp32", "fp64"):
                measurement_kind = (f"{descriptor['math_mode']}_tensor_peak" if info["native_tensor_verified"]
                                    else f"{descriptor['math_mode']}_matrix_throughput")
            else:
                measurement_kind = "native_tensor_peak" if info["native_tensor_verified"] else "unverified"
            row = {"mode": "peak", "dtype": args.dtype,
                   "config": {"block_m": m, "block_n": n, "block_k": k, "chains": chains,
                              "b_layout": "nk" if config["b_nk"] else "kn", "threads": config["threads"],
                              "mfma_m": config["mfma_m"]},
                   "kernel": kernel, "measurement_kind": measurement_kind,
                   "execution_kind": info["execution_kind"],
                   "precision_verified": bool(metadata.get("tensor_precision_probe"))
                   if args.dtype in ("fp32", "fp64") else info["instruction_precision_verified"],
                   "accumulator_dtype": accumulator, "output_dtype": accumulator, "blocks": blocks,
                   "blocks_per_sm": blocks_per_sm, "iterations": args.iterations, **row_rates, **descriptor,
                   "input_pattern": ("random one-hot A; random signed B; dense MFMA operations" if args.dtype == "fp8"
                                     else "random ternary integers" if args.dtype == "int8"
                                     else "random E2M1 codes for +/-0.5 and +/-1.0, packed two per uint8; unit "
                                          "E8M0 scales" if args.dtype == "fp4"
                                     else "random ternary exact binary fractions"),
                   "accumulation_policy": accumulation_policy(args.dtype),
                   "precision_probe": metadata.get("tensor_precision_probe"),
                   "correctness": correctness, "compiled": info, "status": "ok",
                   "roofline": roofline.describe(f"tensor_{args.dtype}", row_rates["peak_teraops_per_second"]),
                   **timing}
            rows.append(row)
            print(f"{m:>4}/{n}/{k:<5} {config['mfma_m']:>2}x{config['mfma_m']:<2} {chains:>6} {blocks_per_sm:10d} {timing['median_ms']:10.4f} "
                  f"{timing['min_ms']:9.4f} {row_rates['median_teraops_per_second']:12.2f} "
                  f"{row_rates['peak_teraops_per_second']:10.2f} "
                  f"{100 * row_rates['peak_teraops_per_second'] / peak_value:7.1f} "
                  f"{info.get('registers_per_thread')!s:>5}", flush=True)
            del a, b, c
    emit_tensor_results(metadata, args, rows)


def accumulation_policy(dtype: str) -> str:
    return {"fp8": "FP8 E4M3 products with FP32 accumulation",
            "fp4": "MX E2M1 multiply with E8M0 group scaling and FP32 accumulation",
            "fp32": "IEEE FP32 multiply and accumulation",
            "int8": "exact INT32 accumulation (no overflow)",
            "fp64": "FP64 multiply and accumulation"}.get(dtype, "FP32 tensor accumulation")


def emit_tensor_results(metadata: dict, args, rows: list[dict]) -> None:
    """Invocation status from the rows (bench_tensor.py:145-157)."""
    successful = [row for row in rows if row.get("status") == "ok"]
    if successful:
        best = max(successful, key=lambda row: row["peak_teraops_per_second"])
        unit = "TOPS" if args.dtype == "int8" else "TFLOP/s"
        frac = best["peak_teraops_per_second"] / roofline.PEAKS[f"tensor_{args.dtype}"][0]
        print(f"Measured {args.mode} {args.dtype}: {best['peak_teraops_per_second']:.2f} {unit} "
              f"({100 * frac:.1f}% of the MI355X dense peak; median {best['median_teraops_per_second']:.2f})")
        baseline = None
        if not getattr(args, "no_cpu_baseline", False):
            # The reference's host path for this row: torch.matmul in float32 (float64 for FP64).
            baseline = cpu_baseline.matmul_baseline(args.dtype, 256 if args.quick else 2048)
            print(f"CPU baseline (host, {baseline['cores']} threads): {baseline['value']:.4g} {baseline['unit']} "
                  f"({baseline['method']}, {baseline['sample']})")
        emit_results("tensor", metadata, args, rows, cpu_baseline=baseline)
        return
    if any(row.get("status") == "unsupported" for row in rows):
        reason = "; ".join(dict.fromkeys(row.get("reason", "unsupported") for row in rows))
        emit_unsupported("tensor", metadata, args, reason, details=rows)
        return
    raise RuntimeError("; ".join(dict.fromkeys(row.get("reason", "No usable configuration") for row in rows))
                       or "No usable configuration")


def build_parser():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--mode", choices=("peak", "gemm"), default="peak",
                        help="resident matrix-compute peak (default), or dense GEMM")
    parser.add_argument("--iterations", type=int, default=1024,
                        help="resident MFMA repeats, 1..262144; FP8/FP4 maximum 4096 (default: 1024)")
    parser.add_argument("--blocks-per-sm", nargs="+", type=int, default=[1, 2, 4, 8],
                        help="launched workgroups per CU (default: 1 2 4 8)")
    parser.add_argument("--sizes", nargs="+", type=int, default=None,
                        help="square GEMM dimensions M=N=K (default: the headline size of the format)")
    parser.add_argument("--dtype", choices=DTYPES, default="fp16",
                        help="matrix input format; TF32 uses FP32 storage; FP8 is E4M3FN and FP4 is OCP MX E2M1")
    parser.add_argument("--input-precision", choices=("ieee", "tf32"),
                        help="math mode for --dtype fp32 (default: ieee); TF32 has no gfx950 instruction")
    parser.add_argument("--b-layout", choices=("kn", "nk", "both"), default="kn",
                        help="peak B tile layout: [K][N] (reference default), [N][K], or both")
    parser.add_argument("--tiles", nargs="+", help="restrict peak tiles, e.g. 128x128x64")
    parser.add_argument("--inputs", choices=("baseline", "reference"), default="baseline",
                        help="GEMM operands: the benchmark configuration's sets (default), or the reference's own "
                             "recipe (N(0,1) A, N(0,1)/sqrt(K) B, INT8 {-1,0,1}; sizes 2048 4096 8192)")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--quick", action="store_true",
                        help="smoke test: one tile and 64 repeats, or GEMM dimensions 256/544")
    add_common_arguments(parser)
    return parser


def normalize_precision_args(parser, args) -> None:
    """FP32 dot policy (bench_tensor.py:358-368)."""
    args.requested_dtype = args.dtype
    if args.dtype == "tf32":
        if args.input_precision not in (None, "tf32"):
            parser.error("--dtype tf32 cannot use --input-precision ieee")
        args.dtype, args.input_precision = "fp32", "tf32"
    elif args.dtype == "fp32":
        args.input_precision = args.input_precision or "ieee"
    elif args.input_precision is not None:
        parser.error("--input-precision is only valid with --dtype fp32")


def capability_reason(args) -> str | None:
    if args.dtype == "fp32" and args.input_precision == "tf32":
        return TF32_REASON
    return None


def main(argv=None) -> None:
    parser = build_parser()
    args = parser.parse_args(argv)
    normalize_precision_args(parser, args)
    args.sizes_given = args.sizes is not None
    args.sizes = args.sizes or [2048, 4096, 8192]
    if any(size <= 0 for size in args.sizes):
        parser.error("--sizes values must be positive")
    if not 1 <= args.iterations <= 262144:
        parser.error("--iterations must be between 1 and 262144 for exact FP32 validation")
    if any(value <= 0 for value in args.blocks_per_sm):
        parser.error("--blocks-per-sm values must be positive")
    if args.dtype in ("fp8", "fp4") and args.mode == "peak" and args.iterations > 4096:
        parser.error(f"{args.dtype.upper()} peak limits --iterations to 4096 for exact FP32 accumulation")
    if args.dtype == "int8" and args.mode == "gemm" and any(size >= 2**24 for size in args.sizes):
        parser.error("INT8 GEMM requires K < 2**24 for an exact FP32 reference")
    if args.quick:
        args.sizes = [256, 544]
    metadata = setup_device(args)
    metadata.update(precision_descriptor(args.dtype, args.input_precision))
    reason = capability_reason(args)
    if reason is not None:
        emit_unsupported("tensor", metadata, args, reason)
        return
    device = get_device(args)
    _torch().manual_seed(0)
    try:
        if args.mode == "peak":
            configs = peak_configs(args.dtype, "both")
            if args.dtype == "fp32":
                metadata["tensor_precision_probe"] = validate_fp32_precision(device, configs)
            elif args.dtype == "fp64":
                metadata["tensor_precision_probe"] = validate_fp64_precision(device, configs)
            elif args.dtype == "fp8":
                metadata["tensor_storage_probe"] = validate_fp8_storage(device)
            elif args.dtype == "fp4":
                metadata["tensor_dot_lowering_probe"] = validate_fp4_arithmetic(device, configs)
    except TensorUnsupportedError as exc:
        emit_unsupported("tensor", metadata, args, str(exc))
        return
    if args.mode == "peak":
        run_peak(args, metadata, device)
        return
    from triton_chip_benchmarks_amd import gemm  # absolute: also valid when this file runs as a script

    gemm.run_gemm(args, metadata, device)


if __name__ == "__main__":
    main()
