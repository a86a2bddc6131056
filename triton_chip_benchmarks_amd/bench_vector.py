#!/usr/bin/env python3
"""Vector (VALU) arithmetic throughput on one MI355X; unsupported types reported explicitly.

Mirrors the reference's bench_vector.py CLI, inputs, validators and row fields
(bench_vector.py:182-1575). Eight independent chains per lane repeat a
multiply-add ITERATIONS times in registers (mb_vector_chains):
  fp32 v_fma_f32, fp64 v_fma_f64, fp16 v_pk_fma_f16 (two chains per VGPR),
  bf16 v_dot2_f32_bf16 + v_cvt_pk_bf16_f32 (bf16 products, fp32 sum, bf16
  state; the promoted v_fma_f32 form is measured beside it), int8 the DP4A
  feedback recurrence on v_dot4_i32_i8. gfx950 has no FP8 or FP4 VALU
  arithmetic, so those rows keep the reference's not_implemented / unsupported
  statuses, with the assembler's verdicts as evidence.
"""

from __future__ import annotations

import argparse
import math
from pathlib import Path
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd import _native, audit, cpu_baseline, formats, roofline
    from triton_chip_benchmarks_amd.common import (add_common_arguments, available_memory_bytes,
                                                   emit_not_implemented, emit_results, emit_unsupported,
                                                   get_device, measure, positive_int, setup_device)
else:
    from . import _native, audit, cpu_baseline, formats, roofline
    from .common import (add_common_arguments, available_memory_bytes, emit_not_implemented, emit_results,
                         emit_unsupported, get_device, measure, positive_int, setup_device)

CHAINS = 8
DEFAULT_ITERATIONS = 4096
DTYPES = ("bf16", "fp16", "fp32", "int8", "fp64", "fp8", "fp4")
KINDS = {"fp32": 0, "fp16": 1, "bf16_dot2": 2, "fp64": 3, "int8": 4, "bf16_fma": 5, "fp8": 6, "fp4": 7,
         "fp8_widened": 8, "fp4_widened": 9}
# (kernel kind, source operation, result-name suffix) per dtype, best-first.
VARIANTS = {"fp32": [("fp32", "FMA", "fma")], "fp64": [("fp64", "FMA", "fma")], "fp16": [("fp16", "FMA", "fma")],
            "bf16": [("bf16_dot2", "DOT2_BF16", "dot2"), ("bf16_fma", "WIDENED_FMA", "widened_fma")],
            "int8": [("int8", "DP4A", "dot4")]}

FP8_VECTOR_REJECTION = (
    "This benchmark has no implemented and verified native FP8 vector arithmetic path: gfx950's VALU has "
    "FP8 conversions (v_cvt_*fp8*) but no FP8 multiply or FMA, and FP8 matrix instructions are the "
    "tensor_fp8 metric. This does not determine chip support")
FP4_VECTOR_REJECTION = (
    "FP4 (E2M1) is not a VALU arithmetic type on gfx950: the ISA offers FP4 only as MFMA operands "
    "(v_mfma_scale_*_f8f6f4) and conversions (v_cvt_scalef32_*fp4*), and PyTorch's float4_e2m1fn_x2 is a "
    "two-element container rather than a scalar type. Where the chip executes FP4 natively, on its matrix "
    "cores, that rate is the tensor_fp4 metric")
# Mnemonics whose absence (and presence) the assembler reports for gfx950.
NARROW_FLOAT_PROBES = {"absent": ["v_dot4_f32_fp8_fp8 v0, v1, v2, v3", "v_pk_fma_bf16 v0, v1, v2, v3",
                                  "v_dot2_f16_f16 v0, v1, v2, v3"],
                       "present": ["v_cvt_pk_f32_fp8 v[0:1], v1", "v_cvt_scalef32_pk_f32_fp4 v[0:1], v1, v2",
                                   "v_dot2_f32_bf16 v0, v1, v2, v3", "v_dot4_i32_i8 v0, v1, v2, v3"]}


class UnsupportedVectorDtype(RuntimeError):
    """The requested arithmetic cannot be provided on this device."""


class NotImplementedVectorDtype(RuntimeError):
    """This benchmark lacks a native path for the requested arithmetic."""


def _torch():
    import torch

    return torch


def storage_dtype(kind: str):
    torch = _torch()
    return {"fp32": torch.float32, "fp64": torch.float64, "fp16": torch.float16, "bf16_dot2": torch.bfloat16,
            "bf16_fma": torch.bfloat16, "int8": torch.int32, "fp8_widened": torch.uint8,
            "fp4_widened": torch.uint8}[kind]


def isa_probe() -> dict:
    """Which narrow-format instructions the gfx950 assembler accepts (checked, not assumed)."""
    import shutil
    import subprocess

    assembler = shutil.which("llvm-mc") or "/opt/rocm/llvm/bin/llvm-mc"
    verdicts = {}
    for expected, lines in NARROW_FLOAT_PROBES.items():
        for line in lines:
            try:
                completed = subprocess.run([assembler, "-arch=amdgcn", "-mcpu=gfx950"], input=line, text=True,
                                           capture_output=True, timeout=30)
                accepted = completed.returncode == 0 and "error" not in completed.stderr
            except (OSError, subprocess.SubprocessError):
                accepted = None
            verdicts[line.split()[0]] = accepted
    return {"assembler": assembler, "mcpu": "gfx950", "accepted": verdicts}


def unsupported_dtype_reason(dtype: str) -> str | None:
    return FP4_VECTOR_REJECTION if dtype == "fp4" else None


def not_implemented_dtype_reason(dtype: str) -> str | None:
    return FP8_VECTOR_REJECTION if dtype == "fp8" else None


def throughput_fields(dtype: str, elements: int, iterations: int, timing: dict) -> dict:
    """Counted operations and rates (bench_vector.py:1271-1280): 8 per DP4A update, else 2."""
    per_update = 8 if dtype == "int8" else 2
    operations = per_update * CHAINS * elements * iterations
    median = operations / (timing["median_ms"] * 1e9)
    peak = operations / (timing["min_ms"] * 1e9)
    if dtype == "int8":
        return {"counted_integer_ops": operations, "tops": median, "peak_tops": peak,
                "throughput_unit": "TOPS", "ops_per_accumulator_update": per_update}
    return {"counted_flops": operations, "tflops": median, "peak_tflops": peak,
            "throughput_unit": "TFLOP/s", "ops_per_accumulator_update": 2}


def _pack_bytes(values) -> int:
    packed = sum((int(v) & 255) << shift for v, shift in zip(values, (0, 8, 16, 24)))
    return packed - 2**32 if packed >= 2**31 else packed


def make_inputs(dtype: str, elements: int, device, inputs_kind: str = "reference", seed: int = 0):
    """Inputs [8, elements] and coefficients [9] in the kernel's storage type.

    reference: the reference's operands (bench_vector.py:1191-1216) - fp32/fp64
      x0 ~ U[0.125, 1), a = 1 - 2^-14, b_c = (c+1) 2^-16; fp16/bf16 the exact
      involution x0 in {1..7}/8, a = -1, b_c = (c+1)/8; int8 random int32 words,
      W = bytes (3, -2, 1, -1), b_c = c + 1.
    baseline: the headline vector workload - x0 ~ U[0.5, 1), a = 0.999,
      b = 1e-3; int8 x0 in [-4, 4], W = bytes (1, 1, 1, 1), b = 1.
    """
    torch = _torch()
    generator = torch.Generator().manual_seed(seed)
    store = storage_dtype({"bf16": "bf16_dot2"}.get(dtype, dtype))
    if dtype == "int8":
        if inputs_kind == "baseline":
            inputs = torch.randint(-4, 5, (CHAINS, elements), generator=generator, dtype=torch.int32)
            coefficients = torch.tensor([_pack_bytes((1, 1, 1, 1))] + [1] * CHAINS, dtype=torch.int32)
        else:
            inputs = torch.randint(-(2**31), 2**31, (CHAINS, elements), generator=generator, dtype=torch.int64)
            inputs = inputs.to(torch.int32)
            coefficients = torch.tensor([_pack_bytes((3, -2, 1, -1))] + list(range(1, CHAINS + 1)),
                                        dtype=torch.int32)
    elif inputs_kind == "baseline":
        inputs = torch.empty((CHAINS, elements), dtype=torch.float64).uniform_(0.5, 1.0, generator=generator)
        inputs = inputs.to(store)
        coefficients = torch.tensor([0.999] + [1e-3] * CHAINS, dtype=torch.float64).to(store)
    elif dtype in ("fp16", "bf16"):
        inputs = (torch.randint(1, 8, (CHAINS, elements), generator=generator).double() / 8).to(store)
        coefficients = torch.tensor([-1.0] + [(i + 1) / 8 for i in range(CHAINS)], dtype=torch.float64).to(store)
    else:
        inputs = torch.empty((CHAINS, elements), dtype=torch.float64).uniform_(0.125, 1.0, generator=generator)
        inputs = inputs.to(store)
        coefficients = torch.tensor([1.0 - 2.0**-14] + [(c + 1) * 2.0**-16 for c in range(CHAINS)],
                                    dtype=torch.float64).to(store)
    return inputs.to(device), coefficients.to(device)


def dot2_regime_reason(inputs, coefficients, iterations: int) -> str | None:
    """Why the BF16 dot2 chains may not run these operands, or None.

    Each v_dot2_f32_bf16 computes a*x_c + 0*x_sibling + b_c, so a sibling
    chain that reached Inf or NaN would turn 0*x_sibling into NaN and poison a
    finite chain. That cannot happen when every state starts finite and
    |a| <= 1: each state then stays within |x0| + iterations * max|b| of zero.
    Other operands must use the bf16_fma variant.
    """
    torch = _torch()
    a, b = coefficients[0].float(), coefficients[1:].float()
    if not bool(torch.isfinite(inputs.float()).all()) or not bool(torch.isfinite(coefficients.float()).all()):
        return "non-finite states or coefficients"
    if abs(a.item()) > 1.0:
        return f"|a| = {abs(a.item()):g} > 1 lets a chain grow without bound"
    bound = inputs.float().abs().max().item() + iterations * b.abs().max().item()
    if bound > 1e38:
        return f"states may reach {bound:.3g}, past the bfloat16 range"
    return None


def require_dot2_regime(inputs, coefficients, iterations: int) -> None:
    """Raises unless the BF16 dot2 chains may run these operands for this many iterations."""
    reason = dot2_regime_reason(inputs, coefficients, iterations)
    if reason:
        raise ValueError(f"BF16 dot2 chains need bounded operands ({reason}); use the bf16_fma variant")


def launch_vector(kind: str, inputs, output, coefficients, iterations: int, unroll: int, block_threads: int,
                  regime_checked: bool = False):
    """One launch of the chain kernel on the current stream.

    The dot2 variant's operand check reads the operands back to the host, so
    a caller that times launches (or captures them in a graph) runs
    require_dot2_regime once, for at least this many iterations, and passes
    regime_checked=True.
    """
    if kind == "bf16_dot2" and not regime_checked:
        require_dot2_regime(inputs, coefficients, iterations)
    elements = inputs.shape[1]
    size = inputs.numel() * inputs.element_size()
    _native.call("mb_vector_chains", KINDS[kind], inputs.data_ptr(), output.data_ptr(), coefficients.data_ptr(),
                 elements, iterations, unroll, block_threads, size, output.numel() * output.element_size(),
                 coefficients.numel() * coefficients.element_size(), _native.stream_handle())


def check_output(inputs, output, coefficients, iterations: int, explicit_fma: bool = True) -> dict:
    """Closed-form check of every output (bench_vector.py:322-372), in float64 on the device.

    a == -1: the exact two-cycle, zero tolerance. Otherwise the contractive
    affine recurrence with the accumulated unit-roundoff bound.
    """
    torch = _torch()
    coefficients = coefficients.double().cpu()
    a = coefficients[0].item()
    exact_cycle = a == -1.0
    if not exact_cycle and not 0.0 < a < 1.0:
        raise ValueError("the closed-form check needs a == -1 or 0 < a < 1")
    decay = None if exact_cycle else math.exp(iterations * math.log(a))
    geometric = None if exact_cycle else -math.expm1(iterations * math.log(a)) / (1.0 - a)
    b = coefficients[1:, None].to(output.device)
    max_error = max_tolerance = 0.0
    for start in range(0, output.shape[1], 1 << 20):
        initial = inputs[:, start:start + (1 << 20)].double()
        actual = output[:, start:start + (1 << 20)].double()
        if exact_cycle:
            reference = b - initial if iterations % 2 else initial
            tolerance = torch.zeros_like(reference)
        else:
            reference = decay * initial + b * geometric
            magnitude = torch.maximum(initial.abs(), (b / (1.0 - a)).abs())
            unit = 2.0 ** (-53 if inputs.dtype == torch.float64 else -24)
            tolerance = (2.0 if explicit_fma else 4.0) * unit * magnitude * geometric + 16 * unit
        error = (actual - reference).abs()
        if not torch.all(error <= tolerance).item():
            raise RuntimeError("Vector correctness failed: non-finite or inaccurate output; "
                               f"max_abs_error={error.max().item():.6g}, max_tolerance={tolerance.max().item():.6g}")
        max_error = max(max_error, error.max().item())
        max_tolerance = max(max_tolerance, tolerance.max().item())
    return {"correctness": "all elements passed analytic FP64 reference and finite check",
            "max_abs_error": max_error, "max_abs_tolerance": max_tolerance,
            "reference_device": str(output.device),
            "validation_recurrence": "exact involution" if exact_cycle else "contractive affine"}


def _signed_bytes(word: int) -> list[int]:
    return [((int(word) >> s) & 255) - (256 if ((int(word) >> s) & 255) >= 128 else 0) for s in (0, 8, 16, 24)]


def _dot4(words, weights):
    torch = _torch()
    result = torch.zeros_like(words, dtype=torch.int64)
    for shift, weight in zip((0, 8, 16, 24), weights):
        lane = (words >> shift) & 255
        result += torch.where(lane >= 128, lane - 256, lane) * weight
    return result


def check_int8_output(inputs, output, coefficients, iterations: int) -> dict:
    """Exact DP4A check with a composed state-transition table (bench_vector.py:390-421)."""
    torch = _torch()
    coefficients = coefficients.cpu().long()
    weights = _signed_bytes(coefficients[0].item())
    bias = coefficients[1:, None]
    bound = 128 * sum(abs(w) for w in weights) + int(bias.abs().max())
    states = torch.arange(-bound, bound + 1).expand(CHAINS, -1)
    power = _dot4(states, weights) + bias + bound
    composed = torch.arange(2 * bound + 1).expand(CHAINS, -1)
    remaining = iterations - 1
    while remaining:
        if remaining & 1:
            composed = power.gather(1, composed)
        remaining >>= 1
        if remaining:
            power = power.gather(1, power)
    for start in range(0, inputs.shape[1], 1 << 18):
        initial = inputs[:, start:start + (1 << 18)].cpu().long()
        reference = composed.gather(1, _dot4(initial, weights) + bias + bound) - bound
        if not torch.equal(output[:, start:start + (1 << 18)].cpu().long(), reference):
            raise RuntimeError("Vector INT8 correctness failed: output differs from exact signed INT8 dot4 / "
                               "INT32 state reference")
    return {"correctness": "all elements passed exact INT64 reference", "max_abs_error": 0,
            "max_abs_tolerance": 0, "reference_device": "cpu",
            "validation_recurrence": "signed INT8 dot4 with INT32 bias/state"}


def check_narrow_steps(inputs, output, coefficients, iterations: int, dtype: str, lanes: int = 4096) -> dict:
    """Step-by-step recompute of sampled lanes for fp16/bf16 states, bit for bit.

    Each update is evaluated in float64 (exact for the suite's operand sets)
    and rounded to the state format - through fp32 first for bf16, as the
    kernels' fp32 result is rounded to bf16.
    """
    torch = _torch()
    count = min(lanes, inputs.shape[1])
    index = torch.linspace(0, inputs.shape[1] - 1, count).long()
    state = inputs[:, index].cpu()
    a = coefficients[0].double().cpu()
    b = coefficients[1:, None].double().cpu()
    for _ in range(iterations):
        exact = state.double() * a + b
        state = (exact.float() if dtype == "bf16" else exact).to(inputs.dtype)
    expected = state.view(torch.int16) if dtype in ("fp16", "bf16") else state
    actual = output[:, index].cpu()
    if not torch.equal(actual.view(torch.int16), expected):
        raise RuntimeError(f"Vector {dtype.upper()} correctness failed: sampled lanes differ from the "
                           "step-by-step recompute")
    return {"step_recompute": f"{count} sampled lanes x 8 chains bit-exact over {iterations} updates"}


def configure_sweep(args):
    if args.quick:
        args.iterations, args.blocks_per_sm, args.block_sizes, args.unroll = 32, [1], [256], [1]
    else:
        args.blocks_per_sm = args.blocks_per_sm or [8, 16]
        args.block_sizes = args.block_sizes or [256, 512, 1024]
        args.unroll = args.unroll or [1, 4, 8, 16]


def build_parser():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    add_common_arguments(parser)
    parser.add_argument("--dtype", choices=DTYPES, default="fp32",
                        help="Arithmetic type (default: fp32); unsupported types emit a status JSON")
    parser.add_argument("--iterations", type=positive_int, default=DEFAULT_ITERATIONS,
                        help=f"Multiply-add iterations per accumulator (default: {DEFAULT_ITERATIONS})")
    parser.add_argument("--blocks-per-sm", type=positive_int, nargs="+",
                        help="Workgroups per compute unit (default: 8 16)")
    parser.add_argument("--block-sizes", type=positive_int, nargs="+",
                        help="Lanes (elements) per workgroup: 64..1024, a multiple of 64 (default: 256 512 1024)")
    parser.add_argument("--unroll", type=int, choices=[1, 4, 8, 16], nargs="+",
                        help="Updates per loop trip (default: 1 4 8 16)")
    parser.add_argument("--inputs", choices=("reference", "baseline"), default="reference",
                        help="Operand set: the reference's (default) or the headline a=0.999, c=1e-3 workload")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--widened", action="store_true",
                        help="FP8/FP4: also measure converted chains (narrow state, FP32 FMA per update); the "
                             "row keeps its not_implemented/unsupported status and the rate goes to details")
    parser.add_argument("--quick", action="store_true", help="One smoke configuration; not a peak result")
    return parser


def validate(dtype, kind, inputs, output, coefficients, iterations, inputs_kind, run) -> dict:
    torch = _torch()
    if dtype == "int8":
        return check_int8_output(inputs, output, coefficients, iterations)
    if dtype in ("fp16", "bf16"):
        if inputs_kind == "baseline":
            return {"correctness": "sampled lanes bit-exact against a step-by-step recompute",
                    **check_narrow_steps(inputs, output, coefficients, iterations, dtype)}
        correctness = check_output(inputs, output, coefficients, iterations, True)
        correctness.update(check_narrow_steps(inputs, output, coefficients, iterations, dtype, lanes=1024))
        if iterations % 2 == 0:  # the two-cycle returns to x0 on even counts: re-run an odd count
            output.fill_(float("nan"))
            run(iterations + 1, 1)
            torch.cuda.synchronize()
            check_output(inputs, output, coefficients, iterations + 1, True)
            correctness["odd_iteration_probe"] = "all elements passed"
        return correctness
    return check_output(inputs, output, coefficients, iterations, True)


def run_benchmark(args, metadata):
    torch = _torch()
    device = get_device(args)
    dtype = args.dtype
    if not metadata.get("sm_count"):
        raise SystemExit("The runtime did not expose the compute-unit count; supply --compute-units")
    unit = "TOPS" if dtype == "int8" else "TFLOP/s"
    peak_key, median_key = ("peak_tops", "tops") if dtype == "int8" else ("peak_tflops", "tflops")
    peak_value = roofline.PEAKS[f"vector_{dtype}"][0]
    print(f"{dtype.upper()} vector: {CHAINS} independent chains, {args.iterations} iterations, "
          f"{args.inputs} operands; {8 if dtype == 'int8' else 2} operations per update")
    print("variant       blocks/CU  block  unroll  regs  median_ms   median      peak   % peak")
    rows, excluded = [], []
    for blocks_per_sm in args.blocks_per_sm:
        for block in args.block_sizes:
            if block % 64 or block > 1024:
                excluded.append({"status": "invalid", "reason": "block size must be a multiple of 64 up to 1024",
                                 "block_size": block})
                continue
            elements = blocks_per_sm * metadata["sm_count"] * block
            for kind, operation, suffix in VARIANTS[dtype]:
                store = storage_dtype(kind)
                required = 2 * CHAINS * elements * torch.empty((), dtype=store).element_size()
                free = available_memory_bytes()
                if free is not None and required > 0.5 * free:
                    raise SystemExit(f"Vector input/output need {required / 2**30:.2f} GiB; reduce the sweep")
                inputs, coefficients = make_inputs(dtype, elements, device, args.inputs, args.seed)
                output = torch.empty_like(inputs)
                if kind == "bf16_dot2":  # once per operand set, outside every timed launch
                    reason = dot2_regime_reason(inputs, coefficients, args.iterations + 1)
                    if reason:
                        excluded.append({"status": "unsupported", "reason": f"dot2 operand regime: {reason}",
                                         "variant": suffix})
                        continue
                for unroll in args.unroll:
                    if args.iterations % unroll:
                        continue
                    kernel = _native.load().mb_vector_kernel_name(KINDS[kind], unroll).decode()
                    output.fill_(-(2**31) if dtype == "int8" else float("nan"))

                    def run(iterations=args.iterations, unroll_value=unroll, kind=kind, inputs=inputs,
                            output=output, coefficients=coefficients, block=block):
                        launch_vector(kind, inputs, output, coefficients, iterations, unroll_value, block,
                                      regime_checked=True)

                    run()
                    torch.cuda.synchronize()
                    try:
                        assembly = audit.audit_vector(audit.instructions(kernel), dtype,
                                                      "fma" if kind == "bf16_fma" else "native")
                    except audit.VectorAuditError as exc:
                        excluded.append({"status": "unsupported", "reason": str(exc), "kernel": kernel})
                        continue
                    resources = audit.resources(kernel)
                    if resources.get("register_spills"):
                        excluded.append({"status": "register_spills", "kernel": kernel,
                                         "reason": f"spills={resources['register_spills']}"})
                        continue
                    correctness = validate(dtype, kind, inputs, output, coefficients, args.iterations,
                                           args.inputs, run)
                    timing = measure(run, args)
                    rates = throughput_fields(dtype, elements, args.iterations, timing)
                    native = assembly["native_arithmetic_verified"]
                    arithmetic = ("int8 products with int32 sum" if dtype == "int8" else
                                  "bf16 products with fp32 sum, bf16 state" if kind == "bf16_dot2" else
                                  "fp32 FMA rounded to bf16 state (promoted)" if kind == "bf16_fma" else dtype)
                    row = {"status": "ok", "requested_dtype": dtype, "dtype": str(inputs.dtype).removeprefix("torch."),
                           "input_storage_dtype": "int8 packed in int32" if dtype == "int8" else dtype,
                           "accumulator_dtype": "int32" if dtype == "int8" else dtype,
                           "source_arithmetic_dtype": dtype, "arithmetic_dtype": arithmetic,
                           "includes_unpacking": False, "operation": operation, "variant": suffix,
                           "loop_structure": "strip_mined", "coefficient_load": "scalar",
                           "hardware_fusion_verified": bool(native and dtype != "int8"),
                           "roundings_per_update": 1 if dtype in ("fp32", "fp64", "fp16") else (
                               0 if dtype == "int8" else 2),
                           "accumulator_chains": CHAINS, "iterations": args.iterations,
                           "blocks_per_sm": blocks_per_sm, "blocks": blocks_per_sm * metadata["sm_count"],
                           "block_size": block, "num_warps": block // 64, "unroll": unroll,
                           "elements_per_chain": elements, "inputs": args.inputs, "kernel": kernel,
                           "smoke_only": args.quick, **rates, **timing, **correctness, **assembly,
                           "registers_per_thread": resources["registers_per_thread"],
                           "register_spills": resources["register_spills"],
                           "roofline": roofline.describe(f"vector_{dtype}", rates[peak_key])}
                    rows.append(row)
                    print(f"{suffix:12s} {blocks_per_sm:10d} {block:6d} {unroll:7d} "
                          f"{resources['registers_per_thread']!s:>5} {timing['median_ms']:10.5f} "
                          f"{rates[median_key]:8.3f} {rates[peak_key]:9.3f} {100 * rates[peak_key] / peak_value:8.1f}",
                          flush=True)
                del inputs, output, coefficients
    if not rows:
        reasons = "; ".join(dict.fromkeys(item["reason"] for item in excluded))
        if excluded and all(item["status"] == "unsupported" for item in excluded):
            raise UnsupportedVectorDtype(f"No configuration provides {dtype.upper()} arithmetic: {reasons}")
        raise RuntimeError(f"No vector configuration produced a valid measurement: {reasons}")
    best = max(rows, key=lambda row: row[peak_key])
    print(f"Peak measured {dtype.upper()} vector throughput: {best[peak_key]:.3f} {unit} "
          f"({100 * best[peak_key] / peak_value:.1f}% of {peak_value:.1f}; variant {best['variant']}, "
          f"blocks/CU={best['blocks_per_sm']}, block={best['block_size']}, unroll={best['unroll']})")
    name = f"vector_{dtype}_{best['variant']}"
    baseline = None
    if not args.no_cpu_baseline:
        # The reference's host path for this row: the recurrence vectorised over the lane set.
        baseline = cpu_baseline.vector_baseline(dtype, 2**16 if args.quick else 2**22, 2 if args.quick else 8)
        print(f"CPU baseline (host, {baseline['cores']} threads): {baseline['value']:.4g} {baseline['unit']} "
              f"({baseline['sample']})")
    emit_results(name, {**metadata, "vector_excluded_configurations": excluded}, args, rows, cpu_baseline=baseline)


# ---- widened (converted) FP8 / FP4 chains ----------------------------------------
# Not native arithmetic: gfx950's VALU has FP8/FP4 conversions but no FP8/FP4
# math. The state stays in the narrow format and each update is
# x <- narrow(fma(f32(x), a, b_c)), the reference's Ascend C "converted" rows
# (ascendc/src/bench_vector.asc:335-572): only the FMA's 2 operations count.
WIDENED_KIND = {"fp8": "fp8_widened", "fp4": "fp4_widened"}
WIDENED_ARITHMETIC = {"fp8": "converted_fp32_fma_fp8_e4m3_state", "fp4": "converted_fp32_fma_fp4_e2m1_state"}


def widened_inputs(dtype: str, elements: int, device, seed: int = 0):
    """Codes for the exact involution the Ascend C suite validates (a = -1): x0
    and b_c on the format's lattice so that b_c - x0 is exact
    (ascendc/src/bench_vector.asc:912-950)."""
    torch = _torch()
    generator = torch.Generator().manual_seed(seed)
    if dtype == "fp8":
        x = torch.randint(1, 8, (CHAINS, elements), generator=generator).double() / 8
        b = torch.arange(1, CHAINS + 1).double() / 8
        encode = lambda v: v.float().to(torch.float8_e4m3fn).view(torch.uint8)
    else:
        x = (torch.randint(0, 5, (CHAINS, elements), generator=generator).double() - 2) * 0.5
        b = (torch.arange(CHAINS).double() % 3 - 1) * 0.5
        encode = formats.e2m1_encode
    coefficients = torch.cat([torch.tensor([-1.0], dtype=torch.float64), b])
    return encode(x).to(device), encode(coefficients).to(device)


def widened_values(dtype: str, codes):
    torch = _torch()
    return codes.view(torch.float8_e4m3fn).double() if dtype == "fp8" else formats.e2m1_decode(codes)


def check_widened(dtype: str, inputs, output, coefficients, iterations: int) -> dict:
    """a = -1 returns x0 after an even count and b_c - x0 after an odd one, exactly."""
    torch = _torch()
    x0 = widened_values(dtype, inputs)
    b = widened_values(dtype, coefficients)[1:, None]
    expected = x0 if iterations % 2 == 0 else b - x0
    got = widened_values(dtype, output)
    if not torch.equal(got, expected):
        raise AssertionError(f"widened {dtype} chains differ from the exact involution")
    return {"correctness": "exact involution (a = -1): every element equals x0 or b - x0", "max_abs_error": 0.0}


def run_widened(args, metadata) -> dict:
    """Sweep the converted kernel; returns the details block for the status document."""
    torch = _torch()
    device = get_device(args)
    dtype, kind = args.dtype, WIDENED_KIND[args.dtype]
    fp32_issue = roofline.ISSUED_CEILINGS["vector_fp32"][0]  # one v_fma_f32 per update
    print(f"{dtype.upper()} widened vector chains (not native arithmetic): {CHAINS} chains, {args.iterations} "
          "iterations, narrow state, FP32 FMA per update")
    rows = []
    for blocks_per_sm in args.blocks_per_sm:
        for block in args.block_sizes:
            if block % 64 or block > 1024:
                continue
            elements = blocks_per_sm * metadata["sm_count"] * block
            inputs, coefficients = widened_inputs(dtype, elements, device, args.seed)
            output = torch.empty_like(inputs)
            for unroll in args.unroll:
                if args.iterations % unroll:
                    continue
                kernel = _native.load().mb_vector_kernel_name(KINDS[kind], unroll).decode()
                assembly = audit.audit_widened(audit.instructions(kernel), dtype)
                output.fill_(255)

                def run(iterations=args.iterations, unroll_value=unroll, inputs=inputs, output=output,
                        coefficients=coefficients, block=block):
                    launch_vector(kind, inputs, output, coefficients, iterations, unroll_value, block)

                run()
                torch.cuda.synchronize()
                correctness = check_widened(dtype, inputs, output, coefficients, args.iterations)
                timing = measure(run, args)
                rates = throughput_fields(dtype, elements, args.iterations, timing)
                rows.append({"status": "ok", "requested_dtype": dtype, "operation": "WIDENED_FMA",
                             "arithmetic_kind": WIDENED_ARITHMETIC[dtype], "arithmetic_dtype": "fp32",
                             "input_storage_dtype": "fp8_e4m3fn" if dtype == "fp8" else "fp4_e2m1",
                             "native_arithmetic_verified": False, "conversions_per_update": 1,
                             "blocks_per_sm": blocks_per_sm, "block_size": block, "unroll": unroll,
                             "elements_per_chain": elements, "kernel": kernel, **rates, **timing,
                             **correctness, **assembly,
                             "fraction_of_fp32_fma_issue_ceiling": rates["peak_tflops"] / fp32_issue})
                print(f"widened {blocks_per_sm:4d} {block:6d} {unroll:4d} {timing['median_ms']:10.5f} "
                      f"{rates['tflops']:8.3f} {rates['peak_tflops']:8.3f}", flush=True)
            del inputs, output, coefficients
    if not rows:
        raise RuntimeError("No widened configuration produced a valid measurement")
    best = max(rows, key=lambda row: row["peak_tflops"])
    print(f"Widened {dtype.upper()} chains: {best['peak_tflops']:.3f} TFLOP/s (not a native {dtype.upper()} rate)")
    return {"widened": {key: best[key] for key in ("kernel", "peak_tflops", "tflops", "arithmetic_kind",
                                                   "blocks_per_sm", "block_size", "unroll", "correctness")},
            "widened_rows": [{k: v for k, v in row.items() if k not in ("samples_ms_per_launch", "batch_samples_ms")}
                             for row in rows]}


def main(argv=None):
    parser = build_parser()
    args = parser.parse_args(argv)
    if args.iterations >= 2**31:
        parser.error("--iterations must be less than 2**31")
    if args.unroll is not None and any(args.iterations % unroll for unroll in args.unroll):
        parser.error("--iterations must be divisible by every --unroll factor")
    metadata = setup_device(args)
    configure_sweep(args)
    if any(args.iterations % unroll for unroll in args.unroll):
        parser.error("--iterations must be divisible by every --unroll factor")
    details = run_widened(args, metadata) if args.widened and args.dtype in WIDENED_KIND else None
    reason = unsupported_dtype_reason(args.dtype)
    if reason:
        metadata["vector_fp4_capability_probe"] = isa_probe()
        emit_unsupported(f"vector_{args.dtype}", metadata, args, reason, details=details)
        return
    reason = not_implemented_dtype_reason(args.dtype)
    if reason:
        metadata["vector_fp8_capability_probe"] = isa_probe()
        emit_not_implemented(f"vector_{args.dtype}", metadata, args, reason, details=details)
        return
    try:
        run_benchmark(args, metadata)
    except UnsupportedVectorDtype as exc:
        emit_unsupported(f"vector_{args.dtype}", metadata, args, str(exc))
    except NotImplementedVectorDtype as exc:
        emit_not_implemented(f"vector_{args.dtype}", metadata, args, str(exc))


if __name__ == "__main__":
    main()
