#!/usr/bin/env python3
"""Independent cross-implementation check on one MI355X: two paths, same silicon limit.

The tensor and memory rows come from this suite's own gfx950 kernels. Here the
same work runs a second way on the same card, with each output checked
against the other:
  copy   mb_copy (the suite's kernel)  vs  dst.copy_(src) (hipMemcpy device-to-device)
  GEMM   mb_gemm (the suite's kernel)  vs  torch.matmul / torch._scaled_mm / torch._int_mm (hipBLASLt)
The MXFP4 GEMM runs at BASELINE's 16384^3, FP64 at its 4096^3 and the others
at 8192^3. torch's
MXFP4 path writes a BF16 C only, so its output is checked elementwise against
the suite's exact FP32 C to within one BF16 unit in the last place.
This follows the reference's practice of comparing its Triton suite with an
independent Ascend C implementation on the same chip (ascendc/RESULTS.md:57-108):
a large gap points at a kernel, not at the silicon. Rates use the suite's
device-event timing (common.measure). The library paths are measurement
references only; nothing in the suite's rows is taken from them.
"""

from __future__ import annotations

import argparse
from pathlib import Path
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd import _native, bench_bandwidth, gemm, roofline
    from triton_chip_benchmarks_amd.common import add_common_arguments, emit_results, measure, setup_device
else:
    from . import _native, bench_bandwidth, gemm, roofline
    from .common import add_common_arguments, emit_results, measure, setup_device

COPY_SHAPE = {"block_threads": 64, "vectors_per_thread": 1, "policy": "stream"}
GEMM_SIZE = 8192
FP4_GEMM_SIZE = 16384
FP64_GEMM_SIZE = 4096


def _torch():
    import torch

    return torch


def copy_rows(args, sizes_mib):
    """mb_copy against hipMemcpy device-to-device on the same buffers."""
    torch = _torch()
    rows = []
    for size_mib in sizes_mib:
        n = size_mib * 2**20 // 4
        generator = torch.Generator(device="cuda").manual_seed(args.seed)
        src = torch.empty(n, device="cuda", dtype=torch.float32).uniform_(-1, 1, generator=generator)
        dst = torch.empty_like(src)
        paths = {
            "mb_copy": lambda: bench_bandwidth.launch_copy(src, dst, COPY_SHAPE["block_threads"],
                                                           COPY_SHAPE["vectors_per_thread"], 0,
                                                           COPY_SHAPE["policy"]),
            "hipMemcpyDtoD": lambda: dst.copy_(src),
        }
        for name, run in paths.items():
            dst.fill_(float("nan"))
            run()
            torch.cuda.synchronize()
            if not torch.equal(src.view(torch.int32), dst.view(torch.int32)):
                raise AssertionError(f"{name}: copy of {size_mib} MiB differs from its source")
            timing = measure(run, args)
            traffic = 2 * n * 4
            peak = traffic / (timing["min_ms"] * 1e6)
            rows.append({"check": "copy", "path": name, "buffer_mib": size_mib, "traffic_bytes": traffic,
                         "peak_gbps": peak, "gbps": traffic / (timing["median_ms"] * 1e6),
                         "fraction_of_hbm_peak": peak / roofline.HBM_PEAK_GBPS,
                         "validation": "bit-exact against the source", **timing})
    return rows


def _library_gemm(dtype, a, b, torch):
    """The library path for C = A . B^T (B stored [N][K]), or None when torch has none."""
    if dtype in ("bf16", "fp16", "fp32", "fp64"):
        bt = b.t()
        return lambda: torch.matmul(a, bt)
    if dtype == "fp8" and hasattr(torch, "_scaled_mm"):
        one = torch.ones((), device=a.device, dtype=torch.float32)
        bt = b.t()
        return lambda: torch._scaled_mm(a, bt, scale_a=one, scale_b=one, out_dtype=torch.float32)
    if dtype == "int8" and hasattr(torch, "_int_mm"):
        bt = b.t()
        return lambda: torch._int_mm(a, bt)
    if dtype == "fp4" and hasattr(torch, "float4_e2m1fn_x2") and hasattr(torch, "float8_e8m0fnu"):
        # Packed E2M1 pairs, even K in the low nibble, with one E8M0 scale per 32 K elements. The suite's
        # operands carry unit scales (127) only, so the library's scale layout cannot change the product.
        m, n, k = a.shape[0], b.shape[0], 2 * a.shape[1]
        a4, bt4 = a.view(torch.float4_e2m1fn_x2), b.view(torch.float4_e2m1fn_x2).t()
        unit = torch.full((), 127, dtype=torch.uint8, device=a.device)
        scale_a = unit.expand(m, k // 32).contiguous().view(torch.float8_e8m0fnu)
        scale_b = unit.expand(n, k // 32).contiguous().view(torch.float8_e8m0fnu)
        return lambda: torch._scaled_mm(a4, bt4, scale_a=scale_a, scale_b=scale_b, out_dtype=torch.bfloat16)
    return None


# Normwise agreement bound between mb_gemm's C and the library's. For BF16/FP16 operands the library returns
# BF16/FP16 C, whose rounding alone (up to 2^-9 of an entry for BF16) exceeds the 2e-3 elementwise check of
# gemm.TOLERANCE, so the comparison allows the benchmark configuration's stated 1e-2 there; exact formats are
# compared entry by entry (below) or to 1e-6 normwise.
AGREEMENT = {"bf16": 1e-2, "fp16": 1e-2, "fp32": 2e-3, "fp64": 1e-12, "fp8": 1e-6, "int8": 1e-6, "fp4": 1e-6}


def _agreement(dtype, theirs, c, torch):
    """Normwise difference of the two outputs; for a BF16 library C of an exact format, the worst entry in ulps.

    The suite's C is exact for FP8/INT8/MXFP4 operands (gemm.TOLERANCE 0), so a BF16 library C must lie within
    one BF16 ulp of it, entry by entry: 2^(e-8) for an exact value m * 2^e with 0.5 <= |m| < 1 (8 significant
    bits). Zeros must match exactly. BF16/FP16 operands give rounded sums on both sides, which only the
    normwise difference compares.
    """
    ref, got = c.double(), theirs.double()
    scale = ref.abs().max().item() or 1.0
    fields = {"normwise_difference": (got - ref).abs().max().item() / scale}
    if gemm.TOLERANCE[dtype] == 0.0 and theirs.dtype == torch.bfloat16 and c.dtype == torch.float32:
        error = (got - ref).abs()
        _, exponent = torch.frexp(ref)
        ulp = torch.where(ref == 0, torch.zeros_like(ref), torch.ldexp(torch.ones_like(ref), exponent - 8))
        fields["library_output"] = "bf16"
        fields["max_bf16_ulps"] = (error / ulp.clamp_min(torch.finfo(torch.float64).tiny)).max().item()
        fields["elementwise_within_one_bf16_ulp"] = bool((error <= ulp).all().item())
    return fields


def gemm_rows(args, dtypes, base_size, fp4_size=FP4_GEMM_SIZE, fp64_size=FP64_GEMM_SIZE):
    """mb_gemm against the torch (hipBLASLt) GEMM on the same operands; outputs cross-checked."""
    torch = _torch()
    rows = []
    for dtype in dtypes:
        size = {"fp4": fp4_size, "fp64": fp64_size}.get(dtype, base_size)
        a, b, c, scales, a_values, b_values = gemm.gemm_inputs(dtype, size, size, size, "cuda", args.seed)
        del a_values, b_values
        config = max(_native.gemm_configs(dtype), key=lambda cfg: cfg["tile_m"] * cfg["tile_n"])
        ours = lambda: _native.gemm(dtype, config, a, b, c, size, size, size, *(scales or (None, None)))
        ours()
        torch.cuda.synchronize()
        peak_value = roofline.PEAKS[f"tensor_{dtype}"][0]
        library = None
        try:
            library = _library_gemm(dtype, a, b, torch)
            if library is not None:
                theirs = library()
                torch.cuda.synchronize()
        except RuntimeError as exc:  # the op exists but this build has no kernel for the dtype
            library, reason = None, f"torch library path unavailable: {exc}".splitlines()[0]
        else:
            reason = None if library is not None else "torch has no library GEMM for this format"
        agreement = {"normwise_difference": None}
        if library is not None:
            agreement = _agreement(dtype, theirs, c, torch)
            normwise = agreement["normwise_difference"]
            if "elementwise_within_one_bf16_ulp" in agreement:
                if not agreement["elementwise_within_one_bf16_ulp"]:
                    raise AssertionError(f"{dtype}: the library's BF16 C is {agreement['max_bf16_ulps']:.3g} BF16 "
                                         "ulps from mb_gemm's exact C (one allowed)")
            elif normwise > AGREEMENT[dtype]:
                raise AssertionError(f"{dtype}: mb_gemm and the library disagree (normwise {normwise:.3g})")
            del theirs
        for name, run in (("mb_gemm", ours), ("torch/hipBLASLt", library)):
            if run is None:
                rows.append({"check": "gemm", "path": name, "dtype": dtype, "m": size, "n": size, "k": size,
                             "status": "unavailable", "reason": reason})
                continue
            timing = measure(run, args)
            peak = 2 * size**3 / (timing["min_ms"] * 1e9)
            rows.append({"check": "gemm", "path": name, "dtype": dtype, "m": size, "n": size, "k": size,
                         "kernel": _native.gemm_kernel_name(dtype, config) if name == "mb_gemm" else "library",
                         "peak_teraops_per_second": peak,
                         "median_teraops_per_second": 2 * size**3 / (timing["median_ms"] * 1e9),
                         "fraction_of_peak": peak / peak_value, **agreement, **timing})
        del a, b, c, scales
        torch.cuda.empty_cache()
    return rows


def build_parser():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--copy-mib", type=int, nargs="+", default=[1024, 2048], help="copy buffer sizes (MiB)")
    parser.add_argument("--gemm-dtypes", nargs="+", default=["bf16", "fp16", "fp8", "int8", "fp4", "fp64", "fp32"],
                        choices=["bf16", "fp16", "fp8", "int8", "fp4", "fp64", "fp32"])
    parser.add_argument("--gemm-size", type=int, default=GEMM_SIZE, help="square GEMM size (default 8192)")
    parser.add_argument("--fp4-size", type=int, default=FP4_GEMM_SIZE,
                        help="square MXFP4 GEMM size (default 16384, BASELINE's configuration)")
    parser.add_argument("--fp64-size", type=int, default=FP64_GEMM_SIZE,
                        help="square FP64 GEMM size (default 4096, BASELINE's configuration)")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--quick", action="store_true", help="small sizes: a smoke check, not a measurement")
    add_common_arguments(parser)
    return parser


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)
    if args.quick:
        args.copy_mib, args.gemm_size, args.fp4_size, args.fp64_size = [8], 512, 512, 512
        args.warmup, args.rep, args.rounds = 5, 10, 3
    metadata = setup_device(args)
    rows = copy_rows(args, args.copy_mib) + gemm_rows(args, args.gemm_dtypes, args.gemm_size, args.fp4_size,
                                                      args.fp64_size)
    print(f"{'check':6s} {'path':18s} {'case':14s} {'peak':>12s} {'median':>12s} {'% peak':>7s}  note")
    for row in rows:
        if row.get("status") == "unavailable":
            print(f"{row['check']:6s} {row['path']:18s} {row['dtype']:14s} {'-':>12s} {'-':>12s} {'-':>7s}  "
                  f"{row['reason']}")
            continue
        if row["check"] == "copy":
            case, peak, median, frac = f"{row['buffer_mib']} MiB", row["peak_gbps"], row["gbps"], \
                row["fraction_of_hbm_peak"]
            note = "GB/s"
        else:
            case, peak, median, frac = f"{row['dtype']} {row['m']}^3", row["peak_teraops_per_second"], \
                row["median_teraops_per_second"], row["fraction_of_peak"]
            note = "TFLOP/s" + (f", normwise diff {row['normwise_difference']:.2g}"
                                if row.get("normwise_difference") is not None else "")
            if row.get("max_bf16_ulps") is not None:
                note += f", library BF16 C within {row['max_bf16_ulps']:.2f} ulp"
        print(f"{row['check']:6s} {row['path']:18s} {case:14s} {peak:12.1f} {median:12.1f} {100 * frac:7.1f}  {note}")
    emit_results("crosscheck", metadata, args, rows)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
