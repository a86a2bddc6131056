#!/usr/bin/env python3
"""Headline benchmark of the MI355X peak-throughput suite (one JSON line).

Metric: "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of MI355X
peak". One step is one launch of every kernel below on inputs already resident
in HBM. Each row is one configuration of the benchmark specification:

  hbm_copy        configs[0]  mb_copy of 2^28 fp32 (1 GiB, uniform[-1,1) from
                              seed 0) into a second buffer; bit-exact
  peak_bf16       configs[2]  resident-operand variant: a 256x256x64 BF16 LDS
                              tile looped 1024 times per workgroup, 1 chain,
                              2 workgroups per CU, in-place 16x16 MFMAs
  gemm_bf16       configs[2]  BF16 GEMM 8192^3, A, B ~ N(0,1), B column-major
  gemm_fp16       configs[2]  FP16 GEMM 8192^3, same operands
  gemm_fp8        configs[3]  FP8 E4M3 GEMM 8192^3 over {+-0.5, +-1, +-2}; exact
  gemm_int8       configs[3]  INT8 GEMM 8192^3 over [-8, 8]; exact
  gemm_fp64       configs[3]  FP64 GEMM 4096^3, N(0,1)
  gemm_mxfp4      configs[4]  MXFP4 GEMM 16384^3, all 16 E2M1 codes, E8M0
                              scale 127 per 32 K elements; exact
  peak_bf16_128x128_c2        the 128x128x64 BF16 tile with 2 chains, 4 per CU
                              (a smaller tile than the specification's; not
                              in the headline mean)
  peak_fp8        17-row table: FP8 resident tile 128x128x128, 2 chains,
                              the reference's one-hot operands
  peak_fp8_dense  the same kernel on the dense {+-0.5, +-1, +-2} set
  peak_mxfp4      17-row table: MXFP4 resident tile 128x128x256, 2 chains,
                              the reference's +-0.5/+-1 codes
  vector_fp32, vector_fp16, vector_bf16, vector_fp64, vector_int8
                  configs[1]  2^22 lanes (16 workgroups of 1024 per CU), 8
                              independent accumulators x 4096 iterations of
                              x = x*a + b, a0 ~ U[0.5, 1), a = 0.999, b = 1e-3
                              (INT8: DP4A, x0 in [-4, 4], weights and bias 1)

The resident tiles issue the 16x16 form of each MFMA (v_mfma_f32_16x16x32_bf16,
v_mfma_f32_16x16x128_f8f6f4, v_mfma_scale_f32_16x16x128_f8f6f4): at the same
MFMA busy fraction it sustains a higher engine clock under the power limit
than the 32x32 form, which moves four times the accumulator bytes per flop.

value = mean of achieved / MI355X published peak, in percent, over the
HEADLINE rows (hbm_copy, peak_bf16, gemm_bf16, gemm_fp8, gemm_mxfp4: the
metric's four formats at the specification's sizes); every row carries its
own fraction. Every output is validated before timing and again on the timed
launches' output (bit-exact copy; exact FP8/INT8/MXFP4 GEMMs; elementwise
|C-R| <= atol + rtol*|R| for BF16/FP16 (the reference's 2e-3; the
specification's 1e-2 is reported beside it) and FP64 (1e-12) against a
float64 device product; the resident tiles against their exact lattice
reference under the reference's tolerance; FP32/FP64 vector chains against
the closed form of the affine recurrence, FP16/BF16 sampled lanes bit-exact
against a step-by-step recompute, INT8 exact).

Timing, per kernel in turn (the reference's policy, common.py:459-461, warms
for a device-time budget): untimed launches until at least --warmup launches
AND --warmup-ms of device time have run, so the clock has settled at this
kernel's load; then exactly --steps launches, bracketed by
torch.cuda.synchronize(), with HIP events on the launch stream between
sub-batches of about --sub-batch-ms. ms_per_launch is the whole timed region
over --steps; min and median are over the sub-batch averages.

Between a row's warmup and its timed launches, a one-wave clock witness on a
second stream measures the engine clock its kernel sustains (ClockWitness);
the row reports it with frac_at_clock = rate / (peak * clock / 2400 MHz).
After every row is timed, a separate pass runs each kernel of POWER_ROWS back
to back for POWER_LOAD_MS while the board's energy counter is read
(PowerMeter, the ROCm SMI library, when importable): power_w per row and the
board's cap, which shows a row whose clock is held down by the power limit.

After the copy's timed launches, the same buffers are streamed read-only
(mb_read_sum) and write-only (mb_fill): their harmonic mean bounds a copy,
which moves equal read and write bytes over the same HBM channels, and the
copy row reports it (rw_bound_frac).

Output: ONE JSON line on stdout, kept under 8 KiB (the contract fields, the
roofline of the dominant headline kernel, a compact cpu_baseline and, per row,
name, kernel, value, unit, fraction, ms per launch, clock and frac_at_clock);
the full per-row records (configuration, validation, min/median, warmup,
traffic, per-row CPU figures, clock measurement) go to the --detail file,
whose path the line names.

cpu_baseline times the reference's own host arithmetic for each row on this
machine's cores (torch.Tensor.copy_ of 1 GiB; torch.matmul in fp32, fp64
for FP64, on sampled rows of the same GEMM shape or a batch of the same
tiles; the recurrence vectorised by torch for the vector rows), best repeat
within a per-row budget.
"""

from __future__ import annotations

import argparse
import json
import math
import os
from pathlib import Path
import statistics
import sys

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of MI355X peak"
HEADLINE = ("hbm_copy", "peak_bf16", "gemm_bf16", "gemm_fp8", "gemm_mxfp4")
COPY_ELEMENTS = 2**28
COPY_SEED = 0
# One 64-lane wave per workgroup, one 16-byte vector per lane, nt loads and
# device-scope stores written through the L2: the fastest shape and policy of
# the bench_bandwidth sweep on MI355X.
COPY_CONFIG = {"block_threads": 64, "vectors_per_thread": 1, "grid_blocks": 0, "nontemporal": "stream"}
PEAK_ITERATIONS = 1024
GEMM_SEED = 0
VECTOR_ITERATIONS = 4096
VECTOR_SEED = 0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_per_launch.txt"
CPU_ROW_BUDGET_S = 2.0
# The stdout line's bound: a driver that keeps the tail of stdout must see all of it.
MAX_LINE_BYTES = 8192
# Clock witness of a row: real-time interval it measures, inside launches of the row's kernel lasting
# CLOCK_LOAD_MS, between the warmup and the timed launches.
CLOCK_WITNESS_MS = 100.0
CLOCK_LOAD_MS = 150.0
# Rows whose board power is measured, and the load that measurement needs: the board's energy counter updates
# once a second, so in a pass after every row is timed, each of these kernels runs back to back for
# POWER_LOAD_MS and the mean power is taken between the first and last counter updates inside that load.
POWER_ROWS = ("hbm_copy", "peak_bf16", "gemm_bf16", "gemm_fp16", "gemm_fp8", "gemm_int8", "gemm_fp64", "gemm_mxfp4",
              "peak_mxfp4")
POWER_LOAD_MS = 2300.0
# Read-only and write-only legs of the copy bound: kernel shapes (the fastest of the bench_bandwidth sweeps) and
# launches timed per leg.
READ_BOUND_CONFIG = {"block_elements": 1024, "block_threads": 64}
WRITE_BOUND_CONFIG = {"block_threads": 256, "grid_blocks": 0, "policy": "stream"}
BOUND_LAUNCHES = 40


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50, help="timed launches of each kernel (default: 50)")
    parser.add_argument("--warmup", type=int, default=20,
                        help="minimum untimed launches of each kernel before its timed ones (default: 20)")
    parser.add_argument("--warmup-ms", type=float, default=250.0,
                        help="minimum device time of those untimed launches, per kernel (default: 250)")
    parser.add_argument("--sub-batch-ms", type=float, default=2.0,
                        help="device time between two events inside the timed launches (default: 2)")
    parser.add_argument("--no-cpu-baseline", action="store_true", help="skip the host CPU leg")
    parser.add_argument("--rows", nargs="+", help="subset of rows to run (default: all)")
    parser.add_argument("--detail", default=str(ROOT / "results" / "bench_detail.json"),
                        help="file for the full per-row records (default: results/bench_detail.json)")
    parser.add_argument("--no-clock", action="store_true",
                        help="do not measure the engine clock each row's kernel runs at")
    return parser.parse_args(argv)


def traffic_table() -> dict[str, float]:
    """Measured HBM bytes per launch by kernel name (committed rocprofv3 counter runs)."""
    table = {}
    if TRAFFIC_FILE.exists():
        for line in TRAFFIC_FILE.read_text().splitlines():
            line = line.split("#", 1)[0].strip()
            if "=" in line:
                key, value = (part.strip() for part in line.split("=", 1))
                try:
                    table[key] = float(value)
                except ValueError:
                    pass
    return table


class Workload:
    """One row: owns its resident device buffers; launch() enqueues one kernel launch."""

    name = row = unit = bound = label = kernel = ""
    work = 0.0
    config: dict = {}

    def launch(self):
        raise NotImplementedError

    def poison(self):
        raise NotImplementedError

    def check(self) -> str:
        raise NotImplementedError

    def cpu(self) -> dict:
        raise NotImplementedError

    def rate(self, ms: float) -> float:
        return self.work / (ms * (1e6 if self.unit == "GB/s" else 1e9))

    def context(self, stream) -> dict | None:
        """Extra figures measured after the row's timed launches (None: the row has none)."""
        del stream
        return None


class CopyWorkload(Workload):
    name, row, unit, bound, label = "hbm_copy", "memory_bandwidth", "GB/s", "hbm", "f32 copy"

    def __init__(self, torch, compute_units):
        from triton_chip_benchmarks_amd import bench_bandwidth

        del compute_units
        self.torch, self.bb = torch, bench_bandwidth
        generator = torch.Generator(device="cuda").manual_seed(COPY_SEED)
        self.src = torch.empty(COPY_ELEMENTS, device="cuda", dtype=torch.float32).uniform_(-1, 1, generator=generator)
        self.dst = torch.empty_like(self.src)
        self.work = 2 * self.src.numel() * 4  # read + write bytes (bench_bandwidth.py:212)
        self.kernel = f"copy_dwordx4_vpt{COPY_CONFIG['vectors_per_thread']}" + bench_bandwidth.POLICY_SUFFIX[
            bench_bandwidth.copy_policy(COPY_CONFIG["nontemporal"])]
        self.config = {"elements": COPY_ELEMENTS, "dtype": "fp32", "seed": COPY_SEED, **COPY_CONFIG}

    def launch(self):
        c = COPY_CONFIG
        self.bb.launch_copy(self.src, self.dst, c["block_threads"], c["vectors_per_thread"], c["grid_blocks"],
                            c["nontemporal"])

    def poison(self):
        self.dst.fill_(float("nan"))

    def check(self):
        self.torch.cuda.synchronize()
        if not self.torch.equal(self.src.view(self.torch.int32), self.dst.view(self.torch.int32)):
            raise AssertionError("hbm_copy: destination differs from its source")
        return "bit-exact: every word of the 1 GiB destination equals the source"

    def cpu(self):
        from triton_chip_benchmarks_amd import cpu_baseline

        return cpu_baseline.copy_baseline(COPY_ELEMENTS * 4, CPU_ROW_BUDGET_S)

    def context(self, stream) -> dict:
        """The copy's read-only and write-only legs on the same buffers (after the copy's own timing and check):
        each leg's GB/s, validated, and their harmonic mean, the copy's read/write bound."""
        torch, bb = self.torch, self.bb
        nbytes = self.src.numel() * 4
        r, w = READ_BOUND_CONFIG, WRITE_BOUND_CONFIG
        sink = torch.full((self.src.numel() // r["block_elements"],), float("nan"), device="cuda")

        def read():
            bb.launch_read(self.src, sink, r["block_elements"], r["block_threads"])

        def write():
            bb.launch_fill(self.dst, w["block_threads"], w["grid_blocks"], w["policy"])

        rates = {}
        for leg, launch, traffic in (("read", read, nbytes + sink.numel() * 4), ("write", write, nbytes)):
            for _ in range(10):
                launch()
            events = _Events(torch, stream)
            events.mark(0)
            for _ in range(BOUND_LAUNCHES):
                launch()
            events.mark(BOUND_LAUNCHES)
            torch.cuda.synchronize()
            rates[leg] = traffic / (events.intervals()[0][1] / BOUND_LAUNCHES * 1e6)
        bb.check_read(self.src, sink, r["block_elements"])
        bb.check_fill(self.dst)
        bound = bb.rw_bound(rates["read"], rates["write"])
        return {"read_only_gbps": rates["read"], "write_only_gbps": rates["write"], "rw_bound_gbps": bound,
                "read_config": dict(r, kernel="read_sum_fp32_vec"), "write_config": dict(w, kernel="fill_dwordx4_stream"),
                "launches_per_leg": BOUND_LAUNCHES,
                "method": "read-only (mb_read_sum) and write-only (mb_fill) streams over the copy's own 1 GiB buffers, "
                          "both validated; bound = harmonic mean of the two rates"}


class PeakWorkload(Workload):
    """A resident-operand MFMA tile looped PEAK_ITERATIONS times per workgroup (tensor rows)."""

    unit, bound = "TFLOP/s", "mfma"
    LABELS = {"bf16": "bf16", "fp8": "fp8_e4m3", "fp4": "mxfp4_e2m1"}

    def __init__(self, torch, compute_units, name, dtype, tile, chains, per_cu, operands="lattice", mfma_m=32):
        from triton_chip_benchmarks_amd import _native, bench_tensor

        self.torch, self.bt, self.dtype, self.name = torch, bench_tensor, dtype, name
        self.row, self.label = f"tensor_{dtype}", self.LABELS[dtype]
        m, n, k = tile
        self.cfg = next(c for c in _native.peak_configs(dtype) if (c["tile_m"], c["tile_n"], c["tile_k"]) == tile
                        and c["chains"] == chains and c["mfma_m"] == mfma_m and not c["b_nk"])
        self.kernel = _native.peak_kernel_name(dtype, self.cfg)
        self.blocks = per_cu * compute_units
        if dtype == "fp4":
            self.a, self.b, self.c, self.scales, self.values = bench_tensor.fp4_peak_inputs(self.blocks, self.cfg,
                                                                                           "cuda")
            operand_text = "codes of +-0.5 and +-1 (the reference's set), E8M0 scale 127"
        else:
            self.a, self.b, self.c, b_logical = bench_tensor.peak_inputs(self.blocks, self.cfg, dtype, "cuda",
                                                                          operands=operands)
            self.scales, self.values = None, (self.a, b_logical)
            operand_text = {"lattice": "the reference's exact lattice" + (" (one-hot A)" if dtype == "fp8" else ""),
                            "dense": "every entry from {+-0.5, +-1, +-2}"}[operands]
        self.reference = bench_tensor.exact_reference(self.values[0], self.values[1], PEAK_ITERATIONS,
                                                      torch.float32)
        self.work = 2 * m * n * k * PEAK_ITERATIONS * chains * self.blocks  # bench_tensor.py:1242
        self.config = {"tile": f"{m}x{n}x{k}", "mfma": f"{mfma_m}x{mfma_m}", "chains": chains,
                       "blocks": self.blocks, "blocks_per_cu": per_cu,
                       "iterations": PEAK_ITERATIONS, "b_layout": "kn", "operands": operand_text}

    def launch(self):
        self.bt.launch_peak(self.dtype, self.cfg, self.a, self.b, self.c, PEAK_ITERATIONS, self.scales)

    def poison(self):
        self.c.fill_(float("nan"))

    def check(self):
        self.torch.cuda.synchronize()
        result = self.bt.validate_peak(self.c, self.reference, self.dtype, self.cfg["tile_k"], PEAK_ITERATIONS)
        return (f"every output within atol {result['atol']:.3g} of the exact lattice reference "
                f"(max error {result['max_abs_error']:.3g})")

    def cpu(self):
        from triton_chip_benchmarks_amd import cpu_baseline

        m, n, k = self.cfg["tile_m"], self.cfg["tile_n"], self.cfg["tile_k"]
        return cpu_baseline.tile_batch_baseline(self.dtype, 64, m, n, k, CPU_ROW_BUDGET_S)


class GemmWorkload(Workload):
    """C = A . B at the specification's size (B column-major), largest tile of mb_gemm."""

    bound = "mfma"
    LABELS = {"bf16": "bf16", "fp16": "fp16", "fp8": "fp8_e4m3", "int8": "int8", "fp64": "f64",
              "fp4": "mxfp4_e2m1"}

    def __init__(self, torch, compute_units, name, dtype, size):
        from triton_chip_benchmarks_amd import _native, gemm

        del compute_units
        self.torch, self.gemm, self.native, self.dtype, self.name, self.size = torch, gemm, _native, dtype, name, size
        self.row, self.label = f"tensor_{dtype}", self.LABELS[dtype]
        self.unit = "TOP/s" if dtype == "int8" else "TFLOP/s"
        self.cfg = max(_native.gemm_configs(dtype), key=lambda c: c["tile_m"] * c["tile_n"])
        self.kernel = _native.gemm_kernel_name(dtype, self.cfg)
        a, b, c, scales, a_values, b_values = gemm.gemm_inputs(dtype, size, size, size, "cuda", GEMM_SEED)
        self.a, self.b, self.c, self.scales = a, b, c, scales or (None, None)
        self.reference = gemm.reference(a_values, b_values)
        del a_values, b_values
        self.work = 2 * size**3
        self.config = {"m": size, "n": size, "k": size, "tile": f"{self.cfg['tile_m']}x{self.cfg['tile_n']}x"
                       f"{self.cfg['tile_k']}", "layout": "A row-major, B column-major",
                       "operands": gemm.INPUT_PATTERN[dtype], "seed": GEMM_SEED}

    def launch(self):
        self.native.gemm(self.dtype, self.cfg, self.a, self.b, self.c, self.size, self.size, self.size, *self.scales)

    def poison(self):
        self.c.fill_(-2**31 if self.dtype == "int8" else float("nan"))

    def check(self):
        self.torch.cuda.synchronize()
        result = self.gemm.validate(self.c, self.reference, self.dtype)
        if result["rtol"]:
            return (f"every entry within |C-R| <= {result['atol']:g} + {result['rtol']:g}*|R| of the float64 "
                    f"product (max error {result['max_abs_error']:.3g}, worst error/allowed "
                    f"{result['max_error_over_allowed']:.3g})")
        return "bit-exact against the float64 product (the operand set is exact in the accumulator)"

    def cpu(self):
        from triton_chip_benchmarks_amd import cpu_baseline

        rows = 256 if self.size <= 8192 else 128
        return cpu_baseline.gemm_sample_baseline(self.dtype, rows, self.size, self.size, CPU_ROW_BUDGET_S)


class VectorWorkload(Workload):
    """Independent FMA (INT8: DP4A) chains on the VALU: 16 workgroups of 1024 lanes per CU, 8 accumulators each."""

    bound = "valu"
    # Updates per loop trip: the suite sweep's best for each format.
    UNROLL = {"fp32": 8, "fp16": 16, "bf16": 8, "fp64": 16, "int8": 16}
    LABELS = {"fp32": "f32", "fp16": "f16", "bf16": "bf16", "fp64": "f64", "int8": "int8"}

    def __init__(self, torch, compute_units, name, dtype):
        from triton_chip_benchmarks_amd import _native, bench_vector

        self.torch, self.bv, self.dtype, self.name = torch, bench_vector, dtype, name
        self.row, self.label = f"vector_{dtype}", self.LABELS[dtype]
        self.unit = "TOP/s" if dtype == "int8" else "TFLOP/s"
        self.variant = bench_vector.VARIANTS[dtype][0]
        self.kind, self.unroll, self.block = self.variant[0], self.UNROLL[dtype], 1024
        self.elements = 16 * compute_units * self.block  # 2^22 lanes on 256 CUs
        self.inputs, self.coefficients = bench_vector.make_inputs(dtype, self.elements, "cuda", "baseline",
                                                                  VECTOR_SEED)
        self.output = torch.empty_like(self.inputs)
        if self.kind == "bf16_dot2":  # once, so no timed launch reads the operands back
            bench_vector.require_dot2_regime(self.inputs, self.coefficients, VECTOR_ITERATIONS)
        self.kernel = _native.load().mb_vector_kernel_name(bench_vector.KINDS[self.kind], self.unroll).decode()
        per_update = 8 if dtype == "int8" else 2  # bench_vector.py:1271-1273
        self.work = per_update * bench_vector.CHAINS * self.elements * VECTOR_ITERATIONS
        self.config = {"lanes": self.elements, "workgroups_per_cu": 16, "block": self.block,
                       "accumulators": bench_vector.CHAINS, "iterations": VECTOR_ITERATIONS, "unroll": self.unroll,
                       "operation": self.variant[1], "inputs": "x0 in [-4, 4], weights and bias 1" if dtype == "int8"
                       else "x0 ~ U[0.5, 1), a = 0.999, b = 1e-3", "seed": VECTOR_SEED}

    def launch(self):
        self.bv.launch_vector(self.kind, self.inputs, self.output, self.coefficients, VECTOR_ITERATIONS, self.unroll,
                              self.block, regime_checked=True)

    def poison(self):
        self.output.fill_(-(2**31) if self.dtype == "int8" else float("nan"))

    def check(self):
        self.torch.cuda.synchronize()
        result = self.bv.validate(self.dtype, self.kind, self.inputs, self.output, self.coefficients,
                                  VECTOR_ITERATIONS, "baseline", None)
        return "; ".join(str(result[key]) for key in ("correctness", "step_recompute") if key in result)

    def cpu(self):
        from triton_chip_benchmarks_amd import cpu_baseline

        return cpu_baseline.vector_baseline(self.dtype, 2**22, 8, CPU_ROW_BUDGET_S)


def _row_specs():
    """(name, factory) in run order; factories take (torch, compute_units)."""
    def peak(name, dtype, tile, chains, per_cu, operands="lattice", mfma_m=16):
        return name, lambda t, cu: PeakWorkload(t, cu, name, dtype, tile, chains, per_cu, operands, mfma_m)

    def gemm(name, dtype, size):
        return name, lambda t, cu: GemmWorkload(t, cu, name, dtype, size)

    def vector(name, dtype):
        return name, lambda t, cu: VectorWorkload(t, cu, name, dtype)

    return [
        ("hbm_copy", CopyWorkload),
        peak("peak_bf16", "bf16", (256, 256, 64), 1, 2),
        gemm("gemm_bf16", "bf16", 8192),
        gemm("gemm_fp16", "fp16", 8192),
        gemm("gemm_fp8", "fp8", 8192),
        gemm("gemm_int8", "int8", 8192),
        gemm("gemm_fp64", "fp64", 4096),
        gemm("gemm_mxfp4", "fp4", 16384),
        peak("peak_bf16_128x128_c2", "bf16", (128, 128, 64), 2, 4),
        peak("peak_fp8", "fp8", (128, 128, 128), 2, 4),
        peak("peak_fp8_dense", "fp8", (128, 128, 128), 2, 4, "dense"),
        peak("peak_mxfp4", "fp4", (128, 128, 256), 2, 4),
        *(vector(f"vector_{dtype}", dtype) for dtype in ("fp32", "fp16", "bf16", "fp64", "int8")),
    ]


class _Events:
    def __init__(self, torch, stream):
        self.torch, self.stream, self.marks = torch, stream, []

    def mark(self, launches_so_far):
        event = self.torch.cuda.Event(enable_timing=True)
        event.record(self.stream)
        self.marks.append((launches_so_far, event))

    def intervals(self):
        """[(launches, ms)] between consecutive marks (call after synchronize)."""
        out = []
        for (n0, e0), (n1, e1) in zip(self.marks, self.marks[1:]):
            ms = float(e0.elapsed_time(e1))
            if not math.isfinite(ms) or ms <= 0:
                raise RuntimeError(f"invalid device event time {ms!r} ms")
            out.append((n1 - n0, ms))
        return out


class ClockWitness:
    """The engine clock a row's kernel sustains (mb_clock_witness), measured on the device.

    One sleeping wave on a second stream counts shader clock cycles against the constant-rate real-time counter
    for CLOCK_WITNESS_MS while the row's kernel runs back to back for CLOCK_LOAD_MS on the launch stream, after
    its warmup (the same steady load the timed launches see) and outside the timed region. The clock is that of
    the witness's CU; rate / (peak * clock / 2400 MHz) then separates a low-clock box from a slow kernel.
    """

    def __init__(self, torch, native):
        self.torch, self.native = torch, native
        self.side = torch.cuda.Stream()
        self.out = torch.zeros(4, dtype=torch.int64, device="cuda")
        self.wall_khz = native.wall_clock_khz()

    def measure(self, stream, workload, estimate_ms: float) -> dict:
        launches = max(2, math.ceil(CLOCK_LOAD_MS / max(estimate_ms, 1e-3)))
        self.out.zero_()
        self.torch.cuda.synchronize()
        self.native.clock_witness(self.out, int(CLOCK_WITNESS_MS * 1000), self.side)
        for _ in range(launches):
            workload.launch()
        self.torch.cuda.synchronize()
        cycles, ticks, polls, _start = (int(v) for v in self.out.tolist())
        complete = ticks >= CLOCK_WITNESS_MS * self.wall_khz * 0.999
        return {"clock_mhz": cycles / ticks * self.wall_khz / 1000 if ticks and complete else None,
                "witness_ms": ticks / self.wall_khz, "polls": polls, "load_launches": launches,
                "method": "mb_clock_witness: s_memtime cycles / s_memrealtime ticks of one wave beside the "
                          "kernel's launches"}


class PowerMeter:
    """Board power while a row's kernel runs, from the GPU's energy counter read through the ROCm SMI library.

    The counter (amdsmi_get_energy_count: accumulated energy and the time stamp of its last update, in ns) is
    updated about once a second. A thread polls it every POLL_S between start() and stop(); stop() returns the
    mean power between the first and the last update seen (energy difference over time-stamp difference), the
    seconds that covers, and the board's power cap, or None when fewer than two updates fell inside the window.
    available() is False when the library cannot be imported or does not see this device (matched by PCI bus
    id), and the rows then carry no power figure. Reading the counter changes nothing on the device.
    """

    POLL_S = 0.01

    def __init__(self, torch):
        self.handle, self.cap_w, self._thread, self._samples = None, None, None, []
        try:
            sys.path.append(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "share", "amd_smi"))
            import amdsmi

            amdsmi.amdsmi_init()
            handles = amdsmi.amdsmi_get_processor_handles()
            props = torch.cuda.get_device_properties(0)
            bus = getattr(props, "pci_bus_id", None)
            matches = [h for h in handles
                       if bus is not None and int(amdsmi.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == bus]
            self.handle = matches[0] if len(matches) == 1 else handles[0] if len(handles) == 1 else None
            self.amdsmi = amdsmi
            if self.handle is not None:
                limit = amdsmi.amdsmi_get_power_info(self.handle).get("power_limit")
                self.cap_w = limit / 1e6 if isinstance(limit, (int, float)) and limit > 1e5 else limit
        except Exception as error:  # the library is optional: no power figures without it
            print(f"[bench] power meter unavailable: {error!r}", file=sys.stderr, flush=True)
            self.handle = None

    def available(self) -> bool:
        return self.handle is not None

    def measure(self, workload, estimate_ms: float) -> dict | None:
        """Mean board power over POWER_LOAD_MS of the row's kernel back to back."""
        launches = max(2, math.ceil(POWER_LOAD_MS / max(estimate_ms, 1e-3)))
        import torch

        torch.cuda.synchronize()
        self.start()
        for _ in range(launches):
            workload.launch()
        torch.cuda.synchronize()
        result = self.stop()
        if result is not None:
            result["launches"] = launches
        return result

    def _read(self):
        import time

        counter = self.amdsmi.amdsmi_get_energy_count(self.handle)
        return (counter["energy_accumulator"] * counter["counter_resolution"], counter["timestamp"],
                time.perf_counter())

    def start(self):
        import threading
        import time

        self._samples, self._stop = [], threading.Event()

        def sample():
            while not self._stop.is_set():
                try:
                    value = self._read()
                except Exception:
                    value = None
                if value is not None and (not self._samples or value[1] != self._samples[-1][1]):
                    self._samples.append(value)  # one entry per counter update
                time.sleep(self.POLL_S)

        self._thread = threading.Thread(target=sample, daemon=True)
        self._thread.start()

    def stop(self) -> dict | None:
        self._stop.set()
        self._thread.join()
        updates = self._samples[1:]  # the first entry is the counter as found, updated before the load began
        if len(updates) < 2:
            return None
        (e0, t0, h0), (e1, t1, h1) = updates[0], updates[-1]
        seconds = (t1 - t0) / 1e9
        if seconds <= 0:
            return None
        return {"mean_w": (e1 - e0) / 1e6 / seconds, "seconds": seconds, "host_seconds": h1 - h0,
                "updates": len(updates),
                "cap_w": self.cap_w,
                "method": "energy counter (amdsmi_get_energy_count) difference between its first and last "
                          "updates during the row's back-to-back launches"}


def warm(torch, stream, workload, min_launches, min_ms):
    """Untimed launches until both minimums are met; returns (launches, device ms)."""
    events = _Events(torch, stream)
    events.mark(0)
    workload.launch()
    events.mark(1)
    torch.cuda.synchronize()
    first = events.intervals()[0][1]
    done, elapsed, estimate = 1, first, first
    # Submit ~50 ms of launches at a time and re-measure, until both minimums hold.
    while done < min_launches or elapsed < min_ms:
        chunk = max(1, min(math.ceil(50.0 / estimate), math.ceil(max(min_ms - elapsed, 0.0) / estimate)),
                    min_launches - done)
        events = _Events(torch, stream)
        events.mark(0)
        for _ in range(chunk):
            workload.launch()
        events.mark(chunk)
        torch.cuda.synchronize()
        ms = events.intervals()[0][1]
        done, elapsed, estimate = done + chunk, elapsed + ms, ms / chunk
    return done, elapsed, estimate


def time_launches(torch, stream, workload, steps, per_batch):
    """Exactly `steps` launches, an event after every `per_batch`; returns [(launches, ms)]."""
    events = _Events(torch, stream)
    torch.cuda.synchronize()
    events.mark(0)
    for index in range(1, steps + 1):
        workload.launch()
        if index % per_batch == 0 or index == steps:
            events.mark(index)
    torch.cuda.synchronize()
    return events.intervals()


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported. Every row runs on a single "
              "GPU; a multi-GPU figure would be the sum of independent per-GPU rates, which this build does not "
              "launch.", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0 or args.warmup_ms < 0 or args.sub_batch_ms <= 0:
        print("--steps and --sub-batch-ms must be positive, --warmup and --warmup-ms non-negative",
              file=sys.stderr)
        return 2
    specs = _row_specs()
    if args.rows:
        unknown = set(args.rows) - {name for name, _ in specs}
        if unknown:
            print(f"unknown rows: {', '.join(sorted(unknown))}", file=sys.stderr)
            return 2
        specs = [(name, factory) for name, factory in specs if name in args.rows]

    import torch

    from triton_chip_benchmarks_amd import _native, roofline
    from triton_chip_benchmarks_amd.common import require_gpu

    require_gpu(0)
    info = _native.device_query(0)
    stream = torch.cuda.current_stream()
    traffic = traffic_table()
    rows, workloads = [], []
    for name, factory in specs:
        print(f"[bench] {name}: building operands and validating", file=sys.stderr, flush=True)
        workload = factory(torch, info["compute_units"])
        workload.poison()
        workload.launch()
        validation = workload.check()
        workloads.append((workload, validation))

    witness = None if args.no_clock else ClockWitness(torch, _native)
    power = None if args.no_clock else PowerMeter(torch)
    if power is not None and not power.available():
        power = None
    estimates = []
    for workload, validation in workloads:
        print(f"[bench] {workload.name}: warmup and {args.steps} timed launches", file=sys.stderr, flush=True)
        warm_launches, warm_ms, estimate = warm(torch, stream, workload, args.warmup, args.warmup_ms)
        per_batch = max(1, min(args.steps, round(args.sub_batch_ms / estimate)))
        clock = witness.measure(stream, workload, estimate) if witness is not None else None
        workload.poison()  # the timed launches must rewrite the whole output
        samples = time_launches(torch, stream, workload, args.steps, per_batch)
        workload.check()  # raises if the timed launches' output is wrong
        validation += "; passed again on the timed launches' output"
        context = workload.context(stream)
        estimates.append(estimate)
        total_ms = sum(ms for _, ms in samples)
        per_launch = [ms / n for n, ms in samples]
        mean_ms = total_ms / args.steps
        achieved = workload.rate(mean_ms)
        peak, _unit, basis = roofline.PEAKS[workload.row]
        rows.append({
            "name": workload.name, "row": workload.row, "in_headline": workload.name in HEADLINE,
            "kernel": workload.kernel, "value": achieved, "unit": workload.unit, "peak": peak,
            "frac": achieved / peak, "peak_basis": basis, "bound": workload.bound,
            "ms_per_launch": mean_ms, "min_ms_per_launch": min(per_launch),
            "median_ms_per_launch": statistics.median(per_launch),
            "value_at_min": workload.rate(min(per_launch)), "value_at_median": workload.rate(statistics.median(per_launch)),
            "sub_batches": len(samples), "launches_per_sub_batch": per_batch,
            "warmup_launches": warm_launches, "warmup_device_ms": warm_ms,
            "algorithmic_work_per_launch": workload.work, "work_unit": "bytes" if workload.bound == "hbm" else "flop",
            "traffic_bytes_per_launch": traffic.get(workload.kernel), "dtype": workload.label,
            "clock": clock, "power": None, "config": workload.config, "validation": validation})
        if context:
            rows[-1]["context"] = context
            if "rw_bound_gbps" in context:
                rows[-1]["rw_bound_frac"] = context["rw_bound_gbps"] / peak
                rows[-1]["frac_of_rw_bound"] = achieved / context["rw_bound_gbps"]
        if clock and clock["clock_mhz"] and workload.bound != "hbm":
            # The same work per clock at the clock this kernel ran at: separates a low-clock box from a slow kernel.
            rows[-1]["frac_at_clock"] = achieved / (peak * clock["clock_mhz"] / roofline.PEAK_CLOCK_MHZ)
        if workload.row in roofline.ISSUED_CEILINGS:  # the instruction this build issues is slower than the datasheet's
            ceiling, ceiling_basis = roofline.ISSUED_CEILINGS[workload.row]
            rows[-1].update(issued_instruction_ceiling=ceiling, issued_instruction_basis=ceiling_basis,
                            frac_of_issued_ceiling=achieved / ceiling)

    if power is not None:
        # A separate pass after every row is timed: the seconds of load it needs must not heat the chip ahead of
        # any row's timed launches.
        for row, (workload, _), estimate in zip(rows, workloads, estimates):
            if workload.name in POWER_ROWS:
                print(f"[bench] {workload.name}: board power", file=sys.stderr, flush=True)
                row["power"] = power.measure(workload, estimate)

    cpu_rows = None
    if not args.no_cpu_baseline:
        cpu_rows = []
        for workload, _ in workloads:
            print(f"[bench] {workload.name}: host CPU baseline", file=sys.stderr, flush=True)
            result = workload.cpu()
            peak = roofline.PEAKS[workload.row][0]
            cpu_rows.append({"name": workload.name, "value": result["value"], "unit": result["unit"],
                             "cores": result["cores"], "method": result["method"], "sample": result["sample"],
                             "frac_of_mi355x_peak": result["value"] / peak})
    from triton_chip_benchmarks_amd.cpu_baseline import host_description

    document = full_document(args, info, rows, cpu_rows, host_description() if cpu_rows else None)
    detail = Path(args.detail)
    detail.parent.mkdir(parents=True, exist_ok=True)
    detail.write_text(json.dumps(document, indent=1) + "\n")
    print(json.dumps(headline_line(document, str(detail))))
    return 0


def full_document(args, info, rows, cpu_rows, host) -> dict:
    """Every figure of the run: the contract fields plus the full per-row records."""
    headline = [r for r in rows if r["in_headline"]] or rows
    value = 100.0 * sum(r["frac"] for r in headline) / len(headline)
    dominant = max(headline, key=lambda r: r["ms_per_launch"])
    roofline_block = {"bound": dominant["bound"], "kernel": dominant["kernel"], "row": dominant["name"],
                      "achieved": dominant["value"], "peak": dominant["peak"], "unit": dominant["unit"],
                      "frac": dominant["frac"], "traffic": dominant["traffic_bytes_per_launch"],
                      "algorithmic_work_per_launch": dominant["algorithmic_work_per_launch"],
                      "work_unit": dominant["work_unit"], "ms_per_launch": dominant["ms_per_launch"],
                      # The conditions it ran under: its engine clock (witness), the fraction at that clock, and the
                      # board power its kernel draws (None where not measured).
                      "clock_mhz": (dominant.get("clock") or {}).get("clock_mhz"),
                      "frac_at_clock": dominant.get("frac_at_clock"),
                      "power_w": (dominant.get("power") or {}).get("mean_w")}
    cpu = None
    if cpu_rows:
        in_mean = [r for r in cpu_rows if r["name"] in HEADLINE] or cpu_rows
        cpu = {"value": 100.0 * sum(r["frac_of_mi355x_peak"] for r in in_mean) / len(in_mean),
               "unit": "% of MI355X peak (mean over the headline rows)", "cores": max(r["cores"] for r in cpu_rows),
               "kind": "port", "host": host, "rows": cpu_rows}
    return {
        "metric": METRIC, "value": value, "unit": "% of MI355X peak (mean over the headline rows)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sum(r["ms_per_launch"] for r in rows), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": ",".join(dict.fromkeys(r["dtype"] for r in headline)),
        "data": "synthetic, seeded, resident in HBM: uniform fp32 copy source; N(0,1) BF16/FP16/FP64 GEMM "
                "operands; exact FP8/INT8/MXFP4 GEMM sets; exact lattices for the resident tiles; vector chain "
                "states x0 ~ U[0.5, 1) (INT8: [-4, 4])",
        "config": {"workload": "mean over " + " + ".join(r["name"] for r in headline)
                   + ("; also reported: " + ", ".join(r["name"] for r in rows if not r["in_headline"])
                      if any(not r["in_headline"] for r in rows) else ""),
                   "device": info["name"], "arch": info["arch"], "compute_units": info["compute_units"],
                   "power_cap_w": next((r["power"]["cap_w"] for r in rows if r.get("power")), None),
                   "warmup_ms_per_kernel": args.warmup_ms, "sub_batch_ms": args.sub_batch_ms,
                   "timing": "per kernel: untimed launches for >= warmup launches and >= warmup_ms, then exactly "
                             "`steps` launches with HIP events on the launch stream between sub-batches"},
        "roofline": roofline_block, "cpu_baseline": cpu, "rows": rows,
    }


def _round(value, digits=5):
    """`value` to `digits` significant digits (None and non-floats unchanged)."""
    if not isinstance(value, float) or not math.isfinite(value) or value == 0.0:
        return value
    return round(value, digits - 1 - int(math.floor(math.log10(abs(value)))))


def headline_line(document: dict, detail_path: str) -> dict:
    """The one stdout line: contract fields, roofline, a compact cpu_baseline and short rows (< MAX_LINE_BYTES)."""
    cpu = document["cpu_baseline"]
    compact_cpu = None
    if cpu:
        host = cpu.get("host") or {}
        sample = "; ".join(f"{r['name']} {_round(r['value'], 3)} {r['unit']}" for r in cpu["rows"]
                           if r["name"] in HEADLINE)
        compact_cpu = {"value": _round(cpu["value"]), "unit": cpu["unit"], "cores": cpu["cores"], "kind": cpu["kind"],
                       "sample": ("torch CPU path per headline row, bounded sample each: " + sample)[:200],
                       "host": f"{host.get('cpu_model')}, {host.get('usable_cpus')} usable CPUs"[:120]}
    rows = []
    for r in document["rows"]:
        row = {"name": r["name"], "kernel": r["kernel"], "value": _round(r["value"]), "unit": r["unit"],
               "frac": _round(r["frac"], 4), "ms_per_launch": _round(r["ms_per_launch"], 4),
               "in_headline": r["in_headline"]}
        clock = r.get("clock") or {}
        if clock.get("clock_mhz"):
            row["clock_mhz"] = round(clock["clock_mhz"])
        if "frac_at_clock" in r:
            row["frac_at_clock"] = _round(r["frac_at_clock"], 4)
        if r.get("power"):
            row["power_w"] = round(r["power"]["mean_w"])
        if "rw_bound_frac" in r:
            row["rw_bound_frac"] = _round(r["rw_bound_frac"], 4)
        rows.append(row)
    roofline_block = {key: _round(value) for key, value in document["roofline"].items()}
    line = {key: document[key] for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                           "higher_is_better", "scaling", "vs_baseline", "dtype", "data")}
    line["value"], line["ms_per_step"] = _round(line["value"]), _round(line["ms_per_step"])
    config = document["config"]
    line["config"] = {"workload": config["workload"], "device": config["device"], "arch": config["arch"],
                      "compute_units": config["compute_units"], "power_cap_w": config.get("power_cap_w")}
    line.update(roofline=roofline_block, cpu_baseline=compact_cpu, rows=rows, detail=detail_path)
    if len(json.dumps(line).encode()) > MAX_LINE_BYTES:  # never let the line outgrow what a reader keeps
        for row in line["rows"]:
            row.pop("kernel", None)
    if len(json.dumps(line).encode()) > MAX_LINE_BYTES:
        line["rows"] = [{"name": r["name"], "frac": r["frac"]} for r in line["rows"]]
    return line


if __name__ == "__main__":
    raise SystemExit(main())
