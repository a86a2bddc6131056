#!/usr/bin/env python3
"""Headline benchmark of the MI355X peak-throughput suite (one JSON line).

Metric: "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of
MI355X peak". One step is one pass of the hot path over resident synthetic
inputs - one launch of each headline kernel:
  hbm_copy    mb_copy of 2^28 fp32 (1 GiB, uniform[-1,1) from seed 0) into a
              second buffer (memory_bandwidth row);
  peak_bf16   mb_tensor_peak BF16: the resident-operand variant that loops a
              256x256x64 LDS tile 1024 times per workgroup, 2 workgroups per
              CU (tensor_bf16 row);
  peak_fp8    FP8 E4M3, 128x128x128 tiles, 2 chains, 1024 iterations, 4
              workgroups per CU (tensor_fp8 row);
  peak_mxfp4  MX FP4 E2M1 + E8M0 scales, 128x128x256 tiles, 2 chains, 1024
              iterations, 4 workgroups per CU (tensor_fp4 row).
Operands follow the reference's peak lattices (bench_tensor.py:614-672). Every
kernel's output is validated before timing with the product's own checks
(bit equality for the copy; exact float64 lattice references under the
reference's tolerance for the MFMA rows).

Timing: for each kernel in turn, W untimed warmup launches, then its K timed
launches back to back - captured once into a HIP graph and replayed - between
two torch.cuda.synchronize() calls, as the reference's batch timing does
(common.py:295-534). The output of the timed launches is checked again.
MI355X raises its clock over ~40 ms when a matrix-bound kernel follows a
memory-bound one, and the per-kernel warmup keeps that ramp out of the timed
launches. A kernel's
ms_per_launch is its batch time between two HIP events on the launch stream
over K (no event between launches, as in the reference's event batches);
ms_per_step is the sum of the kernels' batch times over K.

value = mean over the headline rows of (achieved rate / MI355X published
peak), in percent; the absolute rates are in "rows". The CPU baseline times
the oracle (numpy) on bounded samples of the same work on the host.
"""

from __future__ import annotations

import argparse
import json
import os
from pathlib import Path
import sys
import time

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of MI355X peak"
COPY_ELEMENTS = 2**28
COPY_SEED = 0
# Launch shapes chosen from the bench_bandwidth / bench_tensor sweeps on MI355X.
# One 64-lane wave per workgroup, one 16-byte vector per lane: the fastest measured
# shape on MI355X (more vectors per lane or larger workgroups lose 1-8%); streaming
# policy: nt loads, device-scope stores written through the L2 (~1% over nt stores).
COPY_CONFIG = {"block_threads": 64, "vectors_per_thread": 1, "grid_blocks": 0, "nontemporal": "stream"}
PEAK_ITERATIONS = 1024
# (tile M, N, K, chains, workgroups per CU). BF16 is the headline resident
# variant (256x256x64 tile); FP8 and MXFP4 use the fastest tiles of the bench_tensor sweep.
PEAK_SHAPES = {"bf16": (256, 256, 64, 1, 2), "fp8": (128, 128, 128, 2, 4), "fp4": (128, 128, 256, 2, 4)}
TRAFFIC_FILE = ROOT / "profiles" / "traffic_per_launch.txt"
CPU_ROW_BUDGET_S = 4.0  # host seconds per row: about 16 s of CPU work in all


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=20,
                        help="untimed launches of each kernel right before its timed ones (default: 20)")
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="Skip the timed CPU baseline leg (it is on by default)")
    parser.add_argument("--rows", nargs="+", help="Subset of headline rows: hbm_copy peak_bf16 peak_fp8 peak_mxfp4")
    return parser.parse_args(argv)


def traffic_table() -> dict[str, float]:
    """Measured HBM bytes per launch by kernel (from committed rocprofv3 counter runs)."""
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


def _best_of(fn, budget_s):
    """Best wall time of repeated host calls within a time budget (CPU leg only)."""
    fn()
    best, spent = None, 0.0
    while spent < budget_s or best is None:
        start = time.perf_counter()
        fn()
        elapsed = time.perf_counter() - start
        spent += elapsed
        best = elapsed if best is None else min(best, elapsed)
    return best


class CopyWorkload:
    """memory_bandwidth row: 1 GiB fp32 device-to-device copy."""

    name, dtype, metric_key, unit, bound = "hbm_copy", "f32", "memory_bandwidth", "GB/s", "hbm"

    def __init__(self, torch):
        from triton_chip_benchmarks_amd import bench_bandwidth

        self.torch = torch
        self.launcher = bench_bandwidth.launch_copy
        generator = torch.Generator(device="cuda")
        generator.manual_seed(COPY_SEED)
        self.src = torch.empty(COPY_ELEMENTS, device="cuda", dtype=torch.float32).uniform_(-1, 1, generator=generator)
        self.dst = torch.empty_like(self.src)
        self.work = 2 * self.src.numel() * 4  # algorithmic bytes: read + write (bench_bandwidth.py:212)
        self.kernel = f"copy_dwordx4_vpt{COPY_CONFIG['vectors_per_thread']}" + bench_bandwidth.POLICY_SUFFIX[
            bench_bandwidth.copy_policy(COPY_CONFIG["nontemporal"])]
        self.config = {"elements": COPY_ELEMENTS, "dtype": "fp32", **COPY_CONFIG}

    def launch(self):
        self.launcher(self.src, self.dst, COPY_CONFIG["block_threads"], COPY_CONFIG["vectors_per_thread"],
                      COPY_CONFIG["grid_blocks"], COPY_CONFIG["nontemporal"])

    def poison(self):
        self.dst.fill_(float("nan"))

    def check(self):
        self.torch.cuda.synchronize()
        if not self.torch.equal(self.src.view(self.torch.int32), self.dst.view(self.torch.int32)):
            raise AssertionError("copy output differs from its source")
        return "bit-exact: every word of the 1 GiB destination equals the source"

    def validate(self):
        self.poison()
        self.launch()
        return self.check()

    def rate(self, ms):
        return self.work / (ms * 1e6)  # GB/s

    def cpu_rate(self):
        """oracle.memory.copy of a 256 MiB host sample."""
        import numpy as np

        from oracle import memory

        sample = np.random.default_rng(COPY_SEED).uniform(-1, 1, size=2**26).astype(np.float32)
        best = _best_of(lambda: memory.copy(sample), CPU_ROW_BUDGET_S)
        return 2 * sample.nbytes / best / 1e9, 1, "oracle.memory.copy (numpy) of 2^26 fp32 (256 MiB)"


class PeakWorkload:
    """tensor_<dtype> row: resident-operand MFMA peak kernel."""

    unit, bound = "TFLOP/s", "mfma"

    def __init__(self, torch, dtype, compute_units):
        from triton_chip_benchmarks_amd import _native, bench_tensor

        self.torch, self.bt, self.dtype = torch, bench_tensor, dtype
        self.name = "peak_mxfp4" if dtype == "fp4" else f"peak_{dtype}"
        self.metric_key = f"tensor_{dtype}"
        m, n, k, chains, per_cu = PEAK_SHAPES[dtype]
        blocks = per_cu * compute_units
        self.config = next(c for c in _native.peak_configs(dtype)
                           if (c["tile_m"], c["tile_n"], c["tile_k"]) == (m, n, k) and c["chains"] == chains
                           and not c["b_nk"])
        self.kernel = _native.peak_kernel_name(dtype, self.config)
        self.blocks = blocks
        if dtype == "fp4":
            self.a, self.b, self.c, self.scales, self.values = bench_tensor.fp4_peak_inputs(blocks, self.config, "cuda")
        else:
            self.a, self.b, self.c, b_logical = bench_tensor.peak_inputs(blocks, self.config, dtype, "cuda")
            self.scales, self.values = None, (self.a, b_logical)
        self.work = 2 * m * n * k * PEAK_ITERATIONS * self.config["chains"] * blocks  # bench_tensor.py:1242
        self.dtype_label = {"bf16": "bf16", "fp8": "fp8_e4m3", "fp4": "mxfp4_e2m1"}[dtype]
        self.config_summary = {"tile": f"{m}x{n}x{k}", "chains": self.config["chains"], "blocks": blocks,
                               "blocks_per_cu": per_cu, "iterations": PEAK_ITERATIONS, "b_layout": "kn"}

    def launch(self):
        self.bt.launch_peak(self.dtype, self.config, self.a, self.b, self.c, PEAK_ITERATIONS, self.scales)

    def poison(self):
        self.c.fill_(float("nan"))

    def check(self):
        reference = self.bt.exact_reference(self.values[0], self.values[1], PEAK_ITERATIONS, self.torch.float32)
        self.torch.cuda.synchronize()
        result = self.bt.validate_peak(self.c, reference, self.dtype, self.config["tile_k"], PEAK_ITERATIONS)
        return (f"every output within atol {result['atol']:.3g} of the exact float64 lattice reference "
                f"(max error {result['max_abs_error']:.3g})")

    def validate(self):
        self.poison()
        self.launch()
        return self.check()

    def rate(self, ms):
        return self.work / (ms * 1e9)  # TFLOP/s

    def cpu_rate(self):
        """The same tile products on the host: oracle.tensor.peak_reference over a block sample."""
        import numpy as np

        from oracle import tensor as ot

        m, n, k, chains, _ = PEAK_SHAPES[self.dtype]
        rng = np.random.default_rng(0)
        blocks = 64
        a = ot.ternary_lattice(rng, (blocks, m, k))
        b = ot.ternary_lattice(rng, (chains, blocks, k, n))
        # One host iteration = every chain's tile product of every sampled block.
        best = _best_of(lambda: ot.peak_reference(a, b, 1), CPU_ROW_BUDGET_S)
        flops = 2 * m * n * k * chains * blocks
        from triton_chip_benchmarks_amd.cpu_baseline import blas_threads

        return flops / best / 1e12, blas_threads(), (
            f"oracle.tensor.peak_reference (numpy float64 matmul) of {blocks} blocks x {chains} chain(s) of "
            f"{m}x{n}x{k} tiles, best repeat within {CPU_ROW_BUDGET_S:g} s")


def host_description(torch) -> dict:
    """The host the CPU baseline ran on (model, CPUs, torch and BLAS threads)."""
    del torch
    from triton_chip_benchmarks_amd.cpu_baseline import host_description as describe

    return describe()


def build_workloads(torch, selected, compute_units):
    workloads = [CopyWorkload(torch)] + [PeakWorkload(torch, d, compute_units) for d in ("bf16", "fp8", "fp4")]
    if selected:
        unknown = set(selected) - {w.name for w in workloads}
        if unknown:
            raise SystemExit(f"unknown rows: {', '.join(sorted(unknown))}")
        workloads = [w for w in workloads if w.name in selected]
    return workloads


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported. Every headline kernel runs "
              "on a single GPU, and a multi-GPU figure would be the sum of independent per-GPU rates, which "
              "this build does not launch.", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0:
        print("--steps must be positive and --warmup non-negative", file=sys.stderr)
        return 2
    import torch

    from triton_chip_benchmarks_amd import _native, roofline
    from triton_chip_benchmarks_amd.common import require_gpu

    require_gpu(0)
    info = _native.device_query(0)
    workloads = build_workloads(torch, args.rows, info["compute_units"])
    checks = {w.name: w.validate() for w in workloads}

    stream = torch.cuda.current_stream()
    batch_ms, timing_modes = [], []
    for w in workloads:
        # W untimed warmup launches right before the kernel's K timed ones, so
        # the clock has settled at this kernel's load when timing starts.
        for _ in range(args.warmup):
            w.launch()
        torch.cuda.synchronize()
        # The K launches are captured once into a HIP graph and replayed, as the
        # reference's event batches are (common.py:311-361); without graph
        # support they are launched directly.
        submit, mode = None, "hip_graph"
        try:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(args.steps):
                    w.launch()
            graph.replay()  # untimed: the first replay uploads the graph
            torch.cuda.synchronize()
            submit = graph.replay
        except RuntimeError:
            torch.cuda.synchronize()
            mode = "direct_launches"

            def submit(w=w):
                for _ in range(args.steps):
                    w.launch()
        w.poison()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        submit()
        end.record(stream)
        torch.cuda.synchronize()
        batch_ms.append(start.elapsed_time(end))
        timing_modes.append(mode)
        w.check()  # raises if the timed launches' output is wrong
        checks[w.name] += "; the same check passed again on the timed launches' output"
    total_ms = sum(batch_ms)

    traffic = traffic_table()
    rows = []
    for index, w in enumerate(workloads):
        average = batch_ms[index] / args.steps
        achieved = w.rate(average)
        peak, _unit, basis = roofline.PEAKS[w.metric_key]
        rows.append({"row": w.metric_key, "name": w.name, "kernel": w.kernel, "value": achieved, "unit": w.unit,
                     "ms_per_launch": average, "peak": peak, "frac": achieved / peak,
                     "peak_basis": basis, "bound": w.bound, "algorithmic_work_per_launch": w.work,
                     "work_unit": "bytes" if w.bound == "hbm" else "flop",
                     "traffic_bytes_per_launch": traffic.get(w.kernel),
                     "config": getattr(w, "config_summary", None) or w.config, "validation": checks[w.name]})
    value = 100.0 * sum(row["frac"] for row in rows) / len(rows)
    dominant = max(rows, key=lambda row: row["ms_per_launch"])
    roofline_block = {"bound": dominant["bound"], "kernel": dominant["kernel"], "row": dominant["row"],
                      "achieved": dominant["value"], "peak": dominant["peak"], "unit": dominant["unit"],
                      "frac": dominant["frac"], "traffic": dominant["traffic_bytes_per_launch"],
                      "algorithmic_work_per_launch": dominant["algorithmic_work_per_launch"],
                      "ms_per_launch": dominant["ms_per_launch"]}
    cpu = None
    if not args.no_cpu_baseline:
        cpu_rows = []
        for w in workloads:
            cpu_value, cores, sample = w.cpu_rate()
            peak = roofline.PEAKS[w.metric_key][0]
            cpu_rows.append({"row": w.metric_key, "value": cpu_value, "unit": w.unit, "cores": cores,
                             "sample": sample, "frac_of_mi355x_peak": cpu_value / peak})
        cpu = {"value": 100.0 * sum(r["frac_of_mi355x_peak"] for r in cpu_rows) / len(cpu_rows),
               "unit": "% of MI355X peak (mean over headline rows)",
               "cores": max(r["cores"] for r in cpu_rows), "kind": "port",
               "sample": "; ".join(f"{r['row']}: {r['sample']}" for r in cpu_rows),
               "host_cpu_count": os.cpu_count(), "host": host_description(torch), "rows": cpu_rows}
    line = {
        "metric": METRIC, "value": value, "unit": "% of MI355X peak (mean over headline rows)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": total_ms / args.steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ",".join(getattr(w, "dtype_label", w.dtype) for w in workloads),
        "data": "synthetic: seeded uniform fp32 copy source; exact-lattice MFMA operands, resident in HBM",
        "config": {"workload": " + ".join(w.name for w in workloads), "device": info["name"], "arch": info["arch"],
                   "compute_units": info["compute_units"], "peak_iterations": PEAK_ITERATIONS,
                   "copy_elements": COPY_ELEMENTS,
                   "timing": "per kernel: W warmup launches, then K launches replayed from one HIP graph "
                             "between two HIP events" if all(m == "hip_graph" for m in timing_modes)
                             else "per kernel: W warmup launches, then K direct launches between two HIP events"},
        "roofline": roofline_block, "cpu_baseline": cpu, "rows": rows,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
