#!/usr/bin/env python3
"""Headline benchmark of the MI355X peak-throughput suite (one JSON line).

Metric: "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of
MI355X peak". One step is one pass of the hot path over resident synthetic
inputs: one launch of each headline kernel,
  - HBM copy of 2^28 fp32 (1 GiB, uniform[-1,1) from a seed) into a second buffer,
  - the resident-operand MFMA peak kernels (BF16, FP8 E4M3, MXFP4) when built.
Every kernel's output is checked against the CPU oracle before timing. The K
timed steps are bracketed by torch.cuda.synchronize(); per-kernel durations come
from HIP events recorded around each launch on the launch stream.

value = mean over the headline rows of (achieved rate / MI355X published peak),
in percent. The per-row absolute rates are in "rows".
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
# Copy launch shape chosen by the bench_bandwidth sweep on MI355X.
COPY_CONFIG = {"block_threads": 256, "vectors_per_thread": 1, "grid_blocks": 0, "nontemporal": True}
TRAFFIC_FILE = ROOT / "profiles" / "traffic_per_launch.txt"


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="Skip the timed CPU baseline leg (it is on by default)")
    parser.add_argument("--rows", nargs="+", help="Subset of headline rows to run")
    return parser.parse_args(argv)


def _traffic_table() -> dict[str, float]:
    """Measured HBM bytes per launch by kernel, from committed rocprofv3 summaries."""
    table = {}
    if TRAFFIC_FILE.exists():
        for line in TRAFFIC_FILE.read_text().splitlines():
            line = line.strip()
            if not line or line.startswith("#") or "=" not in line:
                continue
            key, value = (part.strip() for part in line.split("=", 1))
            try:
                table[key] = float(value)
            except ValueError:
                continue
    return table


class CopyWorkload:
    """memory_bandwidth row: 1 GiB fp32 device-to-device copy."""

    name = "hbm_copy"
    dtype = "f32"
    metric_key = "memory_bandwidth"
    unit = "GB/s"
    bound = "hbm"

    def __init__(self, torch):
        from triton_chip_benchmarks_amd import bench_bandwidth

        self.torch = torch
        self.launcher = bench_bandwidth.launch_copy
        generator = torch.Generator(device="cuda")
        generator.manual_seed(COPY_SEED)
        self.src = torch.empty(COPY_ELEMENTS, device="cuda", dtype=torch.float32).uniform_(-1, 1, generator=generator)
        self.dst = torch.empty_like(self.src)
        self.work = 2 * self.src.numel() * 4  # algorithmic bytes: read + write (bench_bandwidth.py:212)
        self.kernel = f"copy_dwordx4_vpt{COPY_CONFIG['vectors_per_thread']}" + (
            "_nt" if COPY_CONFIG["nontemporal"] else "")

    def launch(self):
        self.launcher(self.src, self.dst, COPY_CONFIG["block_threads"], COPY_CONFIG["vectors_per_thread"],
                      COPY_CONFIG["grid_blocks"], COPY_CONFIG["nontemporal"])

    def validate(self):
        from oracle import memory

        self.dst.fill_(float("nan"))
        self.launch()
        self.torch.cuda.synchronize()
        # Bit-exact: compare raw bits on the device, then an oracle sample on the host.
        if not self.torch.equal(self.src.view(self.torch.int32), self.dst.view(self.torch.int32)):
            raise AssertionError("copy output differs from source")
        sample = self.src[:1 << 20].cpu().numpy()
        expected = memory.copy(sample)
        if not (self.dst[:1 << 20].cpu().numpy().view("u4") == expected.view("u4")).all():
            raise AssertionError("copy sample differs from the oracle")
        return "bit-exact: full buffer on device, 1 Mi-element sample against oracle.memory.copy"

    def rate(self, ms_per_launch):
        return self.work / (ms_per_launch * 1e6)  # GB/s

    def cpu_baseline(self):
        """oracle.memory.copy of a 256 MiB host sample, best of 5 (bounded ~1 s)."""
        import numpy as np

        from oracle import memory

        sample = np.random.default_rng(COPY_SEED).uniform(-1, 1, size=2**26).astype(np.float32)
        memory.copy(sample)
        best = None
        for _ in range(5):
            start = time.perf_counter()
            memory.copy(sample)
            elapsed = time.perf_counter() - start
            best = elapsed if best is None else min(best, elapsed)
        return {"value": 2 * sample.nbytes / best / 1e9, "unit": "GB/s",
                "sample": "numpy copy (oracle.memory.copy) of 2^26 fp32 (256 MiB) on the host, best of 5"}


def build_workloads(torch, selected):
    workloads = [CopyWorkload(torch)]
    try:
        from triton_chip_benchmarks_amd import headline
    except ImportError:
        headline = None
    if headline is not None:
        workloads += headline.peak_workloads(torch)
    if selected:
        workloads = [w for w in workloads if w.name in selected]
    return workloads


def main(argv=None):
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported. Every headline kernel "
              "runs on a single GPU; a multi-GPU figure would be the sum of independent per-GPU rates, "
              "which this build does not launch.", file=sys.stderr)
        return 2
    if args.steps <= 0 or args.warmup < 0:
        print("--steps must be positive and --warmup non-negative", file=sys.stderr)
        return 2
    import torch

    from triton_chip_benchmarks_amd import _native, roofline
    from triton_chip_benchmarks_amd.common import require_gpu

    require_gpu(0)
    info = _native.device_query(0)
    workloads = build_workloads(torch, args.rows)
    checks = {w.name: w.validate() for w in workloads}
    for _ in range(args.warmup):
        for w in workloads:
            w.launch()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(workloads) + 1)]
              for _ in range(args.steps)]
    total_start, total_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    total_start.record(stream)
    for step in range(args.steps):
        events[step][0].record(stream)
        for index, w in enumerate(workloads):
            w.launch()
            events[step][index + 1].record(stream)
    total_end.record(stream)
    torch.cuda.synchronize()
    total_ms = total_start.elapsed_time(total_end)

    traffic = _traffic_table()
    rows = []
    for index, w in enumerate(workloads):
        durations = [events[s][index].elapsed_time(events[s][index + 1]) for s in range(args.steps)]
        average = sum(durations) / len(durations)
        achieved = w.rate(average)
        peak, unit, basis = roofline.PEAKS[w.metric_key]
        rows.append({"row": w.metric_key, "kernel": w.kernel, "value": achieved, "unit": w.unit,
                     "ms_per_launch": average, "min_ms": min(durations), "peak": peak,
                     "frac": achieved / peak, "peak_basis": basis, "bound": w.bound,
                     "work_per_launch": w.work, "validation": checks[w.name],
                     "traffic_bytes_per_launch": traffic.get(w.kernel)})
    value = 100.0 * sum(row["frac"] for row in rows) / len(rows)
    dominant = max(rows, key=lambda row: row["ms_per_launch"])
    roofline_block = {
        "bound": dominant["bound"], "kernel": dominant["kernel"],
        "achieved": dominant["value"],
        "peak": dominant["peak"], "unit": dominant["unit"], "frac": dominant["frac"],
        "traffic": dominant["traffic_bytes_per_launch"],
        "work_per_launch": dominant["work_per_launch"],
    }
    cpu = None
    if not args.no_cpu_baseline:
        baseline = workloads[0].cpu_baseline()
        cores = 1  # numpy copy is single-threaded
        cpu = {"value": baseline["value"], "unit": baseline["unit"], "cores": cores, "kind": "port",
               "sample": baseline["sample"], "host_cpu_count": os.cpu_count(),
               "gpu_over_cpu": rows[0]["value"] / baseline["value"] if rows[0]["unit"] == baseline["unit"] else None}
    line = {
        "metric": METRIC, "value": value, "unit": "% of MI355X peak (mean over headline rows)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": total_ms / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": ",".join(sorted({w.dtype for w in workloads})),
        "data": "synthetic (seeded uniform / exact-lattice operands, resident in HBM)",
        "config": {"workload": " + ".join(w.name for w in workloads),
                   "copy_elements": COPY_ELEMENTS, "device": info["name"], "arch": info["arch"],
                   "compute_units": info["compute_units"]},
        "roofline": roofline_block, "cpu_baseline": cpu, "rows": rows,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
