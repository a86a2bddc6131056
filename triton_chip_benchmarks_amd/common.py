"""Device setup, device-event timing and result documents for the MI355X suite.

Host code uses PyTorch-ROCm only for allocation, streams and HIP events; every
measured kernel is a launch of libmi355x_bench.so. Timing follows the
reference harness (common.py:295-534): batches of R back-to-back launches
bracketed by device events, optionally captured into one HIP graph, reporting
the minimum and median batch-average time. The host clock is never used for
device time.
"""

from __future__ import annotations

import argparse
from datetime import datetime, timezone
import json
import math
import os
from pathlib import Path
import statistics

from . import _native, roofline

GFX950 = "gfx950"


def positive_int(value):
    number = int(value)
    if number <= 0:
        raise argparse.ArgumentTypeError("must be a positive integer")
    return number


def positive_float(value):
    number = float(value)
    if not math.isfinite(number) or number <= 0:
        raise argparse.ArgumentTypeError("must be a finite positive number")
    return number


def add_common_arguments(parser):
    """The reference's shared flags (common.py:117-133), same names and defaults."""
    parser.add_argument("--device", type=int, default=0, help="HIP device index (default: 0)")
    parser.add_argument("--warmup", type=positive_float, default=100,
                        help="Approximate device warmup duration in ms (default: 100)")
    parser.add_argument("--rep", type=positive_float, default=200,
                        help="Approximate measurement budget in ms (default: 200)")
    parser.add_argument("--timing", choices=("auto", "graph", "events"), default="auto",
                        help="Auto uses a HIP graph of each batch, falling back to event batches")
    parser.add_argument("--batch-ms", type=positive_float, default=10,
                        help="Target batch duration in ms (default: 10)")
    parser.add_argument("--rounds", type=positive_int, default=10,
                        help="Minimum number of measured batches (default: 10)")
    parser.add_argument("--compute-units", type=positive_int,
                        help="Override the compute-unit count reported by the runtime")
    parser.add_argument("--l2-mib", type=positive_float,
                        help="Last-level cache capacity in MiB for the HBM-sized buffer rule "
                             "(default: the MI355X 256 MiB Infinity Cache)")
    parser.add_argument("--output", type=Path, help="Save metadata and all samples as JSON")
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="Skip timing the reference's host computation beside the device rate")


def _torch():
    import torch

    return torch


def require_gpu(device: int = 0):
    """Select `device`, failing loudly when no HIP device or no library is present."""
    torch = _torch()
    if not torch.cuda.is_available():
        raise SystemExit("No HIP device is visible; this suite measures an AMD Instinct MI355X (gfx950)")
    count = torch.cuda.device_count()
    if not 0 <= device < count:
        raise SystemExit(f"Invalid --device {device}; available indices: 0..{count - 1}")
    torch.cuda.set_device(device)
    _native.load()
    return torch.device("cuda", device)


def get_device(args):
    index = args if isinstance(args, int) else args.device
    return _torch().device("cuda", index)


def available_memory_bytes():
    try:
        return int(_torch().cuda.mem_get_info()[0])
    except RuntimeError:
        return None


def setup_device(args):
    """Device metadata block; mirrors the reference's keys (common.py:266-284)."""
    torch = _torch()
    require_gpu(args.device)
    torch.manual_seed(0)
    info = _native.device_query(args.device)
    arch = info["arch"].split(":")[0]
    units, unit_source = info["compute_units"], "hipDeviceProp_t.multiProcessorCount"
    if getattr(args, "compute_units", None) is not None:
        units, unit_source = args.compute_units, "--compute-units"
    if getattr(args, "l2_mib", None) is not None:
        llc, llc_source = int(args.l2_mib * 2**20), "--l2-mib"
    elif arch == GFX950:
        llc = roofline.INFINITY_CACHE_BYTES
        llc_source = ("MI355X Infinity Cache (256 MiB last-level cache); HIP reports "
                      f"{info['l2_cache_bytes'] / 2**20:g} MiB, one XCD's L2")
    else:
        llc, llc_source = info["l2_cache_bytes"], "hipDeviceProp_t.l2CacheSize"
    total = info["total_memory_bytes"]
    metadata = {
        "device_index": args.device, "device_type": "cuda", "device_name": info["name"],
        "vendor_name": "amd", "backend": "hip", "architecture": arch,
        "gcn_arch_name": info["arch"],
        "sm_count": units, "compute_units_source": unit_source,
        "total_memory_bytes": int(total) if total else None,
        "memory_capacity_gib": total / 2**30 if total else None,
        "l2_cache_bytes": int(llc), "l2_cache_source": llc_source,
        "hip_l2_cache_bytes": info["l2_cache_bytes"],
        "lds_bytes_per_cu": info["lds_bytes_per_cu"],
        "wavefront_size": info["wavefront_size"],
        "peak_clock_mhz": info["clock_khz"] / 1000,
        "memory_clock_mhz": info["memory_clock_khz"] / 1000,
        "memory_bus_bits": info["memory_bus_bits"],
        "supports_fp64": True, "supports_bf16": True,
        "torch_version": torch.__version__,
        "hip_version": getattr(torch.version, "hip", None),
        "native_library": str(_native.LIBRARY_PATH),
        "device_api": "libmi355x_bench.so (ctypes) + torch.cuda streams/events",
    }
    if arch != GFX950:
        raise SystemExit(f"This suite's kernels are built for {GFX950}; device {args.device} is {arch}")
    print(f"Device cuda:{args.device}: {info['name']} | arch={info['arch']} | compute units={units} | "
          f"memory={total / 2**30:.1f} GiB | clock={info['clock_khz'] / 1000:.0f} MHz")
    print(f"PyTorch {torch.__version__} (HIP {metadata['hip_version']}); library {_native.LIBRARY_PATH.name}; "
          f"timing={args.timing}, warmup={args.warmup:g} ms, rep={args.rep:g} ms")
    return metadata


def _quantile(samples, quantile):
    ordered = sorted(samples)
    position = (len(ordered) - 1) * quantile
    lower, upper = math.floor(position), math.ceil(position)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


class GraphUnavailable(RuntimeError):
    """HIP graph capture or replay is not usable for this launch."""


INITIAL_CALIBRATION_LAUNCHES = 5
MAX_BATCH_LAUNCHES = 2048
MIN_RESOLVED_EVENT_TICKS = 20


class _EventClock:
    """Device time of one submission, between two HIP events on the current stream."""

    def __init__(self, torch):
        self.torch = torch
        self.begin = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)

    def time(self, submit) -> float:
        self.begin.record()
        submit()
        self.end.record()
        self.torch.cuda.synchronize()
        elapsed = float(self.begin.elapsed_time(self.end))
        if not (math.isfinite(elapsed) and elapsed >= 0):
            raise RuntimeError(f"Invalid device event time: {elapsed!r} ms")
        return elapsed


class _Submitter:
    """Callables that issue `count` launches of fn: a captured HIP graph's replay, or direct launches.

    Captured graphs stay cached (alive) for the life of the sampler, since a
    replay may still be in flight when a new batch size is captured.
    """

    def __init__(self, torch, fn, use_graph: bool):
        self.torch, self.fn, self.use_graph = torch, fn, use_graph
        self.graphs = {}

    def direct(self, count):
        def submit():
            for _ in range(count):
                self.fn()
        return submit

    def __call__(self, count):
        if not self.use_graph:
            return self.direct(count)
        if count not in self.graphs:
            try:
                graph = self.torch.cuda.CUDAGraph()
                with self.torch.cuda.graph(graph):
                    self.direct(count)()
            except RuntimeError as exc:
                raise GraphUnavailable(f"HIP graph capture: {exc}") from exc
            self.graphs[count] = graph
        return self.graphs[count].replay


class _Sampler:
    """Batch-average device time per launch, the reference's measurement policy (common.py:394-534).

    1. Probe: direct launches, doubling from INITIAL_CALIBRATION_LAUNCHES until
       the event pair resolves them. If a probe read 0 ms the timer is coarse:
       its first positive reading counts as one tick and every batch must then
       span MIN_RESOLVED_EVENT_TICKS of them (and at least the probe's launches).
    2. Size: launches per batch for min(batch_ms, rep / rounds), corrected at
       most twice while a measured batch is off that target by more than 2x.
    3. Warm: whole batches for at least --warmup ms.
    4. Sample: at least --rounds batches and --rep ms. A batch that reads 0 or
       under the floor doubles the batch size and restarts the sampling, so all
       samples share one denominator.
    """

    def __init__(self, torch, fn, args, use_graph: bool):
        self.torch, self.args, self.use_graph = torch, args, use_graph
        self.clock = _EventClock(torch)
        self.batches = _Submitter(torch, fn, use_graph)
        self.floor_ms = 0.0
        self.min_launches = 1
        self.coarse = False

    def _failure(self, launches, elapsed):
        if elapsed == 0:
            error = RuntimeError(f"Invalid device event time: 0 ms for {launches} launches; "
                                 "events are too coarse for this workload")
        else:
            error = RuntimeError(f"Device event resolution is too coarse: {launches} launches measured "
                                 f"{elapsed:g} ms, but at least {self.floor_ms:g} ms is needed for a "
                                 "reliable peak measurement")
        return GraphUnavailable(f"HIP graph timing: {error}") if self.use_graph else error

    def probe(self):
        launches = INITIAL_CALIBRATION_LAUNCHES
        while True:
            elapsed = self.clock.time(self.batches.direct(launches))
            if elapsed > 0:
                break
            if launches >= MAX_BATCH_LAUNCHES:
                raise RuntimeError(f"Invalid device event time: 0 ms for {launches} launches; "
                                   "events are too coarse for this workload")
            self.coarse, launches = True, min(MAX_BATCH_LAUNCHES, 2 * launches)
        if self.coarse:
            self.floor_ms, self.min_launches = elapsed * MIN_RESOLVED_EVENT_TICKS, launches
        return launches, max(elapsed / launches, 0.001)

    def resolve(self, launches):
        """(launches, submit, ms) of the first batch size from `launches` up whose time resolves."""
        while True:
            submit = self.batches(launches)
            elapsed = self.clock.time(submit)
            if elapsed == 0 and not self.coarse:
                self.coarse = True  # floor set by the next positive reading
            elif elapsed > 0 and self.coarse and self.floor_ms == 0:
                self.floor_ms = elapsed * MIN_RESOLVED_EVENT_TICKS
            if elapsed > 0 and elapsed >= self.floor_ms:
                return launches, submit, elapsed
            if launches >= MAX_BATCH_LAUNCHES:
                raise self._failure(launches, elapsed)
            launches = min(MAX_BATCH_LAUNCHES, 2 * launches)

    def bounded(self, launches):
        return max(self.min_launches, min(MAX_BATCH_LAUNCHES, launches))

    def run(self):
        args = self.args
        probe_launches, per_launch = self.probe()
        target = min(args.batch_ms, args.rep / args.rounds)
        launches, submit, batch_ms = self.resolve(self.bounded(math.ceil(target / per_launch)))
        for _ in range(2):
            if 0.5 * target <= batch_ms <= 2 * target:
                break
            resized = self.bounded(math.ceil(launches * target / batch_ms))
            if resized == launches:
                break
            launches, submit, batch_ms = self.resolve(resized)
        for _ in range(max(1, math.ceil(args.warmup / batch_ms))):
            submit()
        self.torch.cuda.synchronize()
        samples = []
        wanted = max(args.rounds, math.ceil(args.rep / batch_ms))
        while len(samples) < wanted:
            elapsed = self.clock.time(submit)
            if elapsed > 0 and elapsed >= self.floor_ms:
                samples.append(elapsed)
                continue
            if launches >= MAX_BATCH_LAUNCHES:
                raise self._failure(launches, elapsed)
            if elapsed == 0 and self.floor_ms == 0:
                self.coarse = True
            launches, submit, batch_ms = self.resolve(min(MAX_BATCH_LAUNCHES, 2 * launches))
            wanted = max(args.rounds, math.ceil(args.rep / batch_ms))
            samples = []
        self.torch.cuda.synchronize()
        return [ms / launches for ms in samples], {
            "launches_per_batch": launches, "batch_samples_ms": samples, "sample_count": len(samples),
            "measured_total_ms": sum(samples),
            "graph_api": "torch.cuda.CUDAGraph (HIP graph)" if self.use_graph else None,
            "calibration_launches": probe_launches, "minimum_resolved_batch_ms": self.floor_ms,
        }


def _sample(fn, args, use_graph):
    torch = _torch()
    with torch.cuda.stream(torch.cuda.Stream()):  # a private stream at the default priority
        return _Sampler(torch, fn, args, use_graph).run()


def measure(fn, args):
    """Device-event timing of `fn` (one kernel launch); never the host clock.

    --timing graph or auto time HIP-graph replays; auto falls back to direct
    event batches (recording why) when capture or graph timing is unusable.
    """
    torch = _torch()
    fn()  # one launch outside any capture or timed sample
    torch.cuda.synchronize()
    requested = args.timing
    method, fallback = ("events" if requested == "events" else "graph"), None
    if method == "graph":
        try:
            samples, details = _sample(fn, args, use_graph=True)
        except GraphUnavailable as exc:
            if requested == "graph":
                raise
            torch.cuda.synchronize()
            method, fallback = "events", str(exc)
            samples, details = _sample(fn, args, use_graph=False)
    else:
        samples, details = _sample(fn, args, use_graph=False)
    if not samples or not all(math.isfinite(value) and value > 0 for value in samples):
        raise RuntimeError("Invalid device timing; increase the workload/--rep")
    notice = f"Timing: {method} via HIP events" + (
        f" (auto fallback: {fallback}; includes host dispatch gaps)" if fallback else "")
    if getattr(args, "_timing_notice", None) != notice:
        print(notice)
        args._timing_notice = notice
    return {
        "median_ms": statistics.median(samples), "p20_ms": _quantile(samples, 0.2),
        "p80_ms": _quantile(samples, 0.8), "min_ms": min(samples), "max_ms": max(samples),
        "timing_method": method, "timing_requested": requested,
        "timing_fallback_reason": fallback, "samples_ms_per_launch": samples, **details,
    }


def _serialized_arguments(args):
    return {key: str(value) if isinstance(value, Path) else value
            for key, value in vars(args).items() if not key.startswith("_")}


def _write_document(args, document):
    if getattr(args, "output", None) is None:
        return
    args.output.parent.mkdir(parents=True, exist_ok=True)
    temporary = args.output.with_name(args.output.name + ".tmp")
    temporary.write_text(json.dumps(document, indent=2, ensure_ascii=False, allow_nan=False) + "\n")
    os.replace(temporary, args.output)
    print(f"JSON: {args.output.resolve()}")


def _emit_no_measurement(name, metadata, args, reason, status, *, details=None):
    document = {"benchmark": name, "status": status, "reason": str(reason),
                "timestamp_utc": datetime.now(timezone.utc).isoformat(), "device": metadata,
                "arguments": _serialized_arguments(args), "results": []}
    if details is not None:
        document["details"] = details
    print(f"{status.upper()}: {reason}")
    _write_document(args, document)
    return document


def emit_unsupported(name, metadata, args, reason, *, details=None):
    """An explicit device or instruction-set capability rejection."""
    return _emit_no_measurement(name, metadata, args, reason, "unsupported", details=details)


def emit_not_implemented(name, metadata, args, reason, *, details=None):
    """A gap in this benchmark, not a statement about the chip."""
    return _emit_no_measurement(name, metadata, args, reason, "not_implemented", details=details)


def emit_results(name, metadata, args, rows, *, cpu_baseline=None):
    if not rows:
        raise RuntimeError("No valid measurements were produced")
    methods = sorted({row["timing_method"] for row in rows if "timing_method" in row})
    document = {
        "benchmark": name, "status": "ok",
        "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "device": metadata, "arguments": _serialized_arguments(args),
        "timing": {
            "provider": "torch.cuda.Event (HIP events) on the launch stream of libmi355x_bench.so",
            "requested": args.timing, "methods_used": methods,
            "method": "device events around batches; elapsed / actual launch count; no cache flush",
            "peak_statistic": "minimum sampled batch-average device time",
            "sustained_statistic": "median sampled batch-average device time",
            "includes": "kernel work, device scheduling and amortized event overhead; "
                        "events mode additionally includes host dispatch gaps",
            "excludes": "compilation, allocation, initialization, validation, capture and warmup",
        },
        "results": rows,
    }
    if cpu_baseline is not None:
        document["cpu_baseline"] = cpu_baseline
    _write_document(args, document)
    return document
