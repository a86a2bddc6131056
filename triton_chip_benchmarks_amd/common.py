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


class _Timer:
    """Event pair on the current stream; elapsed device time of one submission."""

    def __init__(self, torch):
        self.torch = torch
        self.start = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)

    def elapsed(self, submit) -> float:
        self.start.record()
        submit()
        self.end.record()
        self.torch.cuda.synchronize()
        elapsed = float(self.start.elapsed_time(self.end))
        if not math.isfinite(elapsed) or elapsed < 0:
            raise RuntimeError(f"Invalid device event time: {elapsed!r} ms")
        return elapsed


def _zero_event_error(launches=None):
    workload = f" for {launches} launches" if launches is not None else ""
    return RuntimeError(f"Invalid device event time: 0 ms{workload}; events are too coarse for this workload")


def _coarse_event_error(launches, elapsed_ms, required_ms):
    return RuntimeError(f"Device event resolution is too coarse: {launches} launches measured {elapsed_ms:g} ms, "
                        f"but at least {required_ms:g} ms is needed for a reliable peak measurement")


def _batch_samples(fn, args, use_graph):
    torch = _torch()
    stream = torch.cuda.Stream()  # default priority
    with torch.cuda.stream(stream):
        timer = _Timer(torch)

        def direct(count):
            for _ in range(count):
                fn()

        # Calibrate: grow the batch until the event pair resolves it.
        launches, saw_zero = INITIAL_CALIBRATION_LAUNCHES, False
        while True:
            elapsed = timer.elapsed(lambda: direct(launches))
            if elapsed > 0:
                break
            if launches == MAX_BATCH_LAUNCHES:
                raise _zero_event_error(launches)
            saw_zero, launches = True, min(MAX_BATCH_LAUNCHES, launches * 2)
        calibration_launches = launches
        estimate_ms = max(elapsed / launches, 0.001)
        minimum_launches = launches if saw_zero else 1
        minimum_batch_ms = elapsed * MIN_RESOLVED_EVENT_TICKS if saw_zero else 0.0
        target_ms = min(args.batch_ms, args.rep / args.rounds)
        launches = max(minimum_launches, min(MAX_BATCH_LAUNCHES, math.ceil(target_ms / estimate_ms)))
        graphs = []  # keep captured graphs alive while their replays may run

        def build_submit(count):
            if not use_graph:
                return lambda: direct(count)
            try:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    direct(count)
            except RuntimeError as exc:
                raise GraphUnavailable(f"HIP graph capture: {exc}") from exc
            graphs.append(graph)
            return graph.replay

        def time_batch(count, zero_seen=False):
            nonlocal minimum_batch_ms
            while True:
                submit = build_submit(count)
                elapsed = timer.elapsed(submit)
                if elapsed > 0 and zero_seen and minimum_batch_ms == 0:
                    minimum_batch_ms = elapsed * MIN_RESOLVED_EVENT_TICKS
                if elapsed > 0 and elapsed >= minimum_batch_ms:
                    return count, submit, elapsed
                if count == MAX_BATCH_LAUNCHES:
                    error = (_zero_event_error(count) if elapsed == 0 else
                             _coarse_event_error(count, elapsed, minimum_batch_ms))
                    if use_graph:
                        raise GraphUnavailable(f"HIP graph timing: {error}")
                    raise error
                zero_seen = zero_seen or elapsed == 0
                count = min(MAX_BATCH_LAUNCHES, count * 2)

        launches, submit, batch_ms = time_batch(launches)
        for _ in range(2):
            refined = max(minimum_launches,
                          min(MAX_BATCH_LAUNCHES, math.ceil(launches * target_ms / batch_ms)))
            if refined == launches or 0.5 * target_ms <= batch_ms <= 2 * target_ms:
                break
            graphs.clear()
            launches, submit, batch_ms = time_batch(refined)
        for _ in range(max(1, math.ceil(args.warmup / batch_ms))):
            submit()
        torch.cuda.synchronize()
        rounds = max(args.rounds, math.ceil(args.rep / batch_ms))
        batches = []
        while len(batches) < rounds:
            elapsed = timer.elapsed(submit)
            if elapsed > 0 and elapsed >= minimum_batch_ms:
                batches.append(elapsed)
                continue
            if launches == MAX_BATCH_LAUNCHES:
                error = (_zero_event_error(launches) if elapsed == 0 else
                         _coarse_event_error(launches, elapsed, minimum_batch_ms))
                if use_graph:
                    raise GraphUnavailable(f"HIP graph timing: {error}")
                raise error
            graphs.clear()
            launches, submit, batch_ms = time_batch(min(MAX_BATCH_LAUNCHES, launches * 2),
                                                    zero_seen=elapsed == 0)
            rounds = max(args.rounds, math.ceil(args.rep / batch_ms))
            batches.clear()
        torch.cuda.synchronize()
    return [elapsed / launches for elapsed in batches], {
        "launches_per_batch": launches, "batch_samples_ms": batches,
        "sample_count": len(batches), "measured_total_ms": sum(batches),
        "graph_api": "torch.cuda.CUDAGraph (HIP graph)" if use_graph else None,
        "calibration_launches": calibration_launches,
        "minimum_resolved_batch_ms": minimum_batch_ms,
    }


def measure(fn, args):
    """Device-event timing of `fn` (one kernel launch); never the host clock."""
    torch = _torch()
    fn()  # first launch outside any capture or timed sample
    torch.cuda.synchronize()
    requested = args.timing
    selected = "events" if requested == "events" else "graph"
    fallback = None
    if selected == "graph":
        try:
            samples, details = _batch_samples(fn, args, use_graph=True)
        except GraphUnavailable as exc:
            if requested == "graph":
                raise
            torch.cuda.synchronize()
            fallback, selected = str(exc), "events"
            samples, details = _batch_samples(fn, args, use_graph=False)
    else:
        samples, details = _batch_samples(fn, args, use_graph=False)
    if not samples or any(not math.isfinite(value) or value <= 0 for value in samples):
        raise RuntimeError("Invalid device timing; increase the workload/--rep")
    notice = f"Timing: {selected} via HIP events"
    if fallback:
        notice += f" (auto fallback: {fallback}; includes host dispatch gaps)"
    if getattr(args, "_timing_notice", None) != notice:
        print(notice)
        args._timing_notice = notice
    return {
        "median_ms": statistics.median(samples), "p20_ms": _quantile(samples, 0.2),
        "p80_ms": _quantile(samples, 0.8), "min_ms": min(samples), "max_ms": max(samples),
        "timing_method": selected, "timing_requested": requested,
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
