#!/usr/bin/env python3
"""Run the complete 17-row chip metric table on one MI355X, one child per metric.

Same CLI, child commands and report document as the reference's
bench_suite.py (bench_suite.py:72-199): every metric runs in an isolated child
process with a timeout, stale child output is deleted before the run, the
report is checkpointed atomically after every metric, and a failed child can
never reuse an old success.
"""

from __future__ import annotations

import argparse
from datetime import datetime, timezone
import json
from pathlib import Path
import subprocess
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd.common import positive_float, positive_int
    from triton_chip_benchmarks_amd.suite_report import METRICS, empty_metric, format_table, summarize
else:
    from .common import positive_float, positive_int
    from .suite_report import METRICS, empty_metric, format_table, summarize

ROOT = Path(__file__).resolve().parent.parent
MEASUREMENT_POLICY = ("Highest observed valid throughput; median from the same configuration. "
                      "Capacity is reported device capacity. Bandwidth is effective copy read+write "
                      "traffic with HBM-sized buffers; read rates are auxiliary details. "
                      "Unsupported and not-implemented metrics have no numeric value; "
                      "errors do not imply unsupported hardware.")


def build_parser():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--device", type=int, default=0)
    parser.add_argument("--timing", choices=("auto", "graph", "events"), default="auto")
    parser.add_argument("--warmup", type=positive_float, default=100)
    parser.add_argument("--rep", type=positive_float, default=200)
    parser.add_argument("--batch-ms", type=positive_float, default=10)
    parser.add_argument("--rounds", type=positive_int, default=10)
    parser.add_argument("--compute-units", type=positive_int)
    parser.add_argument("--l2-mib", type=positive_float)
    parser.add_argument("--quick", action="store_true",
                        help="Smoke checks; these rates are not peak measurements")
    parser.add_argument("--output", type=Path, default=Path("results/chip_metrics.json"),
                        help="Complete table JSON, checkpointed after every metric")
    parser.add_argument("--results-dir", type=Path,
                        help="Per-metric raw JSON and logs (default: OUTPUT_STEM_runs)")
    parser.add_argument("--timeout", type=positive_float, default=900,
                        help="Maximum seconds per metric (default: 900)")
    parser.add_argument("--only", nargs="+", metavar="METRIC",
                        help="Run only these metric keys; the others stay 'skipped'")
    parser.add_argument("--resume", action="store_true",
                        help="Keep rows of an existing --output report that finished (ok, unverified, "
                             "unsupported, not_implemented) and run only the others")
    parser.add_argument("--widened", action="store_true",
                        help="Also measure converted FP8/FP4 vector chains; they stay details of the "
                             "not_implemented/unsupported rows, never a row value")
    parser.add_argument("--probe-device", action="store_true", help=argparse.SUPPRESS)
    return parser


def metric_command(metric, args, output):
    """Child argv: the active interpreter and the repository-local scripts, no shell."""
    if metric.key == "memory_capacity":
        script, extra = "bench_suite.py", ["--probe-device"]
    elif metric.key == "memory_bandwidth":
        script, extra = "bench_bandwidth.py", ["--mode", "all", "--dtype", "fp32"]
    elif metric.group == "Tensor":
        script = "bench_tensor.py"
        extra = ["--mode", "peak", "--dtype", "fp32" if metric.precision == "tf32" else metric.precision]
        if metric.precision in ("fp32", "tf32"):
            extra += ["--input-precision", "tf32" if metric.precision == "tf32" else "ieee"]
    else:
        script, extra = "bench_vector.py", ["--dtype", metric.precision]
        if getattr(args, "widened", False) and metric.precision in ("fp8", "fp4"):
            extra.append("--widened")
    command = [sys.executable, "-u", str(ROOT / script), *extra,
               "--device", str(args.device), "--timing", args.timing,
               "--warmup", str(args.warmup), "--rep", str(args.rep),
               "--batch-ms", str(args.batch_ms), "--rounds", str(args.rounds),
               "--output", str(output)]
    for flag, value in (("--compute-units", args.compute_units), ("--l2-mib", args.l2_mib)):
        if value is not None:
            command += [flag, str(value)]
    if args.quick:
        command.append("--quick")
    return command


def write_json(path, document):
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_name(path.name + ".tmp")
    temporary.write_text(json.dumps(document, indent=2, allow_nan=False) + "\n")
    temporary.replace(path)


def probe_device(args):
    """The memory_capacity child: only the device block."""
    if __package__ in (None, ""):
        from triton_chip_benchmarks_amd.common import setup_device
    else:
        from .common import setup_device
    metadata = setup_device(args)
    write_json(args.output, {"status": "ok", "device": metadata, "results": []})


def run_metric(metric, args, directory):
    output = directory / f"{metric.key}.json"
    log = directory / f"{metric.key}.log"
    command = metric_command(metric, args, output)
    output.unlink(missing_ok=True)  # an old success must never stand in for a new failure
    document = result = returncode = None
    try:
        with log.open("w") as stream:
            completed = subprocess.run(command, cwd=ROOT, stdout=stream, stderr=subprocess.STDOUT,
                                       timeout=args.timeout, check=False)
        returncode = completed.returncode
        if output.exists():
            try:
                document = json.loads(output.read_text())
                if not isinstance(document, dict):
                    raise ValueError("expected a JSON object")
                result = summarize(metric, document)
                if args.quick and result["status"] in ("ok", "unverified") and metric.group != "Memory":
                    result["smoke_only"] = True
            except (OSError, ValueError, TypeError, AttributeError, KeyError) as exc:
                result = empty_metric(metric, "error", f"Invalid benchmark JSON: {exc}")
        else:
            result = empty_metric(metric, "error", "Benchmark did not write result JSON")
        if returncode and result["status"] not in ("unsupported", "not_implemented"):
            partial = result if result["status"] in ("ok", "unverified") else None
            result = empty_metric(metric, "error", f"Benchmark exited with code {returncode}; see log")
            if partial is not None:
                result["partial_measurement"] = partial
    except subprocess.TimeoutExpired:
        result = empty_metric(metric, "error", f"Exceeded {args.timeout:g} seconds; see log")
    except OSError as exc:
        result = empty_metric(metric, "error", f"Cannot execute benchmark: {exc}")
    result.update(command=command, source_json=str(output), log_file=str(log), returncode=returncode)
    return result, document


FINISHED = ("ok", "unverified", "unsupported", "not_implemented")


def resumable_rows(path, quick):
    """Finished rows of an earlier report at `path`, by metric key.

    Only a report of this schema, with the same 17 metric keys and the same
    --quick setting, is reused; anything else resumes nothing.
    """
    try:
        previous = json.loads(Path(path).read_text())
    except (OSError, ValueError):
        return {}
    if not isinstance(previous, dict) or previous.get("schema_version") != 1:
        return {}
    rows = previous.get("results")
    if not isinstance(rows, list) or [r.get("metric") for r in rows if isinstance(r, dict)] != \
            [metric.key for metric in METRICS]:
        return {}
    if bool(previous.get("smoke_only")) != bool(quick):
        return {}
    return {row["metric"]: row for row in rows if row.get("status") in FINISHED}


def run_suite(args):
    args.output = args.output.resolve()
    directory = (args.results_dir or args.output.with_name(args.output.stem + "_runs")).resolve()
    directory.mkdir(parents=True, exist_ok=True)
    selected = set(args.only) if getattr(args, "only", None) else None
    resumed = resumable_rows(args.output, args.quick) if getattr(args, "resume", False) else {}
    if selected:
        unknown = selected - {metric.key for metric in METRICS}
        if unknown:
            raise SystemExit(f"Unknown metric keys for --only: {', '.join(sorted(unknown))}")
    report = {
        "schema_version": 1, "benchmark": "chip_metric_suite",
        "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "status": "running", "device": {}, "smoke_only": args.quick,
        "measurement_policy": MEASUREMENT_POLICY,
        "results": [empty_metric(metric) for metric in METRICS],
    }
    write_json(args.output, report)
    for index, metric in enumerate(METRICS):
        if selected is not None and metric.key not in selected:
            report["results"][index] = empty_metric(metric, "skipped", "not selected with --only")
            continue
        if metric.key in resumed:
            report["results"][index] = dict(resumed[metric.key], resumed=True)
            write_json(args.output, report)
            print(f"[{index + 1}/{len(METRICS)}] {metric.key}: kept from the earlier report "
                  f"({resumed[metric.key]['status']})", flush=True)
            continue
        print(f"[{index + 1}/{len(METRICS)}] {metric.key} ...", flush=True)
        result, document = run_metric(metric, args, directory)
        report["results"][index] = result
        if document and isinstance(document.get("device"), dict) and document["device"] and not report["device"]:
            report["device"] = document["device"]
        write_json(args.output, report)
        print(f"  {result['status']}" + (f": {result['reason']}" if result.get("reason") else ""), flush=True)
    report["status"] = ("complete_with_errors" if any(item["status"] == "error" for item in report["results"])
                        else "complete")
    write_json(args.output, report)
    print("\n" + format_table(report["results"]))
    print(f"\nJSON: {args.output}")
    print(f"Raw results and logs: {directory}")
    return report


def main(argv=None):
    args = build_parser().parse_args(argv)
    if args.probe_device:
        probe_device(args)
        return 0
    report = run_suite(args)
    return 1 if report["status"] == "complete_with_errors" else 0


if __name__ == "__main__":
    raise SystemExit(main())
