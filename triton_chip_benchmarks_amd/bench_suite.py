#!/usr/bin/env python3
"""Run the complete 17-row chip metric table on one MI355X, one child per metric.

The CLI, the child command lines and the report document are the reference's
contract (bench_suite.py:72-199), so reports diff row for row: every metric
runs in its own child process under a timeout, the child's stale output is
deleted first so an old success can never stand in for a new failure, and the
report is rewritten atomically after every metric.

Structure here: `metric_command` builds a child's argv from a per-group
table; `launch_child` runs it and returns a `ChildRun` record (exit code,
parsed document, or the problem that prevented one); `classify` turns that
record into the report row by a fixed sequence of rules; `SuiteReport` owns
the document and its checkpoints.
"""

from __future__ import annotations

import argparse
from dataclasses import dataclass, field
from datetime import datetime, timezone
import json
from pathlib import Path
import subprocess
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd.common import positive_float, positive_int
    from triton_chip_benchmarks_amd.counters import attach as attach_counters
    from triton_chip_benchmarks_amd.suite_report import METRICS, empty_metric, format_table, summarize
else:
    from .common import positive_float, positive_int
    from .counters import attach as attach_counters
    from .suite_report import METRICS, empty_metric, format_table, summarize

ROOT = Path(__file__).resolve().parent.parent

# Report text the contract fixes (reference bench_suite.py:138-155, 171-172).
MEASUREMENT_POLICY = ("Highest observed valid throughput; median from the same configuration. "
                      "Capacity is reported device capacity. Bandwidth is effective copy read+write "
                      "traffic with HBM-sized buffers; read rates are auxiliary details. "
                      "Unsupported and not-implemented metrics have no numeric value; "
                      "errors do not imply unsupported hardware.")
REASONS = {
    "missing": "Benchmark did not write result JSON",
    "invalid": "Invalid benchmark JSON: {error}",
    "exit": "Benchmark exited with code {code}; see log",
    "timeout": "Exceeded {seconds:g} seconds; see log",
    "launch": "Cannot execute benchmark: {error}",
}
DECLARED = ("unsupported", "not_implemented")  # a child's own verdict, kept whatever its exit code
MEASURED = ("ok", "unverified")
FINISHED = MEASURED + DECLARED                  # rows that --resume keeps

# Child program and fixed arguments per metric group; tensor and vector rows
# add their precision (TF32 is FP32 storage with the tf32 input precision).
_GROUP_CHILD = {
    "Tensor": ("bench_tensor.py", ["--mode", "peak"]),
    "Vector": ("bench_vector.py", []),
}
_SPECIAL_CHILD = {
    "memory_capacity": ("bench_suite.py", ["--probe-device"]),
    "memory_bandwidth": ("bench_bandwidth.py", ["--mode", "all", "--dtype", "fp32"]),
}


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
    parser.add_argument("--counters", type=Path,
                        help="Attach the per-kernel hardware counters of this summary "
                             "(counters.py summarize --json) to the rows that ran those kernels")
    parser.add_argument("--probe-device", action="store_true", help=argparse.SUPPRESS)
    return parser


def _metric_arguments(metric, args) -> tuple[str, list[str]]:
    """(child script, metric-specific arguments)."""
    if metric.key in _SPECIAL_CHILD:
        script, fixed = _SPECIAL_CHILD[metric.key]
        return script, list(fixed)
    script, fixed = _GROUP_CHILD[metric.group]
    precision = metric.precision
    if metric.group == "Tensor":
        extra = ["--dtype", "fp32" if precision == "tf32" else precision]
        if precision in ("fp32", "tf32"):
            extra += ["--input-precision", precision if precision == "tf32" else "ieee"]
    else:
        extra = ["--dtype", precision]
        if getattr(args, "widened", False) and precision in ("fp8", "fp4"):
            extra.append("--widened")
    return script, fixed + extra


def metric_command(metric, args, output):
    """Child argv: this interpreter and the repository's own scripts, no shell."""
    script, specific = _metric_arguments(metric, args)
    shared = {"--device": args.device, "--timing": args.timing, "--warmup": args.warmup, "--rep": args.rep,
              "--batch-ms": args.batch_ms, "--rounds": args.rounds, "--output": output,
              "--compute-units": args.compute_units, "--l2-mib": args.l2_mib}
    command = [sys.executable, "-u", str(ROOT / script), *specific]
    for flag, value in shared.items():
        if value is not None:
            command += [flag, str(value)]
    if args.quick:
        command.append("--quick")
    return command


def atomic_json(path: Path, document) -> None:
    """Write `document` to `path` through a temporary sibling and a rename."""
    path.parent.mkdir(parents=True, exist_ok=True)
    staging = path.with_name(path.name + ".tmp")
    staging.write_text(json.dumps(document, indent=2, allow_nan=False) + "\n")
    staging.replace(path)


def probe_device(args):
    """The memory_capacity child: only the device block."""
    if __package__ in (None, ""):
        from triton_chip_benchmarks_amd.common import setup_device
    else:
        from .common import setup_device
    atomic_json(args.output, {"status": "ok", "device": setup_device(args), "results": []})


@dataclass
class ChildRun:
    """What one child left behind: its exit code and document, or why there is neither."""

    command: list
    output: Path
    log: Path
    returncode: int | None = None
    document: object = None
    problem: str | None = None
    notes: dict = field(default_factory=dict)


def launch_child(metric, args, directory: Path) -> ChildRun:
    output, log = directory / f"{metric.key}.json", directory / f"{metric.key}.log"
    run = ChildRun(metric_command(metric, args, output), output, log)
    output.unlink(missing_ok=True)  # only this run's document may be read back
    try:
        with log.open("w") as stream:
            run.returncode = subprocess.run(run.command, cwd=ROOT, stdout=stream, stderr=subprocess.STDOUT,
                                            timeout=args.timeout, check=False).returncode
    except subprocess.TimeoutExpired:
        run.problem = REASONS["timeout"].format(seconds=args.timeout)
        return run
    except OSError as exc:
        run.problem = REASONS["launch"].format(error=exc)
        return run
    if output.exists():
        try:
            run.document = json.loads(output.read_text())
        except (OSError, ValueError) as exc:
            run.notes["invalid"] = str(exc)
    return run


def classify(metric, run: ChildRun, quick: bool) -> dict:
    """The report row for a child run.

    Rules, in order: no run at all is an error; no document, or one that does
    not summarise, is an error; otherwise the summary is the row (a quick
    run's measured rate is smoke only, except memory rows); finally a
    non-zero exit turns a row into an error unless the child declared the
    metric unsupported or not implemented, and a measured rate stays
    attached as the partial measurement.
    """
    if run.problem is not None:
        return empty_metric(metric, "error", run.problem)
    if "invalid" in run.notes:
        row = empty_metric(metric, "error", REASONS["invalid"].format(error=run.notes["invalid"]))
    elif run.document is None:
        row = empty_metric(metric, "error", REASONS["missing"])
    else:
        try:
            if not isinstance(run.document, dict):
                raise ValueError("expected a JSON object")
            row = summarize(metric, run.document)
        except (ValueError, TypeError, AttributeError, KeyError) as exc:
            row = empty_metric(metric, "error", REASONS["invalid"].format(error=exc))
        else:
            if quick and row["status"] in MEASURED and metric.group != "Memory":
                row["smoke_only"] = True
    if run.returncode and row["status"] not in DECLARED:
        failed = empty_metric(metric, "error", REASONS["exit"].format(code=run.returncode))
        if row["status"] in MEASURED:
            failed["partial_measurement"] = row
        row = failed
    return row


def run_metric(metric, args, directory):
    """(row, child document) of one metric."""
    run = launch_child(metric, args, directory)
    row = classify(metric, run, args.quick)
    row.update(command=run.command, source_json=str(run.output), log_file=str(run.log),
               returncode=run.returncode)
    return row, run.document if isinstance(run.document, dict) else None


def resumable_rows(path, quick):
    """Finished rows of an earlier report at `path`, by metric key.

    Only a schema-1 report of these 17 metric keys, written with the same
    --quick setting, is reused; anything else resumes nothing.
    """
    try:
        previous = json.loads(Path(path).read_text())
    except (OSError, ValueError):
        return {}
    rows = previous.get("results") if isinstance(previous, dict) else None
    if not isinstance(rows, list) or previous.get("schema_version") != 1:
        return {}
    if [row.get("metric") for row in rows if isinstance(row, dict)] != [m.key for m in METRICS]:
        return {}
    if bool(previous.get("smoke_only")) != bool(quick):
        return {}
    return {row["metric"]: row for row in rows if row.get("status") in FINISHED}


class SuiteReport:
    """The suite document: one row per metric, rewritten atomically on every change."""

    def __init__(self, path: Path, quick: bool):
        self.path = path
        self.document = {
            "schema_version": 1, "benchmark": "chip_metric_suite",
            "timestamp_utc": datetime.now(timezone.utc).isoformat(),
            "status": "running", "device": {}, "smoke_only": quick,
            "measurement_policy": MEASUREMENT_POLICY,
            "results": [empty_metric(metric) for metric in METRICS],
        }
        self.checkpoint()

    @property
    def rows(self):
        return self.document["results"]

    def checkpoint(self):
        atomic_json(self.path, self.document)

    def record(self, index: int, row: dict, child_document=None):
        self.rows[index] = row
        device = child_document.get("device") if isinstance(child_document, dict) else None
        if isinstance(device, dict) and device and not self.document["device"]:
            self.document["device"] = device
        self.checkpoint()

    def finish(self):
        errors = any(row["status"] == "error" for row in self.rows)
        self.document["status"] = "complete_with_errors" if errors else "complete"
        self.checkpoint()
        return self.document


def run_suite(args):
    args.output = args.output.resolve()
    directory = (args.results_dir or args.output.with_name(args.output.stem + "_runs")).resolve()
    directory.mkdir(parents=True, exist_ok=True)
    selected = set(args.only) if getattr(args, "only", None) else None
    if selected and selected - {metric.key for metric in METRICS}:
        unknown = ", ".join(sorted(selected - {metric.key for metric in METRICS}))
        raise SystemExit(f"Unknown metric keys for --only: {unknown}")
    kept = resumable_rows(args.output, args.quick) if getattr(args, "resume", False) else {}
    report = SuiteReport(args.output, args.quick)
    for index, metric in enumerate(METRICS):
        label = f"[{index + 1}/{len(METRICS)}] {metric.key}"
        if selected is not None and metric.key not in selected:
            report.rows[index] = empty_metric(metric, "skipped", "not selected with --only")
            continue
        if metric.key in kept:
            report.record(index, dict(kept[metric.key], resumed=True))
            print(f"{label}: kept from the earlier report ({kept[metric.key]['status']})", flush=True)
            continue
        print(f"{label} ...", flush=True)
        row, document = run_metric(metric, args, directory)
        report.record(index, row, document)
        print(f"  {row['status']}" + (f": {row['reason']}" if row.get("reason") else ""), flush=True)
    if getattr(args, "counters", None):
        attach_counters(report.document, json.loads(Path(args.counters).read_text()))
    document = report.finish()
    print("\n" + format_table(document["results"]))
    print(f"\nJSON: {args.output}")
    print(f"Raw results and logs: {directory}")
    return document


def main(argv=None):
    args = build_parser().parse_args(argv)
    if args.probe_device:
        probe_device(args)
        return 0
    return 1 if run_suite(args)["status"] == "complete_with_errors" else 0


if __name__ == "__main__":
    raise SystemExit(main())
