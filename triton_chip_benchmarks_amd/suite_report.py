"""The 17-row chip metric contract and the child-document -> row summary.

Row keys, groups, precisions and units are the reference's
(suite_report.py:7-24), so reports diff row for row against its published
tables. The selection rules follow suite_report.py:88-148: the highest valid
peak wins, its median comes from the same configuration, a missing value is
never zero, and a measured rate whose instruction audit did not pass is kept
but marked `unverified`. Rows additionally carry a `roofline` block against
the MI355X peak.
"""

from __future__ import annotations

from dataclasses import dataclass
import math

from . import roofline


@dataclass(frozen=True)
class Metric:
    key: str
    group: str
    precision: str | None
    unit: str


TENSOR_PRECISIONS = ("bf16", "fp16", "fp32", "tf32", "int8", "fp64", "fp8", "fp4")
VECTOR_PRECISIONS = ("bf16", "fp16", "fp32", "int8", "fp64", "fp8", "fp4")


def _unit(precision: str) -> str:
    return "TOP/s" if precision == "int8" else "TFLOP/s"


METRICS = (
    Metric("memory_capacity", "Memory", None, "GiB"),
    Metric("memory_bandwidth", "Memory", None, "GB/s"),
    *(Metric(f"tensor_{p}", "Tensor", p, _unit(p)) for p in TENSOR_PRECISIONS),
    *(Metric(f"vector_{p}", "Vector", p, _unit(p)) for p in VECTOR_PRECISIONS),
)

_DETAIL_KEYS = ("execution_kind", "native_tensor_verified", "native_arithmetic_verified",
                "instruction_precision_verified", "precision_verified", "assembly_check",
                "assembly_audit", "assembly_audit_note", "arithmetic_dtype", "includes_unpacking",
                "input_storage_dtype", "accumulator_dtype", "output_dtype", "operation",
                "measurement_kind", "timing_method", "timing_fallback_reason",
                "kernel", "tensor_instruction_types", "amdgcn_instruction_types")
_CONFIGURATION_KEYS = ("config", "block_size", "num_warps", "unroll", "blocks_per_sm", "blocks",
                       "iterations", "pattern", "buffer_mib", "cache_regime", "peak_eligible",
                       "block_threads", "vectors_per_thread", "grid_blocks", "nontemporal", "variant")


def empty_metric(metric, status="pending", reason=None):
    row = {"metric": metric.key, "group": metric.group, "precision": metric.precision,
           "unit": metric.unit, "status": status, "value": None, "median_value": None}
    if reason:
        row["reason"] = reason
    return row


def _positive(value) -> bool:
    return (isinstance(value, (int, float)) and not isinstance(value, bool)
            and math.isfinite(value) and value > 0)


def rates(metric, row):
    """(peak, median) of a child row in the metric's unit."""
    if metric.key == "memory_bandwidth":
        return row.get("peak_gbps"), row.get("gbps")
    peak = row.get("peak_teraops_per_second")
    median = row.get("median_teraops_per_second")
    suffix = "tops" if metric.precision == "int8" else "tflops"
    if peak is None:
        peak = row.get(f"peak_{suffix}")
    if median is None:
        median = row.get(suffix)
    return peak, median


def _details(metric, row):
    peak, median = rates(metric, row)
    details = {"value": peak, "median_value": median, "smoke_only": bool(row.get("smoke_only", False))}
    compiled = row.get("compiled") or {}
    for key in _DETAIL_KEYS:
        if key in row or key in compiled:
            details[key] = row.get(key, compiled.get(key))
    details["configuration"] = {key: row[key] for key in _CONFIGURATION_KEYS if key in row}
    block = roofline.describe(metric.key, peak)
    if block is not None:
        details["roofline"] = block
    return details


def _verification_reason(metric, details):
    if metric.group == "Tensor":
        execution = details.get("execution_kind")
        known = execution == "simt" or (execution == "tensor" and details.get("native_tensor_verified") is True)
        if details.get("instruction_precision_verified") is not True or not known:
            return "Measured matrix rate retained; native instruction precision or execution unit is unverified"
    elif metric.group == "Vector" and details.get("native_arithmetic_verified") is not True:
        if metric.precision == "int8" and details.get("includes_unpacking"):
            return ("Measured portable INT8-input path uses INT32 arithmetic and includes unpacking; "
                    "native INT8 execution is unverified")
        return "Measured vector rate retained; native arithmetic instruction precision is unverified"
    return None


def summarize(metric, document):
    """One report row; a measured row also carries the child's host CPU baseline."""
    result = _summarize(metric, document)
    baseline = document.get("cpu_baseline")
    if result.get("status") in ("ok", "unverified") and isinstance(baseline, dict):
        result["cpu_baseline"] = baseline
    return result


# Child statuses that are reported as they are, without looking at measurements.
_DECLARED_STATUSES = frozenset(("unsupported", "not_implemented", "error", "unavailable"))
# The memory row's per-pattern record: which patterns are kept, and which of them may set the row value.
_MEMORY_PATTERNS = ("copy", "read")
_MEMORY_VALUE_PATTERN = "copy"
_NO_HBM_COPY = ("No HBM-sized copy candidate: use a non-quick run with known last-level cache capacity "
                "and buffers at least 4x that capacity; observed pattern rates remain in patterns")


@dataclass(frozen=True)
class _Candidate:
    """One child row with both rates positive: (peak, median) in the metric's unit."""
    peak: float
    median: float
    row: dict

    @property
    def hbm_sized(self) -> bool:
        return self.row.get("peak_eligible") is True and not self.row.get("smoke_only", False)


def _candidates(metric, rows):
    """(valid candidates, rejected dict rows): a row is valid when its status is ok and both rates are positive."""
    valid, rejected = [], []
    for row in rows:
        if not isinstance(row, dict):
            continue
        rejected.append(row)
        peak, median = rates(metric, row)
        if row.get("status", "ok") == "ok" and _positive(peak) and _positive(median):
            valid.append(_Candidate(peak, median, row))
    return valid, rejected


def _best(candidates):
    """The highest peak; the first of equal peaks (its median comes from the same configuration)."""
    return max(candidates, key=lambda candidate: candidate.peak)


def _declared(metric, document):
    status = document.get("status")
    if status not in _DECLARED_STATUSES:
        return None
    result = empty_metric(metric)
    result.update(status=status, reason=document.get("reason", status))  # kept even when the child gave None
    details = document.get("details")
    widened = details.get("widened") if isinstance(details, dict) else None
    if isinstance(widened, dict):
        # A converted (widened) measurement is a detail of the row, never its value.
        result["widened_measurement"] = widened
    return result


def _capacity(metric, document):
    if metric.key != "memory_capacity":
        return None
    capacity = document.get("device", {}).get("total_memory_bytes")
    if not _positive(capacity):
        return empty_metric(metric, "unavailable", "Backend did not report total memory capacity")
    result = empty_metric(metric, "ok")
    result.update(value=capacity / 2**30, capacity_bytes=capacity, measurement_kind="reported_device_capacity")
    return result


def _measured(metric, document):
    rows = document.get("results", [])
    if not isinstance(rows, list):
        return empty_metric(metric, "error", "Benchmark results must be a list")
    valid, rejected = _candidates(metric, rows)
    if not valid:
        # Every rejected configuration declared unsupported -> the row is unsupported; anything else is an error.
        status = "unsupported" if rejected and all(row.get("status") == "unsupported" for row in rejected) else "error"
        reasons = dict.fromkeys(str(row.get("reason", "No valid throughput")) for row in rejected)
        return empty_metric(metric, status,
                            "; ".join(reasons) or "Benchmark produced no valid throughput measurements")
    result = empty_metric(metric)
    if metric.key == "memory_bandwidth":
        by_pattern = {pattern: [c for c in valid if c.row.get("pattern") == pattern] for pattern in _MEMORY_PATTERNS}
        result["patterns"] = {pattern: _details(metric, _best([c for c in group if c.hbm_sized] or group).row)
                              for pattern, group in by_pattern.items() if group}
        valid = [c for c in by_pattern[_MEMORY_VALUE_PATTERN] if c.hbm_sized]
        if not valid:
            result.update(status="not_measured", reason=_NO_HBM_COPY)
            return result
    result.update(status="ok", **_details(metric, _best(valid).row))
    if document.get("arguments", {}).get("quick") and metric.group != "Memory":
        result["smoke_only"] = True
    reason = _verification_reason(metric, result)
    if reason:
        result.update(status="unverified", reason=reason)
    result["successful_configurations"] = len(valid)
    return result


# Stages in order; the first that returns a row decides it.
_STAGES = (_declared, _capacity, _measured)


def _summarize(metric, document):
    """One report row from a child's result document (suite_report.py:88-148).

    A declared status (unsupported, not_implemented, error, unavailable) is
    kept as is; capacity comes from the device block; otherwise the highest
    valid peak wins, with its own configuration's median, and a run with no
    valid row is an error unless every rejected configuration declared itself
    unsupported.
    """
    for stage in _STAGES:
        result = stage(metric, document)
        if result is not None:
            return result
    raise AssertionError("the last stage always returns a row")


def _number(value, digits=3):
    return "-" if value is None else f"{value:.{digits}f}"


# Table columns: (header, width, alignment, cell). Notes: (rule, message) pairs applied to every row in order.
_COLUMNS = (
    ("Metric", 20, "<", lambda item: item["metric"]),
    ("Peak / capacity", 17, ">", lambda item: _number(item.get("value"))),
    ("Median", 12, ">", lambda item: _number(item.get("median_value"))),
    ("Unit", 8, "<", lambda item: item["unit"]),
    ("% peak", 7, ">", lambda item: _number(None if (item.get("roofline") or {}).get("frac") is None
                                            else 100 * item["roofline"]["frac"], 1)),
    ("Status", 0, "<", lambda item: item["status"]),
)


def _widened_note(item):
    widened = item.get("widened_measurement")
    if isinstance(widened, dict) and widened.get("peak_tflops"):
        return (f"widened ({widened.get('arithmetic_kind', 'converted')}) {widened['peak_tflops']:.3f} TFLOP/s "
                "- not native arithmetic, not the row value")
    return None


_NOTES = (
    lambda item: item.get("reason") or None,
    lambda item: "smoke test; not a peak result" if item.get("smoke_only") else None,
    _widened_note,
    lambda item: ("measured matrix rate using SIMT scalar/vector instructions (no native tensor MMA)"
                  if item.get("execution_kind") == "simt" else None),
)


def _line(cells):
    return " ".join(f"{cell:{align}{width}}" if width else cell
                    for cell, (_, width, align, _) in zip(cells, _COLUMNS))


def format_table(results):
    """One line per requested metric (missing ones included), then the host baselines, then notes."""
    header = _line([title for title, *_ in _COLUMNS])
    lines = [header, "-" * (len(header) + 8)]
    lines += [_line([cell(item) for *_, cell in _COLUMNS]) for item in results]
    notes = [f"{item['metric']}: {note}" for item in results for rule in _NOTES
             for note in (rule(item),) if note]
    baselines = [item for item in results if isinstance(item.get("cpu_baseline"), dict)]
    if baselines:
        first = baselines[0]["cpu_baseline"]
        host = first.get("host") or {}
        lines += ["", f"Host CPU baseline (the reference's host computation, {host.get('cpu_model') or 'CPU'}, "
                      f"{first.get('cores')} threads):"]
        lines += [f"  {item['metric']:<20} {item['cpu_baseline']['value']:>12.4g} {item['cpu_baseline']['unit']:<8} "
                  f"{item['cpu_baseline'].get('method', '')}; {item['cpu_baseline'].get('sample', '')}"
                  for item in baselines]
    if notes:
        lines += ["", *notes]
    return "\n".join(lines)
