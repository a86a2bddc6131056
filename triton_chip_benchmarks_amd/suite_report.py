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


def _summarize(metric, document):
    """One report row from a child's result document.

    A declared status (unsupported, not_implemented, error, unavailable) is
    kept as is. Otherwise the best valid row wins; failures are errors unless
    every rejected configuration was itself declared unsupported.
    """
    result = empty_metric(metric)
    status = document.get("status")
    if status in ("unsupported", "not_implemented", "error", "unavailable"):
        result.update(status=status, reason=document.get("reason", status))
        widened = (document.get("details") or {}).get("widened") if isinstance(document.get("details"), dict) else None
        if isinstance(widened, dict):
            # A converted (widened) measurement is a detail of the row, never its value.
            result["widened_measurement"] = widened
        return result
    if metric.key == "memory_capacity":
        capacity = document.get("device", {}).get("total_memory_bytes")
        if _positive(capacity):
            result.update(status="ok", value=capacity / 2**30, capacity_bytes=capacity,
                          measurement_kind="reported_device_capacity")
        else:
            result.update(status="unavailable", reason="Backend did not report total memory capacity")
        return result

    rows = document.get("results", [])
    if not isinstance(rows, list):
        return empty_metric(metric, "error", "Benchmark results must be a list")
    valid = [row for row in rows if isinstance(row, dict) and row.get("status", "ok") == "ok"
             and all(_positive(value) for value in rates(metric, row))]
    if not valid:
        rejected = [row for row in rows if isinstance(row, dict)]
        unsupported = bool(rejected) and all(row.get("status") == "unsupported" for row in rejected)
        reasons = list(dict.fromkeys(str(row.get("reason", "No valid throughput")) for row in rejected))
        return empty_metric(metric, "unsupported" if unsupported else "error",
                            "; ".join(reasons) or "Benchmark produced no valid throughput measurements")

    if metric.key == "memory_bandwidth":
        patterns = {}
        for pattern in ("copy", "read"):
            candidates = [row for row in valid if row.get("pattern") == pattern]
            eligible = [row for row in candidates
                        if row.get("peak_eligible") is True and not row.get("smoke_only", False)]
            if candidates:
                best = max(eligible or candidates, key=lambda row: rates(metric, row)[0])
                patterns[pattern] = _details(metric, best)
        result["patterns"] = patterns
        valid = [row for row in valid if row.get("pattern") == "copy"
                 and row.get("peak_eligible") is True and not row.get("smoke_only", False)]
        if not valid:
            result.update(status="not_measured", reason=(
                "No HBM-sized copy candidate: use a non-quick run with known last-level cache capacity "
                "and buffers at least 4x that capacity; observed pattern rates remain in patterns"))
            return result

    best = max(valid, key=lambda row: rates(metric, row)[0])
    result.update(status="ok", **_details(metric, best))
    if document.get("arguments", {}).get("quick") and metric.group != "Memory":
        result["smoke_only"] = True
    reason = _verification_reason(metric, result)
    if reason:
        result.update(status="unverified", reason=reason)
    result["successful_configurations"] = len(valid)
    return result


def format_table(results):
    """One line per requested metric, including missing ones, then notes."""
    lines = [f"{'Metric':<20} {'Peak / capacity':>17} {'Median':>12} {'Unit':<8} {'% peak':>7} Status",
             "-" * 94]
    notes = []
    for item in results:
        value = "-" if item.get("value") is None else f"{item['value']:.3f}"
        median = "-" if item.get("median_value") is None else f"{item['median_value']:.3f}"
        frac = (item.get("roofline") or {}).get("frac")
        percent = "-" if frac is None else f"{100 * frac:.1f}"
        lines.append(f"{item['metric']:<20} {value:>17} {median:>12} {item['unit']:<8} {percent:>7} "
                     f"{item['status']}")
        if item.get("reason"):
            notes.append(f"{item['metric']}: {item['reason']}")
        if item.get("smoke_only"):
            notes.append(f"{item['metric']}: smoke test; not a peak result")
        widened = item.get("widened_measurement")
        if isinstance(widened, dict) and widened.get("peak_tflops"):
            notes.append(f"{item['metric']}: widened ({widened.get('arithmetic_kind', 'converted')}) "
                         f"{widened['peak_tflops']:.3f} TFLOP/s - not native arithmetic, not the row value")
        if item.get("execution_kind") == "simt":
            notes.append(f"{item['metric']}: measured matrix rate using SIMT scalar/vector instructions "
                         "(no native tensor MMA)")
    baselines = [item for item in results if isinstance(item.get("cpu_baseline"), dict)]
    if baselines:
        host = baselines[0]["cpu_baseline"].get("host") or {}
        lines.extend(("", f"Host CPU baseline (the reference's host computation, {host.get('cpu_model') or 'CPU'}, "
                          f"{baselines[0]['cpu_baseline'].get('cores')} threads):"))
        for item in baselines:
            baseline = item["cpu_baseline"]
            lines.append(f"  {item['metric']:<20} {baseline['value']:>12.4g} {baseline['unit']:<8} "
                         f"{baseline.get('method', '')}; {baseline.get('sample', '')}")
    if notes:
        lines.extend(("", *notes))
    return "\n".join(lines)
