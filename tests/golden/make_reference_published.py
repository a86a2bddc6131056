#!/usr/bin/env python3
"""Extract the reference's published numbers that pin the oracle (data only).

Reads result JSON files shipped in the reference repository (no reference
code is imported or run) and writes tests/golden/reference_published.json.
Every value records the file and field it came from.

Usage: python tests/golden/make_reference_published.py /root/reference
"""

import json
from pathlib import Path
import sys


def _row(root, path, index=0):
    document = json.loads((root / path).read_text())
    return document["results"][index]


def main(reference):
    root = Path(reference)
    out = {}
    row = _row(root, "results/bw1100_metrics_runs/vector_fp32.json")
    out["vector_fp32"] = {
        "source": "results/bw1100_metrics_runs/vector_fp32.json results[0]",
        "iterations": row["iterations"], "elements_per_chain": row["elements_per_chain"],
        "counted_flops": row["counted_flops"], "max_abs_tolerance": row["max_abs_tolerance"],
        "max_abs_error": row["max_abs_error"], "operation": row["operation"]}
    row = _row(root, "results/h20_metrics_runs/vector_fp32.json")
    out["vector_fp32_h20"] = {
        "source": "results/h20_metrics_runs/vector_fp32.json results[0]",
        "iterations": row["iterations"], "elements_per_chain": row["elements_per_chain"],
        "counted_flops": row["counted_flops"], "max_abs_tolerance": row["max_abs_tolerance"],
        "max_abs_error": row["max_abs_error"]}
    row = _row(root, "results/bw1100_metrics_runs/vector_fp64.json")
    out["vector_fp64"] = {
        "source": "results/bw1100_metrics_runs/vector_fp64.json results[0]",
        "iterations": row["iterations"], "elements_per_chain": row["elements_per_chain"],
        "max_abs_tolerance": row["max_abs_tolerance"], "max_abs_error": row["max_abs_error"]}
    row = _row(root, "results/bw1100_metrics_runs/vector_fp16.json")
    out["vector_fp16"] = {
        "source": "results/bw1100_metrics_runs/vector_fp16.json results[0]",
        "validation_recurrence": row["validation_recurrence"], "max_abs_tolerance": row["max_abs_tolerance"],
        "max_abs_error": row["max_abs_error"]}
    row = _row(root, "results/bw1100_metrics_runs/tensor_bf16.json")
    out["tensor_bf16_peak"] = {
        "source": "results/bw1100_metrics_runs/tensor_bf16.json results[0]",
        "config": row["config"], "blocks": row["blocks"], "iterations": row["iterations"],
        "operation_count": row["operation_count"], "atol": row["correctness"]["atol"],
        "rtol": row["correctness"]["rtol"]}
    row = _row(root, "results/bw1100_metrics_runs/tensor_int8.json")
    out["tensor_int8_peak"] = {
        "source": "results/bw1100_metrics_runs/tensor_int8.json results[0]",
        "config": row["config"], "blocks": row["blocks"], "iterations": row["iterations"],
        "operation_count": row["operation_count"], "atol": row["correctness"]["atol"]}
    copy = _row(root, "results/bw1100_metrics_runs/memory_bandwidth.json", 0)
    read = _row(root, "results/bw1100_metrics_runs/memory_bandwidth.json", 1)
    out["bandwidth"] = {
        "source": "results/bw1100_metrics_runs/memory_bandwidth.json results[0:2]",
        "copy": {key: copy[key] for key in ("buffer_bytes", "elements", "read_bytes", "write_bytes",
                                            "traffic_bytes", "block_size", "median_ms", "gbps")},
        "read": {key: read[key] for key in ("buffer_bytes", "elements", "read_bytes", "write_bytes",
                                            "traffic_bytes", "block_size")}}
    capacity = json.loads((root / "results/bw1100_metrics_runs/memory_capacity.json").read_text())
    out["memory_capacity"] = {"source": "results/bw1100_metrics_runs/memory_capacity.json device",
                              "total_memory_bytes": capacity["device"]["total_memory_bytes"],
                              "memory_capacity_gib": capacity["device"]["memory_capacity_gib"]}
    # The reference's GEMM mode on its own operand recipe (bench_tensor.py:249-299, 1509-1595): the
    # best-rate row per size of its FP16 run, with the tolerance it was checked at.
    gemm = json.loads((root / "results/h20_tensor.json").read_text())
    best = {}
    for row in gemm["results"]:
        if row.get("status") == "ok" and (row["m"] not in best or row["tflops"] > best[row["m"]]["tflops"]):
            best[row["m"]] = row
    out["gemm_fp16_h20"] = {
        "source": "results/h20_tensor.json results (best tflops per size)", "dtype": gemm["arguments"]["dtype"],
        "sizes": gemm["arguments"]["sizes"], "device": gemm["device"].get("device_name"),
        "rows": [{"m": r["m"], "n": r["n"], "k": r["k"], "flops": r["flops"], "tflops": r["tflops"],
                  "rtol": r["correctness"]["rtol"], "atol": r["correctness"]["atol"],
                  "max_abs_error": r["correctness"]["max_abs_error"], "config": r["config"]}
                 for r in (best[m] for m in sorted(best))]}
    # Known answers stated in the reference's tests.
    out["e2m1_packing"] = {"source": "tests/test_tensor_formats.py:55-64",
                           "codes": [[1, 2, 9, 10]], "packed": [[2 << 4 | 1, 10 << 4 | 9]],
                           "values": {"1": 0.5, "2": 1.0, "9": -0.5, "10": -1.0}}
    out["peak_tolerance"] = {"source": "tests/test_tensor_precision.py:180-216",
                             "bf16_block_k": 32, "iterations": 1024,
                             "below": 1 / 256 / 64, "above": 1.9073486328125e-06}
    out["int8_weights"] = {"source": "tests/test_vector_dtypes.py:162-174", "weights": [3, -2, 1, -1]}
    target = Path(__file__).with_name("reference_published.json")
    target.write_text(json.dumps(out, indent=2, sort_keys=True) + "\n")
    print(f"wrote {target}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
