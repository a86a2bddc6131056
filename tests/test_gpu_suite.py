"""End-to-end GPU run of the suite CLI: real child processes, one per selected metric.

The reference's suite runs every metric in an isolated child and folds the
child documents into the 17-row report (bench_suite.py:72-199). Here a
--quick run of a few metrics goes through the same path on the card: each
selected row must come back measured (or with its declared status), the
others "skipped", and the report must keep the 17-row contract.
"""

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
SELECTED = ["memory_capacity", "tensor_bf16", "vector_fp32", "vector_fp8"]


def test_quick_suite_runs_children_and_keeps_the_row_contract(gpu, tmp_path):
    from triton_chip_benchmarks_amd.suite_report import METRICS

    output = tmp_path / "chip_metrics.json"
    command = [sys.executable, "-u", str(ROOT / "bench_suite.py"), "--quick", "--widened", "--timeout", "240",
               "--output", str(output), "--only", *SELECTED]
    completed = subprocess.run(command, cwd=ROOT, capture_output=True, text=True, timeout=600, check=False)
    assert completed.returncode == 0, completed.stdout[-2000:] + completed.stderr[-2000:]
    report = json.loads(output.read_text())
    assert report["status"] == "complete" and report["smoke_only"] is True
    rows = {row["metric"]: row for row in report["results"]}
    assert [row["metric"] for row in report["results"]] == [metric.key for metric in METRICS]
    for key, row in rows.items():
        if key not in SELECTED:
            assert row["status"] == "skipped", row
    assert rows["memory_capacity"]["status"] == "ok" and rows["memory_capacity"]["value"] > 200
    for key in ("tensor_bf16", "vector_fp32"):
        assert rows[key]["status"] == "ok" and rows[key]["value"] > 0, rows[key]
        assert rows[key].get("smoke_only") is True
        assert Path(rows[key]["log_file"]).exists()
        baseline = rows[key]["cpu_baseline"]  # the reference's host computation, timed beside the row
        assert baseline["value"] > 0 and baseline["cores"] >= 1 and baseline["host"]["os_cpu_count"] >= 1
    fp8 = rows["vector_fp8"]
    assert fp8["status"] == "not_implemented" and fp8["value"] is None
    assert fp8["widened_measurement"]["peak_tflops"] > 0
    assert report["device"]["gcn_arch_name"].startswith("gfx950")
