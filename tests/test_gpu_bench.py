"""GPU test of the headline line's contract: one JSON line under 8 KiB with every
field the driver reads, a roofline block for the dominant kernel and a CPU
baseline, and the full per-row records in the detail file the line names.

The run is short (2 timed launches per kernel after a 30 ms warmup) and
exercises the same code path as the default run: every row of the
benchmark specification, validated before and after timing.
"""

import json
import math
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
TOP_LEVEL = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
             "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "rows"}


def test_bench_prints_one_contract_line(gpu, tmp_path):
    detail_path = tmp_path / "bench_detail.json"
    completed = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), "--steps", "2", "--warmup", "1",
                                "--warmup-ms", "30", "--detail", str(detail_path)],
                               cwd=ROOT, capture_output=True, text=True, timeout=600, check=False)
    assert completed.returncode == 0, completed.stderr[-3000:]
    lines = [line for line in completed.stdout.splitlines() if line.strip()]
    assert len(lines) == 1, lines
    assert len(lines[0].encode()) <= 8192, len(lines[0].encode())
    line = json.loads(lines[0])
    assert TOP_LEVEL <= set(line), TOP_LEVEL - set(line)
    assert line["detail"] == str(detail_path)
    detail = json.loads(detail_path.read_text())
    assert [row["name"] for row in detail["rows"]] == [row["name"] for row in line["rows"]]
    assert detail["value"] == pytest.approx(line["value"], rel=1e-4)
    assert line["metric"] == "MFMA TFLOP/s (BF16/FP8/MXFP4) + HBM copy GB/s, as % of MI355X peak"
    assert (line["n_gpus"], line["steps"], line["warmup"]) == (1, 2, 1)
    assert line["higher_is_better"] is True and line["vs_baseline"] is None
    assert "workload" in line["config"] and "model" not in line["config"]
    compact = {row["name"]: row for row in line["rows"]}
    rows = {row["name"]: row for row in detail["rows"]}
    assert set(rows) == {"hbm_copy", "peak_bf16", "gemm_bf16", "gemm_fp16", "gemm_fp8", "gemm_int8", "gemm_fp64",
                         "gemm_mxfp4", "peak_bf16_128x128_c2", "peak_fp8", "peak_fp8_dense", "peak_mxfp4",
                         "vector_fp32", "vector_fp16", "vector_bf16", "vector_fp64", "vector_int8"}
    for name, row in compact.items():
        assert {"name", "kernel", "value", "unit", "frac", "ms_per_launch", "in_headline"} <= set(row)
        assert row["kernel"] == rows[name]["kernel"] and row["frac"] == pytest.approx(rows[name]["frac"], rel=1e-3)
    # The headline BF16 row is the specification's resident variant: a 256x256x64 tile looped 1024 times.
    assert rows["peak_bf16"]["config"]["tile"] == "256x256x64" and rows["peak_bf16"]["config"]["iterations"] == 1024
    assert rows["peak_bf16"]["kernel"].startswith("tensor_peak_bf16_256x256x64_")
    # The vector rows (the specification's FMA-chain configuration) carry the issue ceiling of the
    # instruction they run where it is below the datasheet figure.
    for name in ("vector_fp32", "vector_bf16"):
        assert 0.5 < rows[name]["frac_of_issued_ceiling"] <= 1.0, rows[name]
    assert rows["vector_int8"]["unit"] == "TOP/s" and rows["vector_int8"]["bound"] == "valu"
    headline = {name for name, row in rows.items() if row["in_headline"]}
    assert headline == {"hbm_copy", "peak_bf16", "gemm_bf16", "gemm_fp8", "gemm_mxfp4"}
    assert all(name in line["config"]["workload"] for name in rows)
    fractions = [rows[name]["frac"] for name in headline]
    assert all(0.2 < row["frac"] < 1.0 for row in rows.values()), {n: r["frac"] for n, r in rows.items()}
    assert line["value"] == pytest.approx(100 * sum(fractions) / len(fractions), rel=1e-4)
    assert line["ms_per_step"] == pytest.approx(sum(row["ms_per_launch"] for row in rows.values()), rel=1e-4)
    for name, row in rows.items():
        # The clock witness ran beside every row's kernel; a kernel cannot beat its peak at the clock it ran at.
        assert 500 < row["clock"]["clock_mhz"] < 2500, (name, row["clock"])
        assert compact[name]["clock_mhz"] == round(row["clock"]["clock_mhz"])
        if row["bound"] != "hbm":
            assert row["frac_at_clock"] < 1.03, (name, row["frac_at_clock"])
    # The copy row carries its read/write bound, measured on its own buffers, which a copy cannot beat by more
    # than timing noise.
    copy = rows["hbm_copy"]
    assert 0.5 < copy["rw_bound_frac"] < 1.0 and copy["frac"] <= 1.05 * copy["rw_bound_frac"], copy["context"]
    assert compact["hbm_copy"]["rw_bound_frac"] == pytest.approx(copy["rw_bound_frac"], rel=1e-3)
    if line["config"]["power_cap_w"] is not None:  # the ROCm SMI library saw the device: metered rows carry power
        import bench

        for name in bench.POWER_ROWS:
            assert 100 < rows[name]["power"]["mean_w"] < 2000, (name, rows[name]["power"])
            assert compact[name]["power_w"] == round(rows[name]["power"]["mean_w"])
    for row in rows.values():
        assert row["min_ms_per_launch"] <= row["median_ms_per_launch"] * (1 + 1e-9)
        assert row["warmup_device_ms"] >= 30 * 0.99 and "timed launches" in row["validation"]
    roofline = line["roofline"]
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(roofline)
    assert roofline["bound"] in ("hbm", "mfma")
    assert roofline["frac"] == pytest.approx(roofline["achieved"] / roofline["peak"], rel=1e-4)
    dominant = max((rows[name] for name in headline), key=lambda row: row["ms_per_launch"])
    assert roofline["kernel"] == dominant["kernel"]
    baseline = line["cpu_baseline"]
    assert {"value", "unit", "cores", "kind", "sample"} <= set(baseline) and len(baseline["sample"]) <= 200
    assert baseline["kind"] in ("port", "reference") and baseline["cores"] >= 1
    assert math.isfinite(baseline["value"]) and baseline["value"] > 0
