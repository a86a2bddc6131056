"""CPU tests of bench.py's stdout line: the contract fields, and a length bound that holds for a full row set.

A reader that keeps only the tail of stdout (about 10 KB) must still see the whole line, so the line is built from
compact rows and the full per-row records go to the detail file. These tests build the line from fake rows as long
as the real ones (every row of the run, long validation, config and CPU sample strings) and check the bound.
"""

import argparse
import json
import math
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

CONTRACT = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"}


def _fake_rows():
    names = [name for name, _ in bench._row_specs()]
    rows = []
    for index, name in enumerate(names):
        unit = "GB/s" if name == "hbm_copy" else "TOP/s" if "int8" in name else "TFLOP/s"
        peak = 8000.0 if unit == "GB/s" else 2516.5824
        value = peak * (0.5 + index / 100.0) + 1.0 / 3.0
        rows.append({
            "name": name, "row": "tensor_bf16", "in_headline": name in bench.HEADLINE,
            "kernel": f"tensor_peak_bf16_256x256x64_c1_mfma16_kn_{'x' * 20}", "value": value, "unit": unit,
            "peak": peak, "frac": value / peak, "peak_basis": "datasheet " * 10, "bound": "mfma",
            "ms_per_launch": 1.0 + index / 7.0, "min_ms_per_launch": 1.0, "median_ms_per_launch": 1.0,
            "value_at_min": value, "value_at_median": value, "sub_batches": 10, "launches_per_sub_batch": 2,
            "warmup_launches": 200, "warmup_device_ms": 250.0, "algorithmic_work_per_launch": 4.398046511104e12,
            "work_unit": "flop", "traffic_bytes_per_launch": 1.23456789e9, "dtype": "bf16",
            "clock": {"clock_mhz": 2011.123, "witness_ms": 100.0, "polls": 753762, "load_launches": 200,
                      "method": "mb_clock_witness: s_memtime cycles / s_memrealtime ticks of one wave beside the "
                                "kernel's launches"},
            "power": {"mean_w": 1399.87654, "seconds": 2.0000001, "host_seconds": 2.0001, "updates": 3,
                      "cap_w": 1400.0, "method": "m" * 200},
            "frac_at_clock": 0.97, "config": {"text": "c" * 400}, "validation": "v" * 1500})
        if name == "hbm_copy":
            rows[-1].update(rw_bound_frac=0.88765432, frac_of_rw_bound=0.9567891,
                            context={"read_only_gbps": 7123.456789, "method": "m" * 300})
    return rows


def _fake_document():
    args = argparse.Namespace(steps=20, warmup=5, warmup_ms=250.0, sub_batch_ms=2.0)
    info = {"name": "AMD Instinct MI355X", "arch": "gfx950:sramecc+:xnack-", "compute_units": 256}
    rows = _fake_rows()
    cpu_rows = [{"name": r["name"], "value": 1.2345678, "unit": r["unit"], "cores": 16, "method": "m" * 300,
                 "sample": "s" * 2000, "frac_of_mi355x_peak": 1e-3} for r in rows]
    host = {"cpu_model": "AMD EPYC 9575F 64-Core Processor", "usable_cpus": 16}
    return bench.full_document(args, info, rows, cpu_rows, host)


def test_line_of_a_full_row_set_stays_under_the_bound():
    line = bench.headline_line(_fake_document(), "results/bench_detail.json")
    encoded = json.dumps(line).encode()
    assert len(encoded) <= bench.MAX_LINE_BYTES == 8192, len(encoded)
    # Room to spare: the real rows are no longer than the fake ones.
    assert len(encoded) <= 6500, len(encoded)


def test_line_keeps_the_contract_fields_and_every_row():
    document = _fake_document()
    line = bench.headline_line(document, "results/bench_detail.json")
    assert CONTRACT <= set(line)
    assert line["n_gpus"] == 1 and line["steps"] == 20 and line["warmup"] == 5
    assert line["detail"] == "results/bench_detail.json"
    assert "workload" in line["config"] and "model" not in line["config"]
    assert [r["name"] for r in line["rows"]] == [r["name"] for r in document["rows"]]
    for row in line["rows"]:
        assert {"name", "kernel", "value", "unit", "frac", "ms_per_launch", "in_headline", "clock_mhz",
                "frac_at_clock"} <= set(row)
    headline = [r for r in document["rows"] if r["in_headline"]]
    assert line["value"] == pytest.approx(100 * sum(r["frac"] for r in headline) / len(headline), rel=1e-4)
    roofline = line["roofline"]
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic", "kernel", "algorithmic_work_per_launch",
            "ms_per_launch"} <= set(roofline)
    assert roofline["frac"] == pytest.approx(roofline["achieved"] / roofline["peak"], rel=1e-4)
    dominant = max(headline, key=lambda r: r["ms_per_launch"])
    assert roofline["row"] == dominant["name"]
    cpu = line["cpu_baseline"]
    assert {"value", "unit", "cores", "kind", "sample"} <= set(cpu)
    assert len(cpu["sample"]) <= 200 and cpu["kind"] == "port" and cpu["cores"] == 16


def test_line_falls_back_to_bare_rows_before_it_outgrows_the_bound(monkeypatch):
    monkeypatch.setattr(bench, "MAX_LINE_BYTES", 3000)
    line = bench.headline_line(_fake_document(), "results/bench_detail.json")
    assert len(json.dumps(line).encode()) <= 3000
    assert all(set(row) == {"name", "frac"} for row in line["rows"])
    assert CONTRACT <= set(line)


def test_rounding_keeps_significant_digits():
    assert bench._round(2283.987654) == 2284.0
    assert bench._round(0.000123456789) == pytest.approx(0.00012346)
    assert bench._round(None) is None and bench._round(7) == 7
    assert math.isnan(bench._round(float("nan")))


def test_power_meter_takes_the_mean_between_counter_updates_inside_the_load():
    """stop(): the first sample is the counter as found (its last update precedes the load) and is skipped; the
    power is the energy difference (uJ) over the time-stamp difference (ns) of the first and last updates after it;
    fewer than two updates give no figure."""
    import threading

    meter = bench.PowerMeter.__new__(bench.PowerMeter)
    meter.cap_w = 1400.0

    def stopped(samples):
        meter._samples, meter._stop = samples, threading.Event()
        meter._thread = threading.Thread(target=lambda: None)
        meter._thread.start()
        return meter.stop()

    found = (5.0e9, 1_000_000_000, 0.0)
    updates = [(5.0e9 + 1.4e9, 2_000_000_000, 1.0), (5.0e9 + 2.8e9, 3_000_000_000, 2.0),
               (5.0e9 + 4.2e9, 4_000_000_000, 3.0)]
    result = stopped([found, *updates])
    assert result["mean_w"] == pytest.approx(1400.0) and result["seconds"] == pytest.approx(2.0)
    assert result["updates"] == 3 and result["cap_w"] == 1400.0 and result["host_seconds"] == pytest.approx(2.0)
    assert stopped([found, updates[0]]) is None
    assert stopped([]) is None


def test_roofline_block_carries_the_dominant_kernels_clock_and_power():
    line = bench.headline_line(_fake_document(), "results/bench_detail.json")
    dominant = max((r for r in _fake_rows() if r["in_headline"]), key=lambda r: r["ms_per_launch"])
    roofline = line["roofline"]
    assert roofline["kernel"] == dominant["kernel"] and roofline["row"] == dominant["name"]
    assert roofline["clock_mhz"] == pytest.approx(dominant["clock"]["clock_mhz"], rel=1e-4)
    assert roofline["frac_at_clock"] == pytest.approx(dominant["frac_at_clock"], rel=1e-4)
    assert roofline["power_w"] == pytest.approx(dominant["power"]["mean_w"], rel=1e-4)
