"""CPU tests of the 17-row report contract, the suite runner and the child documents.

The behaviours pinned here are the reference's (tests/test_suite.py,
suite_report.py:88-148, bench_suite.py:99-199): selection of the highest
valid peak with its own median, explicit statuses that are never zero,
HBM-sized eligibility for the bandwidth row, isolation of child failures and a
checkpoint after every metric. No GPU is used: children are replaced by
`subprocess.run` stand-ins that write documents.
"""

from __future__ import annotations

import argparse
import contextlib
import io
import json
from pathlib import Path
import subprocess
import sys
from unittest import mock

import pytest

from oracle import memory as om
from triton_chip_benchmarks_amd import bench_suite as suite
from triton_chip_benchmarks_amd import common, roofline
from triton_chip_benchmarks_amd.bench_bandwidth import cache_regime
from triton_chip_benchmarks_amd.suite_report import METRICS, empty_metric, format_table, summarize

ROOT = Path(__file__).resolve().parent.parent


def metric(key):
    return next(item for item in METRICS if item.key == key)


# ---- the table --------------------------------------------------------------

def test_seventeen_rows_in_reference_order_with_units():
    assert len(METRICS) == 17
    keys = [m.key for m in METRICS]
    assert keys[:2] == ["memory_capacity", "memory_bandwidth"]
    assert [m.precision for m in METRICS if m.group == "Tensor"] == [
        "bf16", "fp16", "fp32", "tf32", "int8", "fp64", "fp8", "fp4"]
    assert [m.precision for m in METRICS if m.group == "Vector"] == [
        "bf16", "fp16", "fp32", "int8", "fp64", "fp8", "fp4"]
    for m in METRICS:
        expected = {"memory_capacity": "GiB", "memory_bandwidth": "GB/s"}.get(
            m.key, "TOP/s" if m.precision == "int8" else "TFLOP/s")
        assert m.unit == expected, m.key


def test_every_measured_row_has_an_mi355x_peak():
    for m in METRICS:
        if m.key == "memory_capacity":
            continue
        if m.key in ("tensor_tf32", "vector_fp8", "vector_fp4"):
            continue  # no gfx950 instruction; the row is a status, never a rate
        value, unit, basis = roofline.PEAKS[m.key]
        assert value > 0 and basis
        assert unit == m.unit


def test_capacity_in_gib_and_missing_capacity_is_unavailable():
    item = metric("memory_capacity")
    row = summarize(item, {"device": {"total_memory_bytes": 288 * 2**30}})
    assert (row["status"], row["value"], row["unit"]) == ("ok", 288, "GiB")
    missing = summarize(item, {"device": {"total_memory_bytes": None}})
    assert missing["status"] == "unavailable" and missing["value"] is None


def test_bandwidth_takes_the_eligible_copy_and_keeps_read_as_a_detail():
    rows = [{"pattern": "copy", "peak_gbps": 20000, "gbps": 19000, "peak_eligible": False},
            {"pattern": "copy", "peak_gbps": 6500, "gbps": 6400, "peak_eligible": True},
            {"pattern": "copy", "peak_gbps": 6300, "gbps": 6290, "peak_eligible": True},
            {"pattern": "read", "peak_gbps": 6600, "gbps": 6550, "peak_eligible": True}]
    row = summarize(metric("memory_bandwidth"), {"results": rows})
    assert (row["status"], row["value"], row["median_value"]) == ("ok", 6500, 6400)
    assert row["patterns"]["read"]["value"] == 6600
    assert row["patterns"]["copy"]["value"] == 6500
    assert row["roofline"]["frac"] == pytest.approx(6500 / 8000)


@pytest.mark.parametrize("eligible,smoke", [(False, False), (True, True)])
def test_cache_resident_or_smoke_copies_never_become_the_hbm_rate(eligible, smoke):
    row = summarize(metric("memory_bandwidth"), {"results": [
        {"pattern": "copy", "peak_gbps": 30000, "gbps": 29000, "peak_eligible": eligible, "smoke_only": smoke}]})
    assert row["status"] == "not_measured" and row["value"] is None
    assert row["patterns"]["copy"]["value"] == 30000


def test_integer_rows_read_integer_rates_only():
    item = metric("tensor_int8")
    ok = summarize(item, {"results": [{"peak_tops": 4000, "tops": 3900, "compiled": {
        "execution_kind": "tensor", "native_tensor_verified": True, "instruction_precision_verified": True}}]})
    assert (ok["status"], ok["value"], ok["unit"]) == ("ok", 4000, "TOP/s")
    wrong = summarize(item, {"results": [{"peak_tflops": 4000, "tflops": 3900}]})
    assert wrong["status"] == "error" and wrong["value"] is None


def test_unaudited_tensor_rate_is_kept_but_unverified():
    for compiled in ({"execution_kind": "tensor", "native_tensor_verified": True,
                      "instruction_precision_verified": False},
                     {"execution_kind": "unverified", "native_tensor_verified": False,
                      "instruction_precision_verified": True},
                     {}):
        row = summarize(metric("tensor_bf16"), {"arguments": {"quick": True},
                                                "results": [{"peak_tflops": 2000, "tflops": 1900,
                                                             "compiled": compiled}]})
        assert row["status"] == "unverified"
        assert (row["value"], row["median_value"]) == (2000, 1900)
        assert row["smoke_only"] is True
        assert "unverified" in format_table([row])


def test_simt_matrix_rate_keeps_its_value_and_is_labelled():
    row = summarize(metric("tensor_fp64"), {"results": [{"peak_tflops": 70, "tflops": 69, "compiled": {
        "execution_kind": "simt", "native_tensor_verified": False, "instruction_precision_verified": True}}]})
    assert (row["status"], row["value"]) == ("ok", 70)
    assert "SIMT scalar/vector instructions" in format_table([row])


def test_vector_rate_without_native_arithmetic_is_unverified():
    row = summarize(metric("vector_int8"), {"results": [{
        "peak_tops": 30, "tops": 29, "native_arithmetic_verified": False,
        "arithmetic_dtype": "int32", "includes_unpacking": True}]})
    assert row["status"] == "unverified" and row["value"] == 30
    assert "includes unpacking" in row["reason"]
    native = summarize(metric("vector_fp16"), {"results": [{
        "peak_tflops": 150, "tflops": 149, "native_arithmetic_verified": True,
        "kernel": "vector_f16_u8", "amdgcn_instruction_types": ["v_pk_fma_f16"]}]})
    assert native["status"] == "ok"
    assert native["kernel"] == "vector_f16_u8"
    assert native["amdgcn_instruction_types"] == ["v_pk_fma_f16"]


def test_statuses_are_never_zero_and_never_guessed():
    item = metric("vector_fp8")
    declared = summarize(item, {"status": "unsupported", "reason": "no FP8 VALU arithmetic on gfx950"})
    assert declared["status"] == "unsupported" and declared["value"] is None
    assert "no FP8 VALU" in format_table([declared])
    gap = summarize(item, {"status": "not_implemented", "reason": "no verified path"})
    assert gap["status"] == "not_implemented" and gap["value"] is None
    failure = summarize(item, {"results": [{"status": "error", "reason": "looks unsupported?"}]})
    assert failure["status"] == "error"
    all_rejected = summarize(item, {"results": [{"status": "unsupported", "reason": "a"},
                                                {"status": "unsupported", "reason": "b"}]})
    assert all_rejected["status"] == "unsupported" and all_rejected["reason"] == "a; b"


def test_nonfinite_or_zero_rates_never_win():
    row = summarize(metric("vector_fp64"), {"results": [
        {"peak_tflops": float("inf"), "tflops": 1}, {"peak_tflops": float("nan"), "tflops": 1},
        {"peak_tflops": 76, "tflops": 75, "native_arithmetic_verified": True},
        {"peak_tflops": 0, "tflops": 0}, {"peak_tflops": True, "tflops": True}]})
    assert row["value"] == 76 and row["successful_configurations"] == 1


def test_median_comes_from_the_winning_configuration():
    row = summarize(metric("vector_fp32"), {"results": [
        {"peak_tflops": 70, "tflops": 69.9, "unroll": 4, "native_arithmetic_verified": True},
        {"peak_tflops": 77, "tflops": 60.0, "unroll": 8, "native_arithmetic_verified": True}]})
    assert (row["value"], row["median_value"], row["configuration"]["unroll"]) == (77, 60.0, 8)


# ---- HBM eligibility ----------------------------------------------------------

@pytest.mark.parametrize("quick", [False, True])
def test_cache_regime_matches_the_oracle_at_the_boundary(quick):
    infinity_cache = roofline.INFINITY_CACHE_BYTES
    assert infinity_cache == 256 * 2**20
    for buffer_bytes in (0, 4 * infinity_cache - 1, 4 * infinity_cache, 2**31, 2**34):
        for cache_bytes in (0, None, 4 * 2**20, infinity_cache):
            got = cache_regime(buffer_bytes, cache_bytes, quick)
            assert got == om.cache_regime(buffer_bytes, cache_bytes or 0, quick)
    assert cache_regime(2**30, infinity_cache, False) == ("larger_than_l2", True)
    assert cache_regime(2**30 - 1, infinity_cache, False) == ("cache_sensitive", False)


# ---- the suite runner -----------------------------------------------------------

def _args(root, *extra):
    return suite.build_parser().parse_args(["--output", str(root / "report.json"), "--quick",
                                            "--timing", "events", *extra])


def test_child_commands_use_this_interpreter_and_explicit_precisions(tmp_path):
    args = _args(tmp_path)
    tf32 = suite.metric_command(metric("tensor_tf32"), args, Path("x.json"))
    assert tf32[0] == sys.executable and Path(tf32[2]).is_absolute()
    assert tf32[tf32.index("--dtype") + 1] == "fp32"
    assert tf32[tf32.index("--input-precision") + 1] == "tf32"
    assert "--quick" in tf32
    capacity = suite.metric_command(metric("memory_capacity"), args, Path("x.json"))
    assert "--probe-device" in capacity
    bandwidth = suite.metric_command(metric("memory_bandwidth"), args, Path("x.json"))
    assert Path(bandwidth[2]).name == "bench_bandwidth.py"
    assert bandwidth[bandwidth.index("--mode") + 1] == "all"
    vector = suite.metric_command(metric("vector_int8"), args, Path("x.json"))
    assert Path(vector[2]).name == "bench_vector.py"
    for command in (tf32, capacity, bandwidth, vector):
        assert (ROOT / Path(command[2]).name).exists()
    # --widened reaches only the FP8/FP4 vector children; by default no child gets it.
    assert all("--widened" not in suite.metric_command(m, args, Path("x.json")) for m in suite.METRICS)
    args.widened = True
    widened = [m.key for m in suite.METRICS if "--widened" in suite.metric_command(m, args, Path("x.json"))]
    assert widened == ["vector_fp8", "vector_fp4"]


def test_failed_child_never_reuses_an_old_success(tmp_path):
    args = _args(tmp_path)
    stale = tmp_path / "vector_fp32.json"
    stale.write_text(json.dumps({"results": [{"peak_tflops": 99, "tflops": 90}]}))
    with mock.patch.object(suite.subprocess, "run", return_value=subprocess.CompletedProcess([], 1)):
        row, _ = suite.run_metric(metric("vector_fp32"), args, tmp_path)
    assert row["status"] == "error" and row["value"] is None
    assert not stale.exists()


def _writing(document, returncode):
    def child(command, **kwargs):
        Path(command[command.index("--output") + 1]).write_text(json.dumps(document))
        return subprocess.CompletedProcess(command, returncode)
    return child


def test_timeout_is_an_error_and_declared_statuses_survive_a_nonzero_exit(tmp_path):
    args = _args(tmp_path)
    with mock.patch.object(suite.subprocess, "run", side_effect=subprocess.TimeoutExpired([], 900)):
        row, _ = suite.run_metric(metric("vector_fp8"), args, tmp_path)
    assert row["status"] == "error" and "Exceeded" in row["reason"]
    for status in ("unsupported", "not_implemented"):
        with mock.patch.object(suite.subprocess, "run",
                               side_effect=_writing({"status": status, "reason": "declared"}, 1)):
            row, _ = suite.run_metric(metric("vector_fp8"), args, tmp_path)
        assert (row["status"], row["reason"]) == (status, "declared")


def test_nonzero_exit_after_a_measurement_is_an_error_that_keeps_the_partial(tmp_path):
    args = _args(tmp_path)
    document = {"results": [{"peak_tflops": 70, "tflops": 69, "native_arithmetic_verified": True}]}
    with mock.patch.object(suite.subprocess, "run", side_effect=_writing(document, 3)):
        row, _ = suite.run_metric(metric("vector_fp64"), args, tmp_path)
    assert row["status"] == "error" and row["value"] is None
    assert row["partial_measurement"]["value"] == 70


def test_quick_success_is_smoke_and_malformed_json_is_an_error(tmp_path):
    args = _args(tmp_path)
    good = {"results": [{"peak_tflops": 150, "tflops": 149, "native_arithmetic_verified": True}]}
    with mock.patch.object(suite.subprocess, "run", side_effect=_writing(good, 0)):
        row, _ = suite.run_metric(metric("vector_fp16"), args, tmp_path)
    assert row["smoke_only"] is True
    with mock.patch.object(suite.subprocess, "run", side_effect=_writing({"device": ["not", "metadata"]}, 0)):
        row, _ = suite.run_metric(metric("memory_capacity"), args, tmp_path)
    assert row["status"] == "error" and "Invalid benchmark JSON" in row["reason"]
    with mock.patch.object(suite.subprocess, "run", side_effect=_writing([1, 2], 0)):
        row, _ = suite.run_metric(metric("vector_fp16"), args, tmp_path)
    assert row["status"] == "error"


def test_suite_checkpoints_after_every_metric_and_continues_past_errors(tmp_path):
    args = _args(tmp_path)
    seen = []

    def child(item, args, directory):
        snapshot = json.loads(args.output.read_text())
        assert len(snapshot["results"]) == 17
        assert sum(r["status"] != "pending" for r in snapshot["results"]) == len(seen)
        seen.append(item.key)
        return empty_metric(item, "error" if len(seen) == 1 else "unsupported", "stand-in"), None

    with mock.patch.object(suite, "run_metric", side_effect=child), contextlib.redirect_stdout(io.StringIO()):
        report = suite.run_suite(args)
    assert len(seen) == 17
    assert report["status"] == "complete_with_errors"
    assert "pending" not in {r["status"] for r in report["results"]}
    assert json.loads(args.output.read_text()) == report


def test_only_runs_the_selected_metrics_and_rejects_unknown_keys(tmp_path):
    args = _args(tmp_path, "--only", "tensor_fp8", "vector_int8")
    seen = []

    def child(item, args, directory):
        seen.append(item.key)
        return empty_metric(item, "unsupported", "stand-in"), None

    with mock.patch.object(suite, "run_metric", side_effect=child), contextlib.redirect_stdout(io.StringIO()):
        report = suite.run_suite(args)
    assert seen == ["tensor_fp8", "vector_int8"]
    assert sum(r["status"] == "skipped" for r in report["results"]) == 15
    with pytest.raises(SystemExit):
        suite.run_suite(_args(tmp_path, "--only", "tensor_tf64"))


# ---- child documents -------------------------------------------------------------

def test_status_documents_are_machine_readable_and_have_no_rates(tmp_path):
    args = argparse.Namespace(output=tmp_path / "child.json", timing="auto", quick=False)
    with contextlib.redirect_stdout(io.StringIO()):
        common.emit_unsupported("tensor", {"device_name": "stand-in"}, args, "gfx950 has no TF32 MFMA")
    document = json.loads(args.output.read_text())
    assert (document["status"], document["results"]) == ("unsupported", [])
    assert document["arguments"]["output"] == str(args.output)
    with contextlib.redirect_stdout(io.StringIO()):
        common.emit_not_implemented("vector", {}, args, "no path", details={"probe": "llvm-mc"})
    document = json.loads(args.output.read_text())
    assert (document["status"], document["details"]) == ("not_implemented", {"probe": "llvm-mc"})
    row = summarize(metric("vector_fp8"), document)
    assert row["status"] == "not_implemented" and row["value"] is None


def test_results_document_refuses_empty_rows_and_nonfinite_values(tmp_path):
    args = argparse.Namespace(output=tmp_path / "child.json", timing="events", quick=False)
    with pytest.raises(RuntimeError):
        common.emit_results("tensor", {}, args, [])
    with pytest.raises(ValueError), contextlib.redirect_stdout(io.StringIO()):
        common.emit_results("tensor", {}, args, [{"peak_tflops": float("nan"), "timing_method": "events"}])
    with contextlib.redirect_stdout(io.StringIO()):
        document = common.emit_results("tensor", {}, args, [{"peak_tflops": 1.0, "timing_method": "events"}])
    assert document["timing"]["methods_used"] == ["events"]
    assert json.loads(args.output.read_text())["status"] == "ok"


def test_bench_refuses_more_than_one_gpu():
    completed = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                               capture_output=True, text=True, timeout=120)
    assert completed.returncode == 2
    assert "one MI355X" in completed.stdout + completed.stderr


def test_resume_keeps_finished_rows_and_reruns_the_rest(tmp_path):
    args = _args(tmp_path)

    def first(item, args, directory):
        status = "ok" if item.key in ("memory_capacity", "tensor_fp8") else \
            "unsupported" if item.key == "tensor_tf32" else "error"
        row = empty_metric(item, status, None if status == "ok" else "stand-in")
        if status == "ok":
            row["value"] = 1.0
        return row, None

    with mock.patch.object(suite, "run_metric", side_effect=first), contextlib.redirect_stdout(io.StringIO()):
        suite.run_suite(args)
    rerun = []

    def second(item, args, directory):
        rerun.append(item.key)
        return empty_metric(item, "not_implemented", "second pass"), None

    resumed_args = _args(tmp_path, "--resume")
    with mock.patch.object(suite, "run_metric", side_effect=second), contextlib.redirect_stdout(io.StringIO()):
        report = suite.run_suite(resumed_args)
    kept = {"memory_capacity", "tensor_fp8", "tensor_tf32"}
    assert set(rerun) == {m.key for m in METRICS} - kept
    by_key = {row["metric"]: row for row in report["results"]}
    assert by_key["tensor_fp8"]["resumed"] is True and by_key["tensor_fp8"]["value"] == 1.0
    assert by_key["tensor_tf32"]["status"] == "unsupported"
    assert by_key["vector_fp32"]["status"] == "not_implemented"


def test_resume_ignores_a_report_of_another_mode_or_shape(tmp_path):
    path = tmp_path / "report.json"
    path.write_text(json.dumps({"schema_version": 1, "smoke_only": False,
                                "results": [{"metric": m.key, "status": "ok"} for m in METRICS]}))
    assert suite.resumable_rows(path, quick=True) == {}          # full report, smoke run
    assert len(suite.resumable_rows(path, quick=False)) == 17
    path.write_text(json.dumps({"schema_version": 1, "smoke_only": False,
                                "results": [{"metric": "memory_capacity", "status": "ok"}]}))
    assert suite.resumable_rows(path, quick=False) == {}         # not the 17-row table
    path.write_text("not json")
    assert suite.resumable_rows(path, quick=False) == {}
    assert suite.resumable_rows(tmp_path / "missing.json", quick=False) == {}


def test_widened_measurement_is_a_detail_never_the_row_value():
    document = {"status": "not_implemented", "reason": "no FP8 VALU arithmetic",
                "details": {"widened": {"peak_tflops": 30.0, "tflops": 29.0,
                                        "arithmetic_kind": "converted_fp32_fma_fp8_e4m3_state"}}}
    row = summarize(metric("vector_fp8"), document)
    assert row["status"] == "not_implemented" and row["value"] is None
    assert row["widened_measurement"]["peak_tflops"] == 30.0
    table = format_table([row])
    assert "widened" in table and "not native" in table


@pytest.mark.parametrize("script", ["bench_tensor.py", "bench_vector.py", "bench_bandwidth.py", "bench_suite.py",
                                    "crosscheck.py"])
def test_package_scripts_import_when_run_directly(script):
    """Each benchmark module also runs as a plain script (its own import branch)."""
    completed = subprocess.run([sys.executable, str(ROOT / "triton_chip_benchmarks_amd" / script), "--help"],
                               capture_output=True, text=True, timeout=120, check=False)
    assert completed.returncode == 0, completed.stderr[-2000:]
    assert "usage" in completed.stdout


def test_measured_rows_carry_the_host_baseline_and_the_table_lists_it():
    baseline = {"value": 1.5, "unit": "TFLOP/s", "cores": 16, "method": "torch.matmul on the host in float32",
                "sample": "2048x2048x2048; best of 5 host runs", "host": {"cpu_model": "Test CPU"}}
    document = {"status": "ok", "cpu_baseline": baseline,
                "results": [{"status": "ok", "peak_teraops_per_second": 2000.0,
                             "median_teraops_per_second": 1990.0,
                             "compiled": {"execution_kind": "tensor", "native_tensor_verified": True,
                                          "instruction_precision_verified": True}}]}
    row = summarize(metric("tensor_bf16"), document)
    assert row["status"] == "ok" and row["cpu_baseline"] == baseline
    declared = summarize(metric("tensor_tf32"), {"status": "unsupported", "reason": "no xf32",
                                                "cpu_baseline": baseline})
    assert "cpu_baseline" not in declared
    table = format_table([row, declared])
    assert "Host CPU baseline" in table and "Test CPU" in table and "torch.matmul" in table


@pytest.mark.parametrize("block", [256, 1024])
def test_read_check_agrees_with_the_oracle_on_whole_and_tail_blocks(block):
    """bench_bandwidth.check_read (run on CPU tensors) and oracle.memory.check_read give the same
    verdict: exact sums pass, and an error just past the bound fails in a whole block, in the
    partial tail block, and as NaN."""
    import numpy as np
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import check_read

    rng = np.random.default_rng(block)
    values = rng.uniform(-1, 1, 7 * block + 37).astype(np.float32)
    sums = om.block_sums(values, block)
    bound = om.read_tolerance(values, block)

    def verdicts(sink):
        product = oracle = True
        try:
            check_read(torch.from_numpy(values), torch.from_numpy(sink.astype(np.float32)), block)
        except AssertionError:
            product = False
        try:
            om.check_read(values, sink.astype(np.float32), block)
        except AssertionError:
            oracle = False
        return product, oracle

    assert verdicts(sums) == (True, True)
    for index in (2, len(sums) - 1):  # a whole block, then the partial tail block
        broken = sums.copy()
        broken[index] += 4 * bound[index]
        assert verdicts(broken) == (False, False)
    broken = sums.copy()
    broken[1] = np.nan
    assert verdicts(broken) == (False, False)


def test_summary_tie_breaks_rejections_and_row_shape():
    """Equal peaks keep the first configuration (its median with it); a run whose rows all declared
    `unsupported` is unsupported, a mixed or empty one an error with the distinct reasons in order; a declared
    status keeps the child's reason even when it is None; the memory row lists its patterns copy, then read."""
    item = metric("tensor_bf16")
    compiled = {"execution_kind": "tensor", "native_tensor_verified": True, "instruction_precision_verified": True}
    tie = summarize(item, {"results": [{"peak_tflops": 100, "tflops": 90, "block_size": 1, "compiled": compiled},
                                       {"peak_tflops": 100, "tflops": 95, "block_size": 2, "compiled": compiled},
                                       {"peak_tflops": 0, "tflops": 99}]})
    assert (tie["value"], tie["median_value"], tie["configuration"]["block_size"]) == (100, 90, 1)
    assert tie["successful_configurations"] == 2
    unsupported = summarize(item, {"results": [{"status": "unsupported", "reason": "a"},
                                               {"status": "unsupported", "reason": "b"}, "not a row"]})
    assert (unsupported["status"], unsupported["reason"]) == ("unsupported", "a; b")
    mixed = summarize(item, {"results": [{"status": "unsupported", "reason": "a"}, {"status": "error", "reason": "b"},
                                         {"status": "error", "reason": "a"}]})
    assert (mixed["status"], mixed["reason"]) == ("error", "a; b")
    empty = summarize(item, {"results": []})
    assert (empty["status"], empty["reason"]) == ("error", "Benchmark produced no valid throughput measurements")
    assert summarize(item, {"results": {}})["reason"] == "Benchmark results must be a list"
    declared = summarize(item, {"status": "error", "reason": None})
    assert "reason" in declared and declared["reason"] is None and declared["status"] == "error"
    memory = summarize(metric("memory_bandwidth"), {"results": [
        {"pattern": "read", "peak_gbps": 7000, "gbps": 6900, "peak_eligible": True},
        {"pattern": "copy", "peak_gbps": 6800, "gbps": 6700, "peak_eligible": True}]})
    assert list(memory["patterns"]) == ["copy", "read"]
    assert list(memory)[:7] == ["metric", "group", "precision", "unit", "status", "value", "median_value"]
