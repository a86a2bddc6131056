"""GPU smoke test of the cross-implementation check (suite kernels against
hipMemcpy device-to-device and torch's library GEMMs on the same card)."""

import json

import pytest

pytestmark = pytest.mark.gpu


def test_crosscheck_quick_runs_both_paths_and_they_agree(gpu, tmp_path, capsys):
    from triton_chip_benchmarks_amd import crosscheck

    output = tmp_path / "crosscheck.json"
    assert crosscheck.main(["--quick", "--output", str(output)]) == 0
    document = json.loads(output.read_text())
    rows = document["results"]
    copy_paths = {row["path"] for row in rows if row["check"] == "copy"}
    assert copy_paths == {"mb_copy", "hipMemcpyDtoD"}
    ours = [row for row in rows if row["check"] == "gemm" and row["path"] == "mb_gemm"]
    assert {row["dtype"] for row in ours} == {"bf16", "fp16", "fp8", "int8", "fp4", "fp64", "fp32"}
    for row in ours:
        assert row["peak_teraops_per_second"] > 0
    library = {row["dtype"]: row for row in rows if row["check"] == "gemm" and row["path"] != "mb_gemm"}
    for dtype in ("bf16", "fp16", "fp32", "fp64"):
        assert library[dtype].get("status") != "unavailable"
    for row in ours:
        if row.get("library_output") == "bf16":      # MXFP4: torch's path writes a BF16 C
            assert row["elementwise_within_one_bf16_ulp"] and row["max_bf16_ulps"] <= 1.0
        elif row["normwise_difference"] is not None:
            assert row["normwise_difference"] <= {"bf16": 1e-2, "fp16": 1e-2, "fp32": 2e-3,
                                                  "fp64": 1e-12}.get(row["dtype"], 1e-6)
