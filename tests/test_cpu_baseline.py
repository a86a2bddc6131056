"""CPU tests of the host baseline timed beside each row (triton_chip_benchmarks_amd.cpu_baseline).

The baseline is the reference's host computation for the row (torch matmul for
tensor rows, the vectorised recurrence for vector rows, a tensor copy for
bandwidth), timed with the host clock on a bounded sample. It is product code
that never touches the test oracle and never produces a device value.
"""

from __future__ import annotations

import ast
import math
from pathlib import Path

import pytest

from triton_chip_benchmarks_amd import cpu_baseline

MODULE = Path(cpu_baseline.__file__)


def _check(result, unit):
    assert result["unit"] == unit
    assert math.isfinite(result["value"]) and result["value"] > 0
    assert result["cores"] >= 1 and result["timer"] == "time.perf_counter"
    host = result["host"]
    assert host["os_cpu_count"] >= 1 and host["torch_threads"] >= 1


def test_copy_baseline_counts_read_and_write_bytes():
    result = cpu_baseline.copy_baseline(8 * 2**20, budget_s=0.05)
    _check(result, "GB/s")
    assert "8 MiB fp32" in result["sample"]


@pytest.mark.parametrize("dtype,unit", [("bf16", "TFLOP/s"), ("fp64", "TFLOP/s"), ("int8", "TOPS"),
                                        ("fp4", "TFLOP/s")])
def test_matmul_baseline_uses_the_references_check_arithmetic(dtype, unit):
    result = cpu_baseline.matmul_baseline(dtype, 128, budget_s=0.05)
    _check(result, unit)
    assert ("float64" in result["method"]) == (dtype == "fp64")
    assert ("upcast" in result["method"]) == (dtype not in ("fp32", "fp64"))


@pytest.mark.parametrize("dtype", ["bf16", "fp64", "fp4"])
def test_gemm_sample_and_tile_batch_baselines(dtype):
    result = cpu_baseline.gemm_sample_baseline(dtype, 16, 96, 64, budget_s=0.05)
    _check(result, "TFLOP/s")
    assert "16x96x64 (rows of A sampled)" in result["sample"]
    assert ("float64" in result["method"]) == (dtype == "fp64")
    tiles = cpu_baseline.tile_batch_baseline(dtype, 4, 32, 32, 16, budget_s=0.05)
    _check(tiles, "TFLOP/s")
    assert "4 tiles of 32x32x16" in tiles["sample"]


@pytest.mark.parametrize("dtype,unit", [("fp32", "TFLOP/s"), ("fp64", "TFLOP/s"), ("fp16", "TFLOP/s"),
                                        ("bf16", "TFLOP/s"), ("int8", "TOPS")])
def test_vector_baseline_runs_every_format(dtype, unit):
    result = cpu_baseline.vector_baseline(dtype, 1024, 3, budget_s=0.05)
    _check(result, unit)
    assert "8 chains x 1024 lanes x 3 iterations" in result["sample"]


def test_dp4a_step_matches_a_scalar_byte_loop():
    import torch

    words = torch.tensor([0x7F80FF01, -1, 0, 0x01020304, -0x80000000], dtype=torch.int32)
    weights = (3, -2, 1, -1)
    bias = torch.full_like(words, 5)
    got = cpu_baseline._dp4a_step(words, weights, bias)
    for word, value in zip(words.tolist(), got.tolist()):
        raw = word & 0xFFFFFFFF
        signed = [((raw >> (8 * j)) & 0xFF) - 256 * (((raw >> (8 * j)) & 0xFF) > 127) for j in range(4)]
        expected = (sum(b * w for b, w in zip(signed, weights)) + 5 + 2**31) % 2**32 - 2**31
        assert value == expected, (hex(raw), value, expected)


def test_baseline_module_never_imports_the_oracle():
    tree = ast.parse(MODULE.read_text())
    imported = {alias.name for node in ast.walk(tree) if isinstance(node, ast.Import) for alias in node.names}
    imported |= {node.module or "" for node in ast.walk(tree) if isinstance(node, ast.ImportFrom)}
    assert not any(name.split(".")[0] == "oracle" for name in imported)
