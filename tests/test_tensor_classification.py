"""CPU tests of how bench_tensor classifies each resident-peak configuration.

The reference keeps four outcomes apart (bench_tensor.py:96-142, 1149-1308;
tests/test_tensor_formats.py): a compiler or instruction-audit rejection is
"unsupported" and never reaches the timer; a wrong result is an error and is
never relabelled "unsupported"; a configuration that spills registers is
skipped; a valid one is timed and reported. Here the native launch, the audit
and the timer are replaced by stand-ins on CPU tensors, so only that
classification logic runs.
"""

from __future__ import annotations

import json

import pytest
import torch

from triton_chip_benchmarks_amd import bench_tensor as bt

CONFIG = {"tile_m": 32, "tile_n": 32, "tile_k": 16, "chains": 2, "b_nk": 0, "mfma_m": 32, "threads": 256}
AUDITED = {"spill_count": 0, "register_spills": 0, "registers_per_thread": 64, "execution_kind": "tensor",
           "native_tensor_verified": True, "instruction_precision_verified": True}


def _args(tmp_path, dtype="bf16"):
    parser = bt.build_parser()
    args = parser.parse_args(["--dtype", dtype, "--blocks-per-sm", "1", "--iterations", "3", "--no-cpu-baseline",
                              "--output", str(tmp_path / "tensor.json")])
    bt.normalize_precision_args(parser, args)
    args.tiles = None
    return args


@pytest.fixture
def stand_ins(monkeypatch):
    """Native launch writes the exact product (optionally corrupted); the timer records its calls."""
    state = {"timed": 0, "corrupt": False, "info": dict(AUDITED), "audit_error": None}

    def launch(dtype, config, a, b, c, iterations, scales=None):
        b_logical = b.transpose(-1, -2) if config.get("b_nk") else b
        result = bt.exact_reference(a, b_logical, iterations, c.dtype)
        if state["corrupt"]:
            result.view(-1)[0] += 1
        c.copy_(result)

    def compiled_info(kernel, dtype, input_precision):
        if state["audit_error"]:
            raise bt.TensorUnsupportedError(state["audit_error"])
        return dict(state["info"])

    def measure(fn, args):
        state["timed"] += 1
        return {"median_ms": 2.0, "min_ms": 1.0, "timing_method": "stand-in"}

    monkeypatch.setattr(bt, "peak_configs", lambda dtype, layout: [dict(CONFIG)])
    monkeypatch.setattr(bt._native, "peak_kernel_name", lambda dtype, config: "tensor_peak_stand_in")
    monkeypatch.setattr(bt, "available_memory_bytes", lambda: None)
    monkeypatch.setattr(bt, "launch_peak", launch)
    monkeypatch.setattr(bt, "compiled_info", compiled_info)
    monkeypatch.setattr(bt, "measure", measure)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *args, **kwargs: None)
    return state


def _run(tmp_path, dtype="bf16"):
    args = _args(tmp_path, dtype)
    bt.run_peak(args, {"sm_count": 2}, "cpu")
    return json.loads((tmp_path / "tensor.json").read_text())


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "int8", "fp64"])
def test_valid_configuration_is_timed_and_counts_every_operation(tmp_path, stand_ins, dtype):
    document = _run(tmp_path, dtype)
    assert document["status"] == "ok" and stand_ins["timed"] == 1
    row = document["results"][0]
    assert row["status"] == "ok" and row["correctness"]["passed"]
    # 2 * M * N * K * iterations * chains * blocks, blocks = 1 per CU x 2 CUs.
    assert row["operation_count"] == 2 * 32 * 32 * 16 * 3 * 2 * 2
    assert row["peak_teraops_per_second"] == pytest.approx(row["operation_count"] / 1e9)
    assert ("peak_tops" in row) == (dtype == "int8") and ("peak_tflops" in row) == (dtype != "int8")


def test_audit_rejection_is_unsupported_and_never_timed(tmp_path, stand_ins):
    stand_ins["audit_error"] = "Generated AMDGCN does not contain v_mfma_f32_32x32x16_bf16"
    document = _run(tmp_path)
    assert document["status"] == "unsupported" and stand_ins["timed"] == 0
    assert "v_mfma_f32_32x32x16_bf16" in document["reason"]
    assert document["results"] == []
    assert all(row["status"] == "unsupported" and "peak_teraops_per_second" not in row
               for row in document["details"])


def test_wrong_result_is_an_error_not_unsupported(tmp_path, stand_ins):
    stand_ins["corrupt"] = True
    with pytest.raises(AssertionError):
        _run(tmp_path)
    assert stand_ins["timed"] == 0
    assert not (tmp_path / "tensor.json").exists()


def test_spilling_configuration_is_skipped_and_the_invocation_fails(tmp_path, stand_ins):
    stand_ins["info"]["spill_count"] = 12
    with pytest.raises(RuntimeError, match="spills registers"):
        _run(tmp_path)
    assert stand_ins["timed"] == 0


def test_measured_document_carries_the_host_matmul_baseline(tmp_path, stand_ins):
    args = _args(tmp_path)
    args.no_cpu_baseline, args.quick = False, True
    bt.run_peak(args, {"sm_count": 2}, "cpu")
    document = json.loads((tmp_path / "tensor.json").read_text())
    baseline = document["cpu_baseline"]
    assert baseline["unit"] == "TFLOP/s" and baseline["value"] > 0 and baseline["cores"] >= 1
    assert "torch.matmul" in baseline["method"] and "256x256x256" in baseline["sample"]
