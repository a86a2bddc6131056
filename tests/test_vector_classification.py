"""CPU tests of how bench_vector classifies each vector configuration.

The reference's vector benchmark (bench_vector.py:623-799, 1054-1268;
tests/test_vector_dtypes.py, tests/test_vector_compilation.py) keeps rates
only from kernels whose assembly passes the audit and whose output passes the
closed-form check: an audit rejection excludes the configuration (and makes
the row "unsupported" when nothing is left), a spilling kernel is excluded,
and a wrong result is an error. The native launch, the instruction listing
and the timer are stand-ins here; the launch stand-in computes the chains with
the oracle, so the real validation code judges real recurrences.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import vector as ov
from triton_chip_benchmarks_amd import bench_vector as bv

NATIVE_FP32 = ["v_fma_f32 v0, v1, s2, v0"]


def _args(tmp_path, dtype):
    parser = bv.build_parser()
    args = parser.parse_args(["--dtype", dtype, "--iterations", "8", "--blocks-per-sm", "1", "--block-sizes", "64",
                              "--unroll", "1", "--no-cpu-baseline", "--output", str(tmp_path / "vector.json")])
    bv.configure_sweep(args)
    return args


class _Library:
    @staticmethod
    def mb_vector_kernel_name(kind, unroll):
        return f"vector_stand_in_{kind}_u{unroll}".encode()


@pytest.fixture
def stand_ins(monkeypatch):
    state = {"timed": 0, "corrupt": False, "listing": list(NATIVE_FP32), "spills": 0}

    def launch(kind, inputs, output, coefficients, iterations, unroll, block, regime_checked=False):
        assert kind == "fp32", kind
        result = ov.run_chains("fp32", inputs.numpy(), coefficients.numpy(), iterations)
        if state["corrupt"]:
            result = np.array(result, copy=True)
            result.flat[5] += 1e-3
        output.copy_(torch.from_numpy(np.asarray(result)).to(output.dtype))

    def measure(fn, args):
        state["timed"] += 1
        return {"median_ms": 2.0, "min_ms": 1.0, "timing_method": "stand-in"}

    monkeypatch.setattr(bv, "get_device", lambda args: "cpu")
    monkeypatch.setattr(bv, "available_memory_bytes", lambda: None)
    monkeypatch.setattr(bv._native, "load", lambda: _Library())
    monkeypatch.setattr(bv, "launch_vector", launch)
    monkeypatch.setattr(bv, "measure", measure)
    monkeypatch.setattr(bv.audit, "instructions", lambda kernel: list(state["listing"]))
    monkeypatch.setattr(bv.audit, "resources",
                        lambda kernel: {"registers_per_thread": 32, "register_spills": state["spills"]})
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *args, **kwargs: None)
    return state


def _run(tmp_path, dtype="fp32"):
    args = _args(tmp_path, dtype)
    bv.run_benchmark(args, {"sm_count": 2})
    return json.loads((tmp_path / "vector.json").read_text())


def test_audited_and_correct_kernel_is_timed_with_reference_op_counts(tmp_path, stand_ins):
    document = _run(tmp_path)
    assert document["status"] == "ok" and stand_ins["timed"] == 1
    row = document["results"][0]
    assert row["native_arithmetic_verified"] is True
    # 2 flops per update x 8 chains x elements (1 WG/CU x 2 CUs x 64 lanes) x 8 iterations.
    assert row["counted_flops"] == 2 * 8 * (2 * 64) * 8
    assert row["peak_tflops"] == pytest.approx(row["counted_flops"] / 1e9)


def test_kernel_without_native_instruction_is_unsupported_and_never_timed(tmp_path, stand_ins):
    stand_ins["listing"] = ["v_mul_f32 v0, v1, v2", "v_add_f32 v0, v0, v3"]
    with pytest.raises(bv.UnsupportedVectorDtype, match="v_fma|native"):
        bv.run_benchmark(_args(tmp_path, "fp32"), {"sm_count": 2})
    assert stand_ins["timed"] == 0


def test_matrix_instruction_in_a_vector_kernel_is_excluded(tmp_path, stand_ins):
    stand_ins["listing"] = NATIVE_FP32 + ["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]"]
    with pytest.raises(bv.UnsupportedVectorDtype, match="matrix"):
        bv.run_benchmark(_args(tmp_path, "fp32"), {"sm_count": 2})
    assert stand_ins["timed"] == 0


def test_spilling_kernel_is_excluded_and_nothing_is_reported(tmp_path, stand_ins):
    stand_ins["spills"] = 4
    with pytest.raises(RuntimeError, match="spills"):
        bv.run_benchmark(_args(tmp_path, "fp32"), {"sm_count": 2})
    assert stand_ins["timed"] == 0


def test_wrong_result_is_an_error_before_timing(tmp_path, stand_ins):
    stand_ins["corrupt"] = True
    with pytest.raises(RuntimeError, match="correctness failed"):
        _run(tmp_path)
    assert stand_ins["timed"] == 0
    assert not (tmp_path / "vector.json").exists()


def test_bf16_dot2_refuses_operands_outside_its_bounded_regime():
    """The dot2 form reads the sibling chain times zero, so it runs only where every chain stays finite."""
    import torch

    from triton_chip_benchmarks_amd import bench_vector, roofline

    inputs = torch.full((8, 64), 0.5, dtype=torch.bfloat16)
    ok = torch.tensor([-1.0] + [0.125] * 8, dtype=torch.bfloat16)
    assert bench_vector.dot2_regime_reason(inputs, ok, 4096) is None
    grows = ok.clone()
    grows[0] = 1.5
    assert "|a|" in bench_vector.dot2_regime_reason(inputs, grows, 4096)
    infinite = inputs.clone()
    infinite[3, 7] = float("inf")
    assert "non-finite" in bench_vector.dot2_regime_reason(infinite, ok, 4096)
    with pytest.raises(ValueError, match="bf16_fma"):
        bench_vector.launch_vector("bf16_dot2", infinite, infinite.clone(), ok, 16, 16, 64)
    ceiling, basis = roofline.ISSUED_CEILINGS["vector_bf16"]
    assert ceiling == pytest.approx(256 * 2.4e9 * 256 / 3 / 1e12) and "1.5" in basis


def test_bf16_dot2_regime_is_checked_once_outside_the_timed_launches(tmp_path, monkeypatch):
    """The dot2 operand check reads the operands back to the host, which a graph
    capture forbids and which would add device work to the timed region: the
    suite checks each operand set once, for the longest run it makes (the odd
    iteration probe), and every launch it times skips the check."""
    calls, launches = [], []
    real_reason = bv.dot2_regime_reason

    def reason(inputs, coefficients, iterations):
        calls.append(iterations)
        return real_reason(inputs, coefficients, iterations)

    def launch(kind, inputs, output, coefficients, iterations, unroll, block, regime_checked=False):
        launches.append((kind, regime_checked))
        result = ov.run_chains("bf16", inputs.float().numpy(), coefficients.float().numpy(), iterations)
        output.copy_(torch.from_numpy(np.asarray(result)).to(output.dtype))

    monkeypatch.setattr(bv, "get_device", lambda args: "cpu")
    monkeypatch.setattr(bv, "available_memory_bytes", lambda: None)
    monkeypatch.setattr(bv._native, "load", lambda: _Library())
    monkeypatch.setattr(bv, "dot2_regime_reason", reason)
    monkeypatch.setattr(bv, "launch_vector", launch)
    monkeypatch.setattr(bv, "measure", lambda fn, args: (fn(), {"median_ms": 2.0, "min_ms": 1.0,
                                                                "timing_method": "stand-in"})[1])
    monkeypatch.setattr(bv.audit, "instructions", lambda kernel: ["v_dot2_f32_bf16 v0, v1, v2, v0"])
    monkeypatch.setattr(bv.audit, "resources", lambda kernel: {"registers_per_thread": 32, "register_spills": 0})
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *args, **kwargs: None)
    bv.run_benchmark(_args(tmp_path, "bf16"), {"sm_count": 1})
    dot2 = [checked for kind, checked in launches if kind == "bf16_dot2"]
    assert dot2 and all(dot2), launches
    assert calls == [9]  # --iterations 8, plus the odd-iteration probe
