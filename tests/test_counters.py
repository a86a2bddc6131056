"""CPU tests of the counter recipe's summary (triton_chip_benchmarks_amd.counters).

A synthetic rocprofv3 counter CSV with known values checks each derived
figure against its formula worked by hand: clock, MFMA busy, VALU issue
utilisation, wave waits, L2 hit rate, and HBM bytes calibrated against the
1 GiB copy; plus the demangled-name mapping and attaching summaries to rows.
"""

import csv
import json

import pytest

from triton_chip_benchmarks_amd import counters

COPY = ("void mb::(anonymous namespace)::copy_kernel<unsigned int __vector(4), 1, 2>"
        "(unsigned int __vector(4) const*, unsigned int __vector(4)*, unsigned long)")
GEMM = ("void mb::(anonymous namespace)::gemm_dma_kernel<mb::MfmaBf16x16>(unsigned char const*, "
        "unsigned char const*, unsigned char const*, unsigned char const*, mb::MfmaBf16x16::Out*, int, int, int, int)")
FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
          "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
          "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _write_pass(directory, records):
    directory.mkdir(parents=True)
    with (directory / "run_counter_collection.csv").open("w", newline="") as stream:
        writer = csv.DictWriter(stream, FIELDS)
        writer.writeheader()
        for dispatch, kernel, counter, value, duration_ns, *grid in records:
            row = dict.fromkeys(FIELDS, 0)
            row.update(Dispatch_Id=dispatch, Kernel_Name=kernel, Counter_Name=counter, Counter_Value=value,
                       Start_Timestamp=1000, End_Timestamp=1000 + duration_ns)
            if grid:
                row.update(Grid_Size=grid[0], Workgroup_Size=grid[1])
            writer.writerow(row)


def test_registered_names_of_demangled_kernels():
    assert counters.registered_name(COPY) == "copy_dwordx4_vpt1_stream"
    assert counters.registered_name(GEMM) == "gemm_bf16_256x256x64"
    assert counters.registered_name(
        "void mb::(anonymous namespace)::tensor_peak_kernel<mb::MfmaMxfp4, 128, 128, 256, 2, 2, 2, false>"
        "(unsigned char const*)") == "tensor_peak_mxfp4_128x128x256_c2_kn"
    assert counters.registered_name(
        "void mb::(anonymous namespace)::tensor_peak_kernel<mb::MfmaBf16x16, 128, 128, 64, 2, 2, 2, true>"
        "(unsigned char const*)") == "tensor_peak_bf16_128x128x64_c2_mfma16_nk"
    assert counters.registered_name(
        "void mb::(anonymous namespace)::gemm_kernel<mb::MfmaF64, 64, 64, 16, 2, 2, true>(int)") == \
        "gemm_f64_64x64x16_checked"
    assert counters.registered_name("void mb::(anonymous namespace)::vector_dot4_kernel<16>(int const*)") == \
        "vector_dot4_u16"
    assert counters.registered_name("Cijk_Alik_Bljk_BBS_BH(int)") == "Cijk_Alik_Bljk_BBS_BH"
    # A name the profiler left mangled maps through the symbol parser.
    assert counters.registered_name("_ZN2mb12_GLOBAL__N_117vector_f16_kernelILi16EEEvPKDF16_PDF16_S3_mj") == \
        "vector_f16_u16"


def test_summary_formulas_and_copy_calibration(tmp_path):
    cycles_per_xcd, duration = 2_000_000, 1_000_000  # 2e6 cycles in 1 ms: 2 GHz
    grbm = cycles_per_xcd * counters.XCDS
    simd_cycles = cycles_per_xcd * counters.SIMDS
    _write_pass(tmp_path / "sq", [
        (1, GEMM, "GRBM_GUI_ACTIVE", grbm, duration),
        (1, GEMM, "SQ_VALU_MFMA_BUSY_CYCLES", 0.75 * simd_cycles, duration),
        (1, GEMM, "SQ_INSTS_VALU", 0.05 * simd_cycles / 4, duration),
        (1, GEMM, "SQ_WAVE_CYCLES", 1000, duration), (1, GEMM, "SQ_WAIT_ANY", 250, duration),
        (1, GEMM, "SQ_INSTS_LDS", 10, duration), (1, GEMM, "SQ_LDS_BANK_CONFLICT", 0, duration),
        (1, GEMM, "SQ_BUSY_CYCLES", 1, duration)])
    _write_pass(tmp_path / "l2", [
        (1, GEMM, "GRBM_GUI_ACTIVE", grbm, duration), (1, GEMM, "TCP_TCC_READ_REQ_sum", 100, duration),
        (1, GEMM, "TCC_HIT_sum", 80, duration), (1, GEMM, "TCC_MISS_sum", 20, duration),
        (1, GEMM, "TCC_REQ_sum", 100, duration)])
    # The copy reads 2^30 bytes and FETCH_SIZE reports half of them; WRITE_SIZE reports them all.
    _write_pass(tmp_path / "fetch", [(2, COPY, "FETCH_SIZE", 2**19, 300_000),
                                     (3, GEMM, "FETCH_SIZE", 2**18, duration)])
    _write_pass(tmp_path / "write", [(2, COPY, "WRITE_SIZE", 2**20, 300_000),
                                     (3, GEMM, "WRITE_SIZE", 2**16, duration)])
    summary = counters.summarize(tmp_path)
    assert summary["calibration_kernel"] == "copy_dwordx4_vpt1_stream"
    assert summary["fetch_size_bytes_per_byte"] == pytest.approx(0.5)
    assert summary["write_size_bytes_per_byte"] == pytest.approx(1.0)
    gemm = summary["kernels"]["gemm_bf16_256x256x64"]
    assert gemm["clock_ghz"] == pytest.approx(2.0)
    assert gemm["mfma_busy"] == pytest.approx(0.75)
    assert gemm["valu_issue_util"] == pytest.approx(0.05)
    assert gemm["wave_wait_frac"] == pytest.approx(0.25)
    assert gemm["l2_hit_rate"] == pytest.approx(0.8)
    assert gemm["mfma_busy_times_clock_over_peak_clock"] == pytest.approx(0.75 * 2.0 / 2.4)
    assert gemm["hbm_read_bytes"] == pytest.approx(2**18 * 1024 / 0.5)
    assert gemm["hbm_write_bytes"] == pytest.approx(2**16 * 1024)
    copy = summary["kernels"]["copy_dwordx4_vpt1_stream"]
    assert copy["hbm_read_bytes"] == pytest.approx(2**30) and copy["hbm_write_bytes"] == pytest.approx(2**30)
    assert "| `gemm_bf16_256x256x64` |" in counters.markdown(summary)

    report = {"results": [{"metric": "tensor_bf16", "kernel": "gemm_bf16_256x256x64"},
                          {"metric": "memory_bandwidth", "kernel": "copy_x",
                           "patterns": {"copy": {"kernel": "copy_dwordx4_vpt1_stream"}}},
                          {"metric": "tensor_tf32", "kernel": None}]}
    assert counters.attach(report, json.loads(json.dumps(summary))) == 1
    assert report["results"][0]["counters"]["mfma_busy"] == pytest.approx(0.75)
    assert report["results"][1]["patterns"]["copy"]["counters"]["hbm_read_bytes"] == pytest.approx(2**30)
    assert "counters" not in report["results"][2]


def test_every_pass_fits_one_rocprofv3_run():
    limits = {"SQ_": 8, "GRBM_": 2, "TCP_": 4}
    for name, group in counters.PASSES.items():
        for prefix, limit in limits.items():
            assert sum(c.startswith(prefix) for c in group) <= limit, name
        tcc = sum(c.startswith("TCC_") for c in group) + 3 * group.count("FETCH_SIZE") + 2 * group.count(
            "WRITE_SIZE")
        assert tcc <= 4, name
    command = counters.rocprof_command(["SQ_WAVE_CYCLES"], "/tmp/x", ["python3", "prog.py"])
    assert command[command.index("--") + 1:] == ["python3", "prog.py"]
    assert not {"--sys-trace", "-s", "--runtime-trace", "-r"} & set(command)


def test_by_grid_keeps_workgroup_counts_apart(tmp_path):
    """A sweep of workgroups per CU launches one kernel over several grids."""
    peak = ("void mb::(anonymous namespace)::tensor_peak_kernel<mb::MfmaBf16x16, 128, 128, 64, 2, 2, 2, false>"
            "(unsigned char const*)")
    records = []
    for dispatch, (blocks, ghz) in enumerate([(256, 2.0), (256, 2.0), (1024, 2.2)], start=1):
        cycles = ghz * 1e6  # per XCD over a 1 ms launch
        records += [(dispatch, peak, "GRBM_GUI_ACTIVE", cycles * counters.XCDS, 1_000_000, 256 * blocks, 256),
                    (dispatch, peak, "SQ_VALU_MFMA_BUSY_CYCLES", 0.9 * cycles * counters.SIMDS, 1_000_000,
                     256 * blocks, 256)]
    _write_pass(tmp_path / "sq", records)
    merged = counters.summarize(tmp_path)["kernels"]
    assert list(merged) == ["tensor_peak_bf16_128x128x64_c2_mfma16_kn"]
    assert merged["tensor_peak_bf16_128x128x64_c2_mfma16_kn"]["clock_ghz"] == pytest.approx(2.0667, rel=1e-3)
    apart = counters.summarize(tmp_path, by_grid=True)["kernels"]
    assert apart["tensor_peak_bf16_128x128x64_c2_mfma16_kn@256wg"]["clock_ghz"] == pytest.approx(2.0)
    assert apart["tensor_peak_bf16_128x128x64_c2_mfma16_kn@1024wg"]["clock_ghz"] == pytest.approx(2.2)
    assert apart["tensor_peak_bf16_128x128x64_c2_mfma16_kn@1024wg"]["mfma_busy"] == pytest.approx(0.9)


def test_optional_stall_and_path_passes(tmp_path):
    """The issue-wait and memory-path passes add per-wave-cycle and per-CU-cycle fractions."""
    cycles_per_xcd, duration = 1_000_000, 500_000
    grbm = cycles_per_xcd * counters.XCDS
    cu_cycles = cycles_per_xcd * counters.CUS
    _write_pass(tmp_path / "stall", [
        (1, GEMM, "GRBM_GUI_ACTIVE", grbm, duration), (1, GEMM, "SQ_WAVE_CYCLES", 1000, duration),
        (1, GEMM, "SQ_WAIT_INST_ANY", 500, duration), (1, GEMM, "SQ_WAIT_INST_LDS", 70, duration),
        (1, GEMM, "SQ_ACTIVE_INST_LDS", 120, duration), (1, GEMM, "SQ_ACTIVE_INST_VMEM", 50, duration),
        (1, GEMM, "SQ_INSTS_MFMA", 64, duration), (1, GEMM, "SQ_ACTIVE_INST_VALU", 200, duration),
        (1, GEMM, "SQ_INST_CYCLES_VMEM_RD", 40, duration)])
    _write_pass(tmp_path / "path", [
        (1, GEMM, "GRBM_GUI_ACTIVE", grbm, duration),
        (1, GEMM, "TA_ADDR_STALLED_BY_TC_CYCLES_sum", 0.05 * cu_cycles, duration),
        (1, GEMM, "TA_TA_BUSY_sum", 0.4 * cu_cycles, duration),
        (1, GEMM, "TCP_TCC_READ_REQ_LATENCY_sum", 3_700_000, duration),
        (1, GEMM, "TCP_TCC_READ_REQ_sum", 10_000, duration),
        (1, GEMM, "TCP_PENDING_STALL_CYCLES_sum", 0.3 * cu_cycles, duration),
        (1, GEMM, "TCC_TAG_STALL_sum", 1234, duration), (1, GEMM, "TD_TC_STALL_sum", 0.2 * cu_cycles, duration)])
    summary = counters.summarize(tmp_path)
    gemm = summary["kernels"]["gemm_bf16_256x256x64"]
    assert gemm["wait_inst_frac"] == pytest.approx(0.5)
    assert gemm["wait_inst_lds_frac"] == pytest.approx(0.07)
    assert gemm["active_lds_frac"] == pytest.approx(0.12)
    assert gemm["mfma_instructions"] == 64
    assert gemm["l2_read_latency_cycles"] == pytest.approx(370)
    assert gemm["ta_stalled_by_l1_frac"] == pytest.approx(0.05)
    assert gemm["ta_busy_frac"] == pytest.approx(0.4)
    assert gemm["l1_pending_stall_frac"] == pytest.approx(0.3)
    assert gemm["l2_tag_stall_cycles"] == 1234
    assert gemm["td_stalled_by_l1_frac"] == pytest.approx(0.2)
    # Neither pass runs by default.
    assert "stall" not in counters.DEFAULT_PASSES and "path" not in counters.DEFAULT_PASSES


def test_registered_names_of_in_place_tiles_fill_and_untemplated_kernels():
    assert counters.registered_name(
        "void mb::(anonymous namespace)::tensor_peak_tied_kernel<mb::MfmaBf16x16, 256, 256, 64, 2, 2, 1, false>"
        "(unsigned char const*, unsigned char const*, unsigned char const*, unsigned char const*, float*, "
        "unsigned int, unsigned int)") == "tensor_peak_bf16_256x256x64_c1_mfma16_kn"
    assert counters.registered_name(
        "void mb::(anonymous namespace)::fill_kernel<2>(unsigned int __vector(4)*, unsigned long, unsigned int)") \
        == "fill_dwordx4_stream"
    assert counters.registered_name(
        "mb::(anonymous namespace)::clock_witness_kernel(unsigned long*, unsigned long, unsigned long)") \
        == "clock_witness"


def _trace_csv(path, dispatches):
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w") as stream:
        stream.write("Kind,Dispatch_Id,Kernel_Name,Start_Timestamp,End_Timestamp\n")
        for index, (name, start, end) in enumerate(dispatches):
            stream.write(f'KERNEL_DISPATCH,{index},"{name}",{start},{end}\n')


def test_trace_report_finds_each_rows_timed_run(tmp_path):
    """The timed launches of a row are the first run of exactly `steps` dispatches of its kernel after the previous
    row's: longer warmup and load runs are skipped, and two rows sharing a kernel take its runs in order."""
    poison = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float> >(int)"
    dispatches, t = [], 0.0

    def run(name, count, ms):
        nonlocal t
        for _ in range(count):
            dispatches.append((name, t, t + ms * 1e6))
            t += ms * 1e6 + 1000

    run(COPY, 40, 0.3)          # warmup
    run(poison, 1, 0.01)
    run(COPY, 3, 0.32)          # timed (steps = 3)
    run(GEMM, 10, 0.7)          # warmup of row 2
    run(poison, 1, 0.01)
    run(GEMM, 3, 0.72)          # timed
    run(poison, 1, 0.01)
    run(GEMM, 3, 0.74)          # a second row on the same kernel
    _trace_csv(tmp_path / "host" / "1" / "run_kernel_trace.csv", dispatches)
    detail = {"steps": 3, "rows": [{"name": "hbm_copy", "kernel": "copy_dwordx4_vpt1_stream", "ms_per_launch": 0.33},
                                   {"name": "gemm_a", "kernel": "gemm_bf16_256x256x64", "ms_per_launch": 0.72},
                                   {"name": "gemm_b", "kernel": "gemm_bf16_256x256x64", "ms_per_launch": 0.74}]}
    text = counters.trace_report(counters.load_trace(tmp_path), detail)
    assert "| hbm_copy | `copy_dwordx4_vpt1_stream` | 0.3200 | 0.3300 | +3.12% |" in text
    assert "| gemm_a | `gemm_bf16_256x256x64` | 0.7200 | 0.7200 | +0.00% |" in text
    assert "| gemm_b | `gemm_bf16_256x256x64` | 0.7400 | 0.7400 | +0.00% |" in text
    assert "| `copy_dwordx4_vpt1_stream` | 43 |" in text


def test_traffic_table_lists_measured_kernels_in_row_order():
    summary = {"fetch_size_bytes_per_byte": 0.5000154, "write_size_bytes_per_byte": 1.0,
               "kernels": {"copy_dwordx4_vpt1_stream": {"hbm_bytes": 2147483648.4},
                           "gemm_bf16_256x256x64": {"hbm_bytes": 1.88e9}, "unmeasured": {}}}
    text = counters.traffic_table(summary, ["copy_dwordx4_vpt1_stream", "unmeasured", "gemm_bf16_256x256x64"], "cmd")
    body = [line for line in text.splitlines() if not line.startswith("#")]
    assert body == ["copy_dwordx4_vpt1_stream = 2147483648", "gemm_bf16_256x256x64 = 1880000000"]
    assert "FETCH_SIZE / 0.5000154" in text and "# Made by: cmd" in text
