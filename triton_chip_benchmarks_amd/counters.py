#!/usr/bin/env python3
"""Hardware counters for every report row: the rocprofv3 recipe and its summary.

The reference attaches resource metadata (registers, spills, LDS) to each row
(bench_tensor.py:1134-1136, 1252-1278). This module adds what the hardware
counters say about the same kernels on MI355X: how busy the matrix cores and
the vector ALUs were, the sustained engine clock, and the HBM bytes moved.

  collect    runs one `rocprofv3 --pmc ... --kernel-trace` pass per counter
             group over a program (by default `counters target`), each pass in
             its own child process, raw CSV under --out/<pass>/
  target     the profiled program: every measured row of a suite report,
             relaunched at the configuration the report selected
  summarize  per-kernel means over all dispatches of every pass; derived
             figures (below) as JSON and a markdown table
  attach     copy each kernel's summary into the report rows that ran it

Derived figures, per dispatch, then averaged over a kernel's dispatches
(GRBM_GUI_ACTIVE is summed over the XCDs; SQ counters over all SIMDs):
  clock_ghz        GRBM_GUI_ACTIVE / XCDS / duration
  mfma_busy        SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDS * SIMDS)
  valu_issue_util  4 * SQ_INSTS_VALU / (GRBM_GUI_ACTIVE / XCDS * SIMDS): a wave64
                   VALU instruction occupies its SIMD for 4 cycles
  wave_wait_frac   SQ_WAIT_ANY / SQ_WAVE_CYCLES
  l2_hit_rate      TCC_HIT_sum / (TCC_HIT_sum + TCC_MISS_sum)
  hbm_read_bytes   FETCH_SIZE (KiB) * 1024 / f_read,  hbm_write_bytes likewise
                   with WRITE_SIZE and f_write, where f_read and f_write are what
                   the counters read per byte for the calibration kernel, a
                   plain 1 GiB copy (2^30 bytes read and 2^30 written)
"""

from __future__ import annotations

import argparse
import csv
import json
import os
from pathlib import Path
import re
import subprocess
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

ROOT = Path(__file__).resolve().parent.parent
XCDS = 8
CUS = 256
SIMDS = CUS * 4
CALIBRATION_BYTES = 2**30  # the 1 GiB copy reads and writes this many bytes
CALIBRATION_KERNELS = ("copy_dwordx4_vpt1_stream", "copy_dwordx4_vpt1_nt", "copy_dwordx4_vpt1")

# One rocprofv3 pass per group; each fits the per-block limits of one pass
# (8 SQ, 4 TCC, 4 TCP, 2 GRBM counters; FETCH_SIZE takes 3 TCC, WRITE_SIZE 2).
PASSES = {
    "sq": ["GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY",
           "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_BUSY_CYCLES"],
    "l2": ["GRBM_GUI_ACTIVE", "TCP_TCC_READ_REQ_sum", "TCC_HIT_sum", "TCC_MISS_sum", "TCC_REQ_sum"],
    "fetch": ["FETCH_SIZE"],
    "write": ["WRITE_SIZE"],
    # Optional issue/wait breakdown (not in the default set): where a wave's cycles go besides MFMA issue.
    "stall": ["GRBM_GUI_ACTIVE", "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_LDS",
              "SQ_ACTIVE_INST_VMEM", "SQ_INSTS_MFMA", "SQ_ACTIVE_INST_VALU", "SQ_INST_CYCLES_VMEM_RD"],
    # Optional memory-path pass: vector L1 -> L2 read latency and the stalls along the load path.
    "path": ["GRBM_GUI_ACTIVE", "TA_ADDR_STALLED_BY_TC_CYCLES_sum", "TA_TA_BUSY_sum", "TCP_TCC_READ_REQ_LATENCY_sum",
             "TCP_TCC_READ_REQ_sum", "TCP_PENDING_STALL_CYCLES_sum", "TCC_TAG_STALL_sum", "TD_TC_STALL_sum"],
}
DEFAULT_PASSES = ("sq", "l2", "fetch", "write")

_MFMA_FORMAT = {"MfmaBf16": "bf16", "MfmaF16": "f16", "MfmaI8": "i8", "MfmaFp8": "fp8", "MfmaMxfp4": "mxfp4",
                "MfmaF32": "f32", "MfmaF64": "f64"}
_ELEM_BITS = {"bf16": 16, "f16": 16, "i8": 8, "fp8": 8, "mxfp4": 4, "f32": 32, "f64": 64}


def _template(demangled: str):
    """(family, [template arguments]) of `void ns::family<a, b, ...>(params)`, or None."""
    text = demangled.removeprefix("void ")
    start = text.find("<")
    if start < 0:
        return None
    depth, args, current = 0, [], ""
    for position in range(start, len(text)):
        char = text[position]
        if char in "<(":
            depth += 1
            if depth == 1:
                continue
        elif char in ">)":
            depth -= 1
            if depth == 0:
                args.append(current.strip())
                return text[:start].rsplit("::", 1)[-1], args
        elif char == "," and depth == 1:
            args.append(current.strip())
            current = ""
            continue
        current += char
    return None


def registered_name(demangled: str) -> str:
    """The library's registry name for a demangled kernel name (as rocprofv3 prints it).

    Kernels outside the library keep a shortened form of their own name.
    """
    if demangled.startswith("_Z"):  # left mangled by the profiler (e.g. _Float16 arguments)
        from .audit import registered_name as from_symbol

        name = from_symbol(demangled)
        if name:
            return name
    parsed = _template(demangled) if "mb::" in demangled else None
    if parsed is None:
        if "mb::" in demangled:  # untemplated library kernels: clock_witness_kernel, copy_tail_kernel, ...
            bare = demangled.replace("void ", "").replace("(anonymous namespace)::", "")
            base = re.sub(r"\(.*$", "", bare).rsplit("::", 1)[-1]
            return base.removesuffix("_kernel")
        return re.sub(r"\(.*$", "", demangled.replace("void ", ""))[:120]
    family, args = parsed[0], [part.replace("mb::", "") for part in parsed[1]]
    if family in ("tensor_peak_kernel", "tensor_peak_tied_kernel"):
        fmt, bm, bn, bk, _wm, _wn, chains, nk = args
        shape = "_mfma16" if fmt.endswith("x16") else ""
        return (f"tensor_peak_{_MFMA_FORMAT[fmt.removesuffix('x16')]}_{bm}x{bn}x{bk}_c{chains}{shape}_"
                f"{'nk' if nk in ('true', '1') else 'kn'}")
    if family == "gemm_kernel":
        fmt, bm, bn, bk, _wm, _wn, checked = args
        return f"gemm_{_MFMA_FORMAT[fmt]}_{bm}x{bn}x{bk}{'_checked' if checked in ('true', '1') else ''}"
    if family in ("gemm_staged_kernel", "gemm_dma_kernel"):
        name = _MFMA_FORMAT[args[0].removesuffix("x16")]
        return f"gemm_{name}_256x256x{128 * 8 // _ELEM_BITS[name]}"
    if family == "gemm_dma_f64_kernel":
        return "gemm_f64_256x128x16"
    if family == "copy_kernel":
        unit = "dwordx4" if "__vector(4)" in args[0] else "byte" if "char" in args[0] else "dword"
        policy = {"0": "", "false": "", "1": "_nt", "true": "_nt", "2": "_stream"}[args[2]]
        return f"copy_{unit}_vpt{args[1]}{policy}"
    if family == "read_sum_kernel":
        kind = {"float": "f32", "_Float16": "f16", "__bf16": "bf16"}.get(args[0], args[0])
        return f"read_sum_{kind}{'_vec' if args[1] != '1' else ''}"
    if family == "fill_kernel":
        return "fill_dwordx4" + {"0": "", "1": "_nt", "2": "_stream"}.get(args[0], "")
    if family.startswith("vector_") and family.endswith("_kernel"):
        return f"{family[:-len('_kernel')]}_u{args[0]}"
    return family


# ---- collect -----------------------------------------------------------------

def rocprof_command(counters, out_dir: Path, program) -> list[str]:
    """rocprofv3 argv for one pass; the profiled program itself follows `--`."""
    return ["rocprofv3", "--pmc", *counters, "--kernel-trace", "--output-format", "csv", "-d", str(out_dir),
            "-o", "run", "--", *program]


def collect(out: Path, program, passes=None, timeout_s: float = 300.0) -> None:
    out.mkdir(parents=True, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    for name in passes or DEFAULT_PASSES:
        directory = out / name
        command = rocprof_command(PASSES[name], directory, program)
        print(f"[counters] pass {name}: {' '.join(PASSES[name])}", flush=True)
        with (out / f"{name}.log").open("w") as log:
            completed = subprocess.run(command, cwd=ROOT, env=env, stdout=log, stderr=subprocess.STDOUT,
                                       timeout=timeout_s, check=False)
        if completed.returncode != 0 and not _complete(directory):
            raise SystemExit(f"counter pass {name} failed with exit code {completed.returncode}; "
                             f"see {out / (name + '.log')}")
        if completed.returncode != 0:
            print(f"[counters] pass {name}: profiler exited {completed.returncode} after a complete run",
                  flush=True)


def _counter_csv(directory: Path) -> Path | None:
    found = sorted(directory.rglob("*counter_collection.csv"))
    return found[0] if found else None


def _complete(directory: Path) -> bool:
    path = _counter_csv(directory)
    return path is not None and path.stat().st_size > 0


# ---- summarize ---------------------------------------------------------------

def load_pass(directory: Path, by_grid: bool = False) -> dict[str, dict[int, dict]]:
    """kernel -> dispatch id -> {counter: value, 'duration_ns': ns} for one pass.

    With by_grid, launches of one kernel over different grids are kept apart
    under `kernel@<workgroups>wg` (a sweep of workgroups per CU, for example).
    """
    path = _counter_csv(directory)
    if path is None:
        return {}
    kernels: dict[str, dict[int, dict]] = {}
    with path.open() as stream:
        for record in csv.DictReader(stream):
            name = registered_name(record["Kernel_Name"])
            if by_grid:
                name += f"@{int(record['Grid_Size']) // max(1, int(record['Workgroup_Size']))}wg"
            dispatch = kernels.setdefault(name, {}).setdefault(int(record["Dispatch_Id"]), {})
            dispatch[record["Counter_Name"]] = dispatch.get(record["Counter_Name"], 0.0) + float(
                record["Counter_Value"])
            dispatch["duration_ns"] = float(record["End_Timestamp"]) - float(record["Start_Timestamp"])
    return kernels


def _mean(values):
    values = [v for v in values if v is not None]
    return sum(values) / len(values) if values else None


def _per_dispatch(dispatches, formula):
    out = []
    for values in dispatches.values():
        try:
            out.append(formula(values))
        except (KeyError, ZeroDivisionError):
            continue
    return _mean(out)


def summarize(out: Path, by_grid: bool = False) -> dict:
    passes = {name: load_pass(out / name, by_grid) for name in PASSES if (out / name).exists()}
    kernels = sorted({kernel for data in passes.values() for kernel in data})
    fetch, write = passes.get("fetch", {}), passes.get("write", {})
    calibration = next((k for base in CALIBRATION_KERNELS for k in fetch
                        if k.split("@")[0] == base and k in write), None)
    f_read = f_write = None
    if calibration:
        f_read = _per_dispatch(fetch[calibration], lambda v: v["FETCH_SIZE"] * 1024) / CALIBRATION_BYTES
        f_write = _per_dispatch(write[calibration], lambda v: v["WRITE_SIZE"] * 1024) / CALIBRATION_BYTES

    def cycles(v):
        return v["GRBM_GUI_ACTIVE"] / XCDS

    summary = {}
    for kernel in kernels:
        sq, l2 = passes.get("sq", {}).get(kernel, {}), passes.get("l2", {}).get(kernel, {})
        stall = passes.get("stall", {}).get(kernel, {})
        path = passes.get("path", {}).get(kernel, {})
        row = {
            "dispatches": {name: len(data.get(kernel, {})) for name, data in passes.items()},
            "duration_ms": _mean([_per_dispatch(data.get(kernel, {}), lambda v: v["duration_ns"] / 1e6)
                                  for data in passes.values()]),
            "clock_ghz": _per_dispatch(sq, lambda v: cycles(v) / v["duration_ns"]),
            "mfma_busy": _per_dispatch(sq, lambda v: v["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles(v) * SIMDS)),
            "valu_issue_util": _per_dispatch(sq, lambda v: 4 * v["SQ_INSTS_VALU"] / (cycles(v) * SIMDS)),
            "wave_wait_frac": _per_dispatch(sq, lambda v: v["SQ_WAIT_ANY"] / v["SQ_WAVE_CYCLES"]),
            "lds_instructions": _per_dispatch(sq, lambda v: v["SQ_INSTS_LDS"]),
            "lds_bank_conflict_cycles": _per_dispatch(sq, lambda v: v["SQ_LDS_BANK_CONFLICT"]),
            "l2_read_requests": _per_dispatch(l2, lambda v: v["TCP_TCC_READ_REQ_sum"]),
            "l2_requests": _per_dispatch(l2, lambda v: v["TCC_REQ_sum"]),
            "l2_hit_rate": _per_dispatch(l2, lambda v: v["TCC_HIT_sum"] / (v["TCC_HIT_sum"] + v["TCC_MISS_sum"])),
            "fetch_size_kib": _per_dispatch(fetch.get(kernel, {}), lambda v: v["FETCH_SIZE"]),
            "write_size_kib": _per_dispatch(write.get(kernel, {}), lambda v: v["WRITE_SIZE"]),
        }
        if stall:
            row.update({
                "mfma_instructions": _per_dispatch(stall, lambda v: v["SQ_INSTS_MFMA"]),
                "wait_inst_frac": _per_dispatch(stall, lambda v: v["SQ_WAIT_INST_ANY"] / v["SQ_WAVE_CYCLES"]),
                "wait_inst_lds_frac": _per_dispatch(stall, lambda v: v["SQ_WAIT_INST_LDS"] / v["SQ_WAVE_CYCLES"]),
                "active_lds_frac": _per_dispatch(stall, lambda v: v["SQ_ACTIVE_INST_LDS"] / v["SQ_WAVE_CYCLES"]),
                "active_vmem_frac": _per_dispatch(stall, lambda v: v["SQ_ACTIVE_INST_VMEM"] / v["SQ_WAVE_CYCLES"]),
                "active_valu_frac": _per_dispatch(stall, lambda v: v["SQ_ACTIVE_INST_VALU"] / v["SQ_WAVE_CYCLES"]),
                "vmem_read_cycles_frac": _per_dispatch(
                    stall, lambda v: v["SQ_INST_CYCLES_VMEM_RD"] / v["SQ_WAVE_CYCLES"]),
            })
        if path:
            row.update({
                "l2_read_latency_cycles": _per_dispatch(
                    path, lambda v: v["TCP_TCC_READ_REQ_LATENCY_sum"] / v["TCP_TCC_READ_REQ_sum"]),
                "ta_stalled_by_l1_frac": _per_dispatch(
                    path, lambda v: v["TA_ADDR_STALLED_BY_TC_CYCLES_sum"] / (cycles(v) * CUS)),
                "ta_busy_frac": _per_dispatch(path, lambda v: v["TA_TA_BUSY_sum"] / (cycles(v) * CUS)),
                "l1_pending_stall_frac": _per_dispatch(
                    path, lambda v: v["TCP_PENDING_STALL_CYCLES_sum"] / (cycles(v) * CUS)),
                "l2_tag_stall_cycles": _per_dispatch(path, lambda v: v["TCC_TAG_STALL_sum"]),
                "td_stalled_by_l1_frac": _per_dispatch(path, lambda v: v["TD_TC_STALL_sum"] / (cycles(v) * CUS)),
            })
        if f_read and row["fetch_size_kib"] is not None:
            row["hbm_read_bytes"] = row["fetch_size_kib"] * 1024 / f_read
        if f_write and row["write_size_kib"] is not None:
            row["hbm_write_bytes"] = row["write_size_kib"] * 1024 / f_write
        if "hbm_read_bytes" in row and "hbm_write_bytes" in row:
            row["hbm_bytes"] = row["hbm_read_bytes"] + row["hbm_write_bytes"]
            if row["duration_ms"]:
                row["hbm_gbps"] = row["hbm_bytes"] / (row["duration_ms"] * 1e6)
        if row["clock_ghz"] and row["mfma_busy"] is not None:
            row["mfma_busy_times_clock_over_peak_clock"] = row["mfma_busy"] * row["clock_ghz"] / 2.4
        summary[kernel] = row
    return {"calibration_kernel": calibration, "fetch_size_bytes_per_byte": f_read,
            "write_size_bytes_per_byte": f_write, "xcds": XCDS, "simds": SIMDS, "kernels": summary}


def markdown(summary: dict, only=None) -> str:
    lines = ["| kernel | ms | clock GHz | MFMA busy | VALU issue | busy×clock/2.4 | wave wait | L2 hit | "
             "HBM read MB | HBM write MB |", "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]

    def fmt(value, scale=1.0, digits=3, percent=False):
        if value is None:
            return "—"
        return f"{100 * value:.1f}%" if percent else f"{value * scale:.{digits}f}"

    for kernel, row in summary["kernels"].items():
        if only is not None and kernel not in only:
            continue
        lines.append(f"| `{kernel}` | {fmt(row['duration_ms'])} | {fmt(row['clock_ghz'], digits=2)} | "
                     f"{fmt(row['mfma_busy'], percent=True)} | {fmt(row['valu_issue_util'], percent=True)} | "
                     f"{fmt(row.get('mfma_busy_times_clock_over_peak_clock'), percent=True)} | "
                     f"{fmt(row['wave_wait_frac'], percent=True)} | {fmt(row['l2_hit_rate'], percent=True)} | "
                     f"{fmt(row.get('hbm_read_bytes'), 1e-6, 1)} | {fmt(row.get('hbm_write_bytes'), 1e-6, 1)} |")
    return "\n".join(lines) + "\n"


# ---- attach ------------------------------------------------------------------

def attach(report: dict, summary: dict) -> int:
    """Put each row's kernel summary under row['counters'] (and patterns[*]['counters']); returns rows touched."""
    touched = 0
    kernels = summary["kernels"]
    for row in report.get("results", []):
        if row.get("kernel") in kernels:
            row["counters"] = kernels[row["kernel"]]
            touched += 1
        for pattern in (row.get("patterns") or {}).values():
            if isinstance(pattern, dict) and pattern.get("kernel") in kernels:
                pattern["counters"] = kernels[pattern["kernel"]]
    return touched


# ---- target ------------------------------------------------------------------

def _target_rows(report: dict, selected):
    for row in report.get("results", []):
        if row.get("status") not in ("ok", "unverified") or not row.get("kernel"):
            continue
        if selected and row["metric"] not in selected:
            continue
        yield row


def target(report_path: Path, launches: int, selected=None) -> None:
    """Relaunch every measured row's kernel at its reported configuration (the program rocprofv3 profiles)."""
    import torch

    from . import _native, bench_bandwidth, bench_tensor, bench_vector
    from .common import require_gpu

    require_gpu(0)
    report = json.loads(Path(report_path).read_text())
    rows = list(_target_rows(report, selected))
    if not any(row["metric"] == "memory_bandwidth" for row in rows):
        rows.insert(0, {"metric": "memory_bandwidth", "kernel": "copy_dwordx4_vpt1_stream",
                        "configuration": {"block_threads": 64, "vectors_per_thread": 1, "grid_blocks": 0,
                                          "buffer_mib": 1024}})
    for row in rows:
        metric, config, kernel = row["metric"], row.get("configuration") or {}, row["kernel"]
        print(f"[target] {metric}: {kernel} x{launches}", flush=True)
        if metric == "memory_bandwidth":
            elements = int(config.get("buffer_mib", 1024)) * 2**20 // 4
            src = torch.empty(elements, device="cuda").uniform_(-1, 1)
            dst = torch.empty_like(src)
            policy = "stream" if kernel.endswith("_stream") else "on" if kernel.endswith("_nt") else "off"
            for _ in range(launches):
                bench_bandwidth.launch_copy(src, dst, config["block_threads"], config["vectors_per_thread"],
                                            config.get("grid_blocks", 0), policy)
            read = (row.get("patterns") or {}).get("read")
            if read:
                rc = read["configuration"]
                sink = torch.empty(-(-src.numel() // rc["block_size"]), device="cuda")
                for _ in range(launches):
                    bench_bandwidth.launch_read(src, sink, rc["block_size"], rc["block_threads"])
            del src, dst
        elif row.get("group") == "Tensor":
            dtype = row["precision"]
            tile = config["config"]
            peak = next(c for c in _native.peak_configs(dtype)
                        if (c["tile_m"], c["tile_n"], c["tile_k"], c["chains"]) ==
                        (tile["block_m"], tile["block_n"], tile["block_k"], tile["chains"])
                        and bool(c["b_nk"]) == (tile.get("b_layout") == "nk")
                        and c["mfma_m"] == tile.get("mfma_m", 32))
            if dtype == "fp4":
                a, b, c, scales, _values = bench_tensor.fp4_peak_inputs(config["blocks"], peak, "cuda")
            else:
                a, b, c, _logical = bench_tensor.peak_inputs(config["blocks"], peak, dtype, "cuda")
                scales = None
            for _ in range(launches):
                bench_tensor.launch_peak(dtype, peak, a, b, c, config["iterations"], scales)
        elif row.get("group") == "Vector":
            dtype = row["precision"]
            kind = next(k for k, _op, suffix in bench_vector.VARIANTS[dtype] if suffix == config["variant"])
            elements = config["blocks"] * config["block_size"]
            inputs, coefficients = bench_vector.make_inputs(dtype, elements, "cuda", "reference")
            output = torch.empty_like(inputs)
            for _ in range(launches):
                bench_vector.launch_vector(kind, inputs, output, coefficients, config["iterations"],
                                           config["unroll"], config["block_size"])
        torch.cuda.synchronize()


# ---- HBM traffic table read by bench.py -------------------------------------------

def traffic_table(summary: dict, kernels, command: str) -> str:
    """`kernel = bytes` lines (HBM read + write per launch) for the given kernels, with the derivation."""
    lines = ["# HBM-side bytes per launch (read + write) of the bench.py kernels at bench.py's",
             "# launch shapes, from rocprofv3 FETCH_SIZE and WRITE_SIZE counter runs (KiB per",
             "# dispatch), each scaled by what the same counter reads for the 1 GiB plain copy",
             f"# in the same run (FETCH_SIZE / {summary['fetch_size_bytes_per_byte']:.7f}, "
             f"WRITE_SIZE / {summary['write_size_bytes_per_byte']:.7f}).",
             f"# Made by: {command}"]
    for kernel in kernels:
        row = summary["kernels"].get(kernel) or {}
        if row.get("hbm_bytes") is not None:
            lines.append(f"{kernel} = {round(row['hbm_bytes'])}")
    return "\n".join(lines) + "\n"


# ---- kernel trace of a bench.py run ---------------------------------------------

def load_trace(directory: Path) -> list[tuple[float, float, str]]:
    """(start ns, end ns, registry name) of every dispatch in a rocprofv3 --kernel-trace run, by start time."""
    found = sorted(directory.rglob("*kernel_trace.csv"))
    if not found:
        raise SystemExit(f"no *kernel_trace.csv under {directory}")
    dispatches = []
    for path in found:
        with path.open() as stream:
            for record in csv.DictReader(stream):
                dispatches.append((float(record["Start_Timestamp"]), float(record["End_Timestamp"]),
                                   registered_name(record["Kernel_Name"])))
    return sorted(dispatches)


def trace_report(dispatches, detail: dict) -> str:
    """Per-kernel statistics of the trace, then each bench.py row's timed launches against its own figure.

    A row's timed launches are the first run, after the previous row's, of exactly `steps` consecutive
    dispatches of the row's kernel: its warmup, clock-witness load and power load are longer runs, and the
    witness kernel or the output poisoning separates them.
    """
    steps = int(detail["steps"])
    total = sum(end - start for start, end, _ in dispatches)
    per_kernel: dict[str, list[float]] = {}
    for start, end, name in dispatches:
        per_kernel.setdefault(name, []).append((end - start) / 1e6)
    rows = detail["rows"]
    ours = {row["kernel"] for row in rows}
    lines = ["| kernel (registry name) | calls | average ms | min ms | max ms | share of GPU time |",
             "|---|---:|---:|---:|---:|---:|"]
    other = 0.0
    for name, times in sorted(per_kernel.items(), key=lambda item: -sum(item[1])):
        if name not in ours:
            other += sum(times)
            continue
        lines.append(f"| `{name}` | {len(times)} | {sum(times) / len(times):.4f} | {min(times):.4f} | "
                     f"{max(times):.4f} | {100 * sum(times) * 1e6 / total:.2f}% |")
    lines += ["", f"All other kernels (input generation, reference products, validation, the copy's read and "
                  f"write legs, outside the timed regions): {100 * other * 1e6 / total:.2f}% of GPU time.", ""]
    runs, current = [], None
    for start, end, name in dispatches:
        if current and current[0] == name:
            current[1].append((end - start) / 1e6)
        else:
            current = (name, [(end - start) / 1e6])
            runs.append(current)
    lines += [f"| row | kernel | rocprofv3 mean ms ({steps} timed) | bench.py ms_per_launch | difference |",
              "|---|---|---:|---:|---:|"]
    position = 0
    for row in rows:
        match = next((i for i in range(position, len(runs))
                      if runs[i][0] == row["kernel"] and len(runs[i][1]) == steps), None)
        if match is None:
            lines.append(f"| {row['name']} | `{row['kernel']}` | not found | {row['ms_per_launch']:.4f} | — |")
            continue
        position = match + 1
        traced = sum(runs[match][1]) / steps
        difference = round(100 * (row["ms_per_launch"] / traced - 1), 2) + 0.0  # + 0.0: no "-0.00"
        lines.append(f"| {row['name']} | `{row['kernel']}` | {traced:.4f} | {row['ms_per_launch']:.4f} | "
                     f"{difference:+.2f}% |")
    return "\n".join(lines) + "\n"


# ---- CLI ---------------------------------------------------------------------

def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = parser.add_subparsers(dest="command", required=True)
    p = sub.add_parser("collect", help="run the rocprofv3 passes over a program")
    p.add_argument("--out", type=Path, required=True)
    p.add_argument("--passes", nargs="+", choices=list(PASSES))
    p.add_argument("--timeout", type=float, default=300.0, help="seconds per pass")
    p.add_argument("program", nargs=argparse.REMAINDER,
                   help="-- program argv (default: this module's `target` over the committed report)")
    p = sub.add_parser("target", help="relaunch every measured row of a report")
    p.add_argument("--report", type=Path, default=ROOT / "results" / "mi355x_chip_metrics.json")
    p.add_argument("--launches", type=int, default=5)
    p.add_argument("--rows", nargs="+")
    p = sub.add_parser("summarize", help="per-kernel summary of collected passes")
    p.add_argument("--out", type=Path, required=True)
    p.add_argument("--json", type=Path)
    p.add_argument("--markdown", type=Path)
    p.add_argument("--by-grid", action="store_true",
                   help="keep launches of one kernel over different grids apart (kernel@<workgroups>wg)")
    p = sub.add_parser("trace", help="kernel-trace statistics of a bench.py run and its timed launches")
    p.add_argument("--trace-dir", type=Path, required=True, help="rocprofv3 -d directory of the run")
    p.add_argument("--detail", type=Path, required=True, help="bench.py --detail file of the same run")
    p.add_argument("--markdown", type=Path)
    p = sub.add_parser("traffic", help="bench.py's HBM traffic table from a counter summary")
    p.add_argument("--summary", type=Path, required=True, help="counters summarize --json output")
    p.add_argument("--detail", type=Path, required=True, help="a bench.py --detail file naming the row kernels")
    p.add_argument("--write", type=Path, required=True)
    p = sub.add_parser("attach", help="copy kernel summaries into a report's rows")
    p.add_argument("--summary", type=Path, required=True)
    p.add_argument("--report", type=Path, required=True)
    p.add_argument("--write", type=Path)
    args = parser.parse_args(argv)
    if args.command == "collect":
        program = [part for part in args.program if part != "--"] or [
            sys.executable, "-u", "-m", "triton_chip_benchmarks_amd.counters", "target"]
        collect(args.out, program, args.passes, args.timeout)
    elif args.command == "target":
        target(args.report, args.launches, args.rows)
    elif args.command == "summarize":
        summary = summarize(args.out, args.by_grid)
        if args.json:
            args.json.write_text(json.dumps(summary, indent=2) + "\n")
        text = markdown(summary)
        if args.markdown:
            args.markdown.write_text(text)
        print(text)
    elif args.command == "traffic":
        detail = json.loads(args.detail.read_text())
        kernels = list(dict.fromkeys(row["kernel"] for row in detail["rows"]))
        command = " ".join(["python -m triton_chip_benchmarks_amd.counters", *(argv or sys.argv[1:])])
        text = traffic_table(json.loads(args.summary.read_text()), kernels, command)
        args.write.write_text(text)
        print(text)
    elif args.command == "trace":
        text = trace_report(load_trace(args.trace_dir), json.loads(args.detail.read_text()))
        if args.markdown:
            args.markdown.write_text(text)
        print(text)
    else:
        summary = json.loads(args.summary.read_text())
        report = json.loads(args.report.read_text())
        touched = attach(report, summary)
        (args.write or args.report).write_text(json.dumps(report, indent=2) + "\n")
        print(f"attached counters to {touched} rows")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
