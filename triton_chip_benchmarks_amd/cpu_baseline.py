"""CPU baseline beside each row: the reference's own host computations, timed on this machine.

The reference checks its device results against host computations: a float32
torch matmul for the tensor rows (bench_tensor.py:277-286, the low-precision
formats upcast), a vectorised recurrence for the vector rows (bench_vector.py:
322-421) and a tensor copy for bandwidth. Each child times the same kind of
computation on the host cores of the GPU box, on a bounded sample of its work,
and reports it next to the device rate with the host described. This is a
reported baseline, never a fallback: every device value still comes from the
gfx950 kernels, and nothing here feeds a device row. The host clock
(time.perf_counter) is used only here.
"""

from __future__ import annotations

import math
import os
from pathlib import Path
import time

CHAINS = 8


def _torch():
    import torch

    return torch


def host_description() -> dict:
    """Model name, logical and usable CPUs, and the thread counts torch and BLAS use."""
    torch = _torch()
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "usable_cpus": usable,
            "torch_threads": torch.get_num_threads(), "blas_threads": blas_threads()}


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max((pool.get("num_threads", 1) for pool in threadpool_info()), default=1)
    except ImportError:
        return os.cpu_count() or 1


def best_seconds(run, budget_s: float, min_repeats: int = 2, max_repeats: int = 50) -> tuple[float, int]:
    """Shortest of repeated host runs after one untimed run: (seconds, repeats)."""
    run()
    best, repeats, start = math.inf, 0, time.perf_counter()
    while repeats < min_repeats or (time.perf_counter() - start < budget_s and repeats < max_repeats):
        began = time.perf_counter()
        run()
        best = min(best, time.perf_counter() - began)
        repeats += 1
    return best, repeats


def _result(value: float, unit: str, method: str, sample: str, repeats: int) -> dict:
    torch = _torch()
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "method": method,
            "sample": f"{sample}; best of {repeats} host runs", "timer": "time.perf_counter",
            "host": host_description()}


def copy_baseline(buffer_bytes: int, budget_s: float = 2.0) -> dict:
    """torch.Tensor.copy_ of an fp32 host buffer; GB/s counts read + write bytes."""
    torch = _torch()
    elements = buffer_bytes // 4
    source = torch.empty(elements, dtype=torch.float32).uniform_(-1, 1)
    destination = torch.empty_like(source)
    seconds, repeats = best_seconds(lambda: destination.copy_(source), budget_s)
    if not torch.equal(source, destination):
        raise AssertionError("host copy baseline produced a different buffer")
    return _result(2 * elements * 4 / (seconds * 1e9), "GB/s", "torch.Tensor.copy_ on host memory",
                   f"{elements * 4 / 2**20:.0f} MiB fp32", repeats)


def matmul_baseline(dtype: str, size: int, budget_s: float = 2.0) -> dict:
    """torch.matmul on the host in float32 (float64 for fp64), the reference's check arithmetic."""
    torch = _torch()
    compute = torch.float64 if dtype == "fp64" else torch.float32
    a = torch.randn((size, size), dtype=compute)
    b = torch.randn((size, size), dtype=compute)
    seconds, repeats = best_seconds(lambda: torch.matmul(a, b), budget_s)
    unit = "TOPS" if dtype == "int8" else "TFLOP/s"
    upcast = "" if dtype in ("fp32", "fp64") else f", {dtype} operands upcast"
    return _result(2 * size**3 / (seconds * 1e12), unit, f"torch.matmul on the host in {str(compute)[6:]}{upcast}",
                   f"{size}x{size}x{size}", repeats)


def gemm_sample_baseline(dtype: str, rows: int, n: int, k: int, budget_s: float = 2.0) -> dict:
    """torch.matmul on the host of a [rows, K] slice of A against the whole [K, N] B.

    The same K and N as the device GEMM with fewer rows of A: float32
    (float64 for fp64), the reference's check arithmetic with the narrow
    formats upcast (bench_tensor.py:277-286).
    """
    torch = _torch()
    compute = torch.float64 if dtype == "fp64" else torch.float32
    a = torch.randn((rows, k), dtype=compute)
    b = torch.randn((k, n), dtype=compute)
    seconds, repeats = best_seconds(lambda: torch.matmul(a, b), budget_s)
    unit = "TOPS" if dtype == "int8" else "TFLOP/s"
    upcast = "" if dtype in ("fp32", "fp64") else f", {dtype} operands upcast"
    return _result(2 * rows * n * k / (seconds * 1e12), unit,
                   f"torch.matmul on the host in {str(compute)[6:]}{upcast}", f"{rows}x{n}x{k} (rows of A sampled)",
                   repeats)


def tile_batch_baseline(dtype: str, blocks: int, m: int, n: int, k: int, budget_s: float = 2.0) -> dict:
    """Batched torch.matmul on the host of `blocks` resident tiles [M, K] x [K, N] (one iteration, one chain)."""
    torch = _torch()
    compute = torch.float64 if dtype == "fp64" else torch.float32
    a = torch.randn((blocks, m, k), dtype=compute)
    b = torch.randn((blocks, k, n), dtype=compute)
    seconds, repeats = best_seconds(lambda: torch.matmul(a, b), budget_s)
    unit = "TOPS" if dtype == "int8" else "TFLOP/s"
    return _result(2 * blocks * m * n * k / (seconds * 1e12), unit,
                   f"batched torch.matmul on the host in {str(compute)[6:]}", f"{blocks} tiles of {m}x{n}x{k}",
                   repeats)


def _dp4a_step(x, weights, bias):
    """x <- sum_j byte_j(x) * w_j + b on int32 lanes (signed bytes, wrapping int32)."""
    total = bias.clone()
    for j, w in enumerate(weights):
        total += ((x << (24 - 8 * j)) >> 24) * w
    return total


def vector_baseline(dtype: str, lanes: int, iterations: int, budget_s: float = 2.0) -> dict:
    """The chain recurrence over CHAINS x lanes states on the host, vectorised by torch.

    Floating formats update x <- x * a + b in their own storage type; INT8 runs
    the DP4A recurrence on int32 words. Operations are counted as on the device:
    2 per floating update, 8 per DP4A update.
    """
    torch = _torch()
    if dtype == "int8":
        state = torch.randint(-4, 5, (CHAINS, lanes), dtype=torch.int32)
        weights = (3, -2, 1, -1)
        bias = torch.arange(1, CHAINS + 1, dtype=torch.int32)[:, None].expand(CHAINS, lanes)

        def run():
            x = state
            for _ in range(iterations):
                x = _dp4a_step(x, weights, bias)
            return x
        per_update, unit = 8, "TOPS"
    else:
        store = {"fp32": torch.float32, "fp64": torch.float64, "fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
        state = torch.empty((CHAINS, lanes), dtype=torch.float64).uniform_(0.5, 1.0).to(store)
        a = torch.tensor(0.999, dtype=store)
        b = torch.full((CHAINS, 1), 1e-3, dtype=store)
        work = state.clone()  # 0 < a < 1: the states stay near b / (1 - a) however long they run

        def run():
            for _ in range(iterations):
                work.mul_(a).add_(b)
            return work
        per_update, unit = 2, "TFLOP/s"
    seconds, repeats = best_seconds(run, budget_s)
    operations = per_update * CHAINS * lanes * iterations
    return _result(operations / (seconds * 1e12), unit, f"torch vectorised {dtype} recurrence on the host",
                   f"{CHAINS} chains x {lanes} lanes x {iterations} iterations", repeats)
