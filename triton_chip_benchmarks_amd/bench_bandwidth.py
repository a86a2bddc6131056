#!/usr/bin/env python3
"""Peak HBM copy and read bandwidth on one MI355X with hand-written gfx950 kernels.

Mirrors the reference's bench_bandwidth.py (bench_bandwidth.py:113-249): the
same CLI, a masked-tail check per configuration, full-output validation of
every measured buffer, the 4x-last-level-cache eligibility rule and the same
row fields. Copy traffic is 2 x buffer bytes; read traffic is buffer bytes plus
the float32 sink. The kernels are mb_copy (16-byte lanes) and mb_read_sum.
"""

from __future__ import annotations

import argparse
import math
from pathlib import Path
import sys

if __package__ in (None, ""):
    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from triton_chip_benchmarks_amd import _native, cpu_baseline, roofline
    from triton_chip_benchmarks_amd.common import (add_common_arguments, available_memory_bytes, emit_results,
                                                   get_device, measure, positive_int, setup_device)
else:
    from . import _native, cpu_baseline, roofline
    from .common import (add_common_arguments, available_memory_bytes, emit_results, get_device, measure,
                         positive_int, setup_device)

DTYPE_CODES = {"fp32": _native.MB_DTYPE_F32, "fp16": _native.MB_DTYPE_F16, "bf16": _native.MB_DTYPE_BF16}
VECTOR_BYTES = 16
WAVE = 64


def torch_dtype(name):
    import torch

    return {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[name]


def copy_geometry(block_size, element_size, num_warps):
    """(threads, vectors per thread) of one workgroup step holding `block_size` elements."""
    threads = WAVE * num_warps
    vectors = block_size * element_size // VECTOR_BYTES
    if vectors % threads:
        return threads, None
    per_thread = vectors // threads
    return threads, per_thread if per_thread in (1, 2, 4, 8, 16) else None


# Copy cache policies: plain, non-temporal loads and stores, or streaming
# (non-temporal loads, device-scope stores written through the XCD's L2).
COPY_POLICIES = {"off": 0, "on": _native.MB_COPY_NONTEMPORAL,
                 "stream": _native.MB_COPY_NONTEMPORAL | _native.MB_COPY_WRITE_THROUGH}
POLICY_SUFFIX = {"off": "", "on": "_nt", "stream": "_stream"}


def copy_policy(nontemporal) -> str:
    """Policy name from a bool (False/True) or a policy name."""
    if isinstance(nontemporal, str):
        if nontemporal not in COPY_POLICIES:
            raise ValueError(f"unknown copy policy {nontemporal!r}")
        return nontemporal
    return "on" if nontemporal else "off"


def launch_copy(src, dst, block_threads, vectors_per_thread, grid_blocks=0, nontemporal=False):
    """dst <- src on the current stream through mb_copy; `nontemporal` is a bool or "off"/"on"/"stream"."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("copy source and destination sizes differ")
    _native.call("mb_copy", src.data_ptr(), dst.data_ptr(), nbytes, block_threads, vectors_per_thread,
                 grid_blocks, COPY_POLICIES[copy_policy(nontemporal)], _native.stream_handle())


FILL_PATTERN = 0x3F800000  # every fp32 word 1.0


def launch_fill(dst, block_threads, grid_blocks=0, policy="stream", pattern=FILL_PATTERN):
    """Every 32-bit word of dst <- pattern through mb_fill (the copy's store stream alone)."""
    _native.call("mb_fill", dst.data_ptr(), dst.numel() * dst.element_size(), pattern, block_threads, grid_blocks,
                 COPY_POLICIES[copy_policy(policy)], _native.stream_handle())


def check_fill(dst, pattern=FILL_PATTERN):
    """Every word of a filled buffer holds the pattern (bit-exact)."""
    import torch

    words = dst.view(torch.int32)
    signed = pattern - (1 << 32) if pattern >= 1 << 31 else pattern
    bad = int((words != signed).sum())
    if bad:
        raise AssertionError(f"Write validation failed: {bad} of {words.numel()} words differ from 0x{pattern:08x}")
    return {"correctness": "passed (every word equals the fill pattern)"}


def rw_bound(read_gbps, write_gbps):
    """Rate of a copy that moves equal read and write bytes, each at its own measured rate, with nothing lost
    to switching between them: the harmonic mean of the two. A copy mixes both streams on the same HBM
    channels, so this bounds it from above."""
    return 2.0 / (1.0 / read_gbps + 1.0 / write_gbps)


def launch_read(src, sink, block_size, block_threads):
    """sink[i] <- sum of src block i, through mb_read_sum."""
    segments = -(-src.numel() // block_size)
    if sink.numel() < segments:
        raise ValueError(f"read sink holds {sink.numel()} sums, {segments} needed")
    dtype = {"torch.float32": "fp32", "torch.float16": "fp16", "torch.bfloat16": "bf16"}[str(src.dtype)]
    _native.call("mb_read_sum", DTYPE_CODES[dtype], src.data_ptr(), sink.data_ptr(), src.numel(), block_size,
                 block_threads, _native.stream_handle())


def check_read(src, sink, block_size):
    """Every block sum of the read kernel against float64 (bench_bandwidth.py:81-110).

    The reference's bound: a float32 reduction of B values over a tree of
    depth log2(B) errs by at most depth * eps * sum|x|; twice that, plus 1e-6
    absolute, is allowed. The float64 sums and absolute sums of all blocks are
    formed first, whole blocks in slabs and the partial last block on its own,
    then compared with the sink in one pass; NaN or infinite sums fail.
    """
    import torch

    count = src.numel()
    blocks, whole = -(-count // block_size), count // block_size
    exact = torch.empty(blocks, dtype=torch.float64, device=src.device)
    magnitude = torch.empty_like(exact)
    per_slab = max(1, (1 << 24) // block_size)  # blocks per float64 slab (<= 128 MiB)
    for first in range(0, whole, per_slab):
        last = min(whole, first + per_slab)
        values = src[first * block_size:last * block_size].view(last - first, block_size).double()
        exact[first:last] = values.sum(dim=1)
        magnitude[first:last] = values.abs().sum(dim=1)
    if whole < blocks:
        tail = src[whole * block_size:].double()
        exact[whole], magnitude[whole] = tail.sum(), tail.abs().sum()
    allowed = magnitude * (2 * torch.finfo(torch.float32).eps * max(1.0, math.log2(block_size))) + 1e-6
    error = (sink[:blocks].double() - exact).abs()
    failed = ~(error <= allowed)
    if bool(failed.any()):
        first_bad = int(torch.nonzero(failed)[0, 0])
        raise AssertionError(f"Read reduction validation failed: {int(failed.sum())} of {blocks} block sums are "
                             f"non-finite or inaccurate (first: block {first_bad}, error "
                             f"{error[first_bad].item():.6g}, allowed {allowed[first_bad].item():.6g})")
    return {"correctness": "passed (all block sums against FP64, plus masked tail)",
            "max_abs_error": error.max().item(), "max_abs_tolerance": allowed.max().item(),
            "reference_device": str(src.device)}


def cache_regime(buffer_bytes, cache_bytes, quick):
    """(regime, peak_eligible): a copy counts as an HBM rate only when each
    buffer is at least 4x the last-level cache (bench_bandwidth.py:181-188)
    and the run is not a smoke run. Unknown cache capacity is never eligible."""
    if not cache_bytes:
        return "unknown_l2", False
    if buffer_bytes >= 4 * cache_bytes:
        return "larger_than_l2", not quick
    return "cache_sensitive", False


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    add_common_arguments(parser)
    parser.add_argument("--mode", choices=["copy", "read", "write", "all", "bound"], default="all",
                        help="Access patterns to measure separately: all = copy and read (default); write = "
                             "the copy's store stream alone (mb_fill); bound = copy, read and write, plus "
                             "the read/write bound of a copy")
    parser.add_argument("--sizes-mib", type=positive_int, nargs="+", default=[256, 512, 1024, 2048],
                        help="Size of EACH source/destination buffer in MiB")
    parser.add_argument("--dtype", choices=["fp16", "bf16", "fp32"], default="fp32")
    parser.add_argument("--block-sizes", type=positive_int, nargs="+", default=[256, 1024, 4096, 16384],
                        help="Elements per workgroup step (copy) or per block sum (read)")
    parser.add_argument("--num-warps", type=positive_int, nargs="+",
                        help="64-lane waves per workgroup (default: 1 4 8)")
    parser.add_argument("--nontemporal", choices=("off", "on", "stream", "both", "all"), default="all",
                        help="Copy cache policy: off (plain), on (nt loads and stores), stream (nt loads, "
                             "write-through device-scope stores), both (off+on) or all (default)")
    parser.add_argument("--grid-blocks", type=int, default=0,
                        help="Copy workgroups striding over the buffer; 0 = one per step (default)")
    parser.add_argument("--seed", type=int, default=0, help="Source RNG seed (uniform [-1, 1))")
    parser.add_argument("--quick", action="store_true",
                        help="Smoke check: 8 MiB, one configuration per mode; not an HBM result")
    args = parser.parse_args(argv)
    if args.quick:
        args.sizes_mib, args.block_sizes, args.num_warps, args.nontemporal = [8], [1024], None, "off"
    if any(block & (block - 1) or block > 65536 for block in args.block_sizes):
        parser.error("--block-sizes must be powers of two no greater than 65536")
    if args.num_warps is not None and any(warps not in (1, 2, 4, 8, 16) for warps in args.num_warps):
        parser.error("--num-warps must be 1, 2, 4, 8 or 16")
    if args.grid_blocks < 0:
        parser.error("--grid-blocks must be non-negative")
    return args


def configurations(args, element_size):
    warps = args.num_warps or ([4] if args.quick else [1, 4, 8])
    nontemporal = {"off": ["off"], "on": ["on"], "stream": ["stream"], "both": ["off", "on"],
                   "all": ["off", "on", "stream"]}[args.nontemporal]
    configs = []
    for block in args.block_sizes:
        for num_warps in warps:
            threads, per_thread = copy_geometry(block, element_size, num_warps)
            configs.append({"block_size": block, "num_warps": num_warps, "block_threads": threads,
                            "vectors_per_thread": per_thread, "nontemporal": nontemporal})
    return configs


def main(argv=None):
    import torch

    args = parse_args(argv)
    metadata = setup_device(args)
    device = get_device(args)
    dtype = torch_dtype(args.dtype)
    element_size = torch.empty((), dtype=dtype).element_size()
    cache_bytes = metadata["l2_cache_bytes"]
    modes = {"all": ["copy", "read"], "bound": ["copy", "read", "write"]}.get(args.mode, [args.mode])
    configs = configurations(args, element_size)
    generator = torch.Generator(device=device)

    for config in configs:
        block, threads = config["block_size"], config["block_threads"]
        generator.manual_seed(args.seed)
        small_src = torch.empty(block + 17, device=device, dtype=dtype).uniform_(-1, 1, generator=generator)
        if "copy" in modes and config["vectors_per_thread"] is not None:
            for nontemporal in config["nontemporal"]:
                small_dst = torch.full_like(small_src, float("nan"))
                launch_copy(small_src, small_dst, threads, config["vectors_per_thread"], args.grid_blocks,
                            nontemporal)
                if not torch.equal(small_src, small_dst):
                    raise AssertionError(f"Copy tail validation failed: block={block}, warps={config['num_warps']}")
        if "write" in modes:
            for policy in config["nontemporal"]:
                small_dst = torch.full_like(small_src, float("nan"))
                launch_fill(small_dst, threads, args.grid_blocks, policy)
                check_fill(small_dst)
        if "read" in modes:
            small_sink = torch.full((-(-small_src.numel() // block),), float("nan"), device=device)
            launch_read(small_src, small_sink, block, threads)
            check_read(small_src, small_sink, block)
    print("Validation: masked tails passed; every measured output is checked in full.")
    print("Copy traffic = 2 * buffer bytes; read traffic = buffer bytes + FP32 reduction sink. "
          "GB/s and TB/s use decimal units; peak uses the shortest timed sample.")
    print("mode   buffer MiB   block  warps  cache      min ms   median ms   peak GB/s  median GB/s  % of 8 TB/s")
    rows = []
    for size_mib in args.sizes_mib:
        buffer_bytes = size_mib * 2**20
        n = buffer_bytes // element_size
        free_bytes = available_memory_bytes()
        max_sink = -(-n // min(args.block_sizes)) * 4 if "read" in modes else 0
        required = (2 if "copy" in modes else 1) * buffer_bytes + max_sink
        if free_bytes is not None and required + 512 * 2**20 > free_bytes:
            raise SystemExit(f"Insufficient free GPU memory for {size_mib} MiB buffers; reduce --sizes-mib.")
        regime, peak_eligible = cache_regime(buffer_bytes, cache_bytes, args.quick)
        if not peak_eligible:
            reason = ("smoke mode" if args.quick else "cache capacity is unavailable" if not cache_bytes
                      else "buffer is smaller than 4x the last-level cache")
            print(f"Note: {size_mib} MiB per buffer excluded from the HBM-sized peak summary: {reason}.")
        generator.manual_seed(args.seed)
        src = torch.empty(n, device=device, dtype=dtype).uniform_(-1, 1, generator=generator)
        dst = torch.empty_like(src) if "copy" in modes or "write" in modes else None
        written = set()  # (threads, policy) of the write rows: the block size does not change a fill
        for config in configs:
            block, warps, threads = config["block_size"], config["num_warps"], config["block_threads"]
            for mode in modes:
                variants = config["nontemporal"] if mode in ("copy", "write") else [None]
                if mode == "copy" and config["vectors_per_thread"] is None:
                    continue  # step size does not split into whole 16-byte lanes
                for nontemporal in variants:
                    sink = None
                    if mode == "write":
                        if (threads, nontemporal) in written:
                            continue
                        written.add((threads, nontemporal))
                        dst.fill_(float("nan"))

                        def run(threads=threads, policy=nontemporal):
                            launch_fill(dst, threads, args.grid_blocks, policy)

                        run()
                        correctness = check_fill(dst)
                        write_bytes = buffer_bytes
                        kernel = f"fill_dwordx4{POLICY_SUFFIX[copy_policy(nontemporal)]}"
                    elif mode == "copy":
                        per_thread = config["vectors_per_thread"]
                        dst.fill_(float("nan"))

                        def run(per_thread=per_thread, nontemporal=nontemporal, threads=threads):
                            launch_copy(src, dst, threads, per_thread, args.grid_blocks, nontemporal)

                        run()
                        if not torch.equal(src, dst):
                            raise AssertionError(f"Copy validation failed: size={size_mib}, block={block}, "
                                                 f"warps={warps}, nt={nontemporal}")
                        correctness = {"correctness": "passed (full output and masked tail)"}
                        write_bytes = buffer_bytes
                        kernel = f"copy_dwordx4_vpt{per_thread}{POLICY_SUFFIX[copy_policy(nontemporal)]}"
                    else:
                        sink = torch.full((-(-n // block),), float("nan"), device=device)

                        def run(block=block, threads=threads, sink=sink):
                            launch_read(src, sink, block, threads)

                        run()
                        correctness = check_read(src, sink, block)
                        write_bytes = sink.numel() * sink.element_size()
                        kernel = f"read_sum_{args.dtype}_vec"
                    timings = measure(run, args)
                    traffic = write_bytes if mode == "write" else buffer_bytes + write_bytes
                    gbps = traffic / (timings["median_ms"] * 1e6)
                    peak_gbps = traffic / (timings["min_ms"] * 1e6)
                    row = {"mode": f"device_global_memory_{mode}", "pattern": mode, "dtype": args.dtype,
                           "buffer_mib": size_mib, "buffer_bytes": buffer_bytes, "elements": n,
                           "read_bytes": 0 if mode == "write" else buffer_bytes, "write_bytes": write_bytes,
                           "traffic_bytes": traffic,
                           "block_size": block, "num_warps": warps, "block_threads": threads,
                           "kernel": kernel, "cache_regime": regime, "peak_eligible": peak_eligible,
                           "smoke_only": args.quick, **timings, "gbps": gbps, "tbps": gbps / 1000,
                           "peak_gbps": peak_gbps, "peak_tbps": peak_gbps / 1000,
                           "fraction_of_hbm_peak": peak_gbps / roofline.HBM_PEAK_GBPS, **correctness}
                    if mode == "write":
                        row.update(cache_policy=copy_policy(nontemporal), grid_blocks=args.grid_blocks,
                                   pattern_word=f"0x{FILL_PATTERN:08x}")
                    if mode == "copy":
                        row.update(vectors_per_thread=config["vectors_per_thread"],
                                   nontemporal=copy_policy(nontemporal) != "off",
                                   cache_policy=copy_policy(nontemporal),
                                   grid_blocks=args.grid_blocks, seed=args.seed,
                                   source_distribution="uniform[-1, 1)")
                    rows.append(row)
                    nt_label = "-" if nontemporal is None else copy_policy(nontemporal)
                    print(f"{mode:4s} {size_mib:11d} {block:7d} {warps:6d} {nt_label:>6} "
                          f"{timings['min_ms']:11.6f} {timings['median_ms']:11.6f} {peak_gbps:11.2f} "
                          f"{gbps:12.2f} {100 * peak_gbps / roofline.HBM_PEAK_GBPS:11.1f}", flush=True)
                    del sink
        del src, dst
    eligible = [row for row in rows if row["peak_eligible"]]
    for mode in modes:
        candidates = [row for row in (eligible or rows) if row["pattern"] == mode]
        if not candidates:
            continue
        best = max(candidates, key=lambda row: row["peak_gbps"])
        label = "Best measured" if eligible else "Best cache-sensitive/smoke"
        print(f"{label} {mode} bandwidth: {best['peak_gbps']:.2f} GB/s ({best['peak_tbps']:.3f} TB/s, "
              f"{100 * best['fraction_of_hbm_peak']:.1f}% of 8 TB/s), {best['buffer_mib']} MiB/buffer, "
              f"block={best['block_size']}, warps={best['num_warps']}.")
    best = {mode: max((row["peak_gbps"] for row in (eligible or rows) if row["pattern"] == mode), default=None)
            for mode in ("copy", "read", "write")}
    if all(best.values()):
        bound = rw_bound(best["read"], best["write"])
        print(f"Read/write bound of a copy (harmonic mean of the best read and write rates): {bound:.2f} GB/s "
              f"({100 * bound / roofline.HBM_PEAK_GBPS:.1f}% of 8 TB/s); the best copy reaches "
              f"{100 * best['copy'] / bound:.1f}% of it.")
    if not eligible:
        print("No HBM-sized peak candidate: eligibility requires buffers >= 4x the last-level cache "
              "and a run without --quick.")
    baseline = None
    if not args.no_cpu_baseline and "copy" in modes:
        # The reference's host path for this row: a tensor copy (1 GiB; 64 MiB in smoke mode).
        baseline = cpu_baseline.copy_baseline((64 if args.quick else 1024) * 2**20)
        print(f"CPU baseline (host, {baseline['cores']} threads): {baseline['value']:.1f} GB/s copy")
    emit_results("bandwidth", metadata, args, rows, cpu_baseline=baseline)


if __name__ == "__main__":
    main()
