"""CPU oracle for the MI355X peak-throughput suite: TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and a little C, under oracle/c/), the CPU
computations the reference suite uses to validate its kernels: the copy
identity and read block sums (bench_bandwidth.py), the vector recurrences and
their validators (bench_vector.py), the exact-lattice matrix references,
tolerances and the OCP MX FP4 / FP8 formats (bench_tensor.py). Each function
cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
it, and only as the checker or the timed CPU baseline. The product path
(triton_chip_benchmarks_amd/) never imports it and has no CPU fallback.

How each part is pinned (checks that a plausible mistake would fail):
  memory   - identity; block sums against exact integer sums on lattice data;
             traffic formula against the reference's published rows.
  vector   - step-by-step single-rounding emulation (C, exact error-free
             transforms) checked against closed forms, the reference's exact
             involution, its published tolerances (golden fixtures), and a
             brute-force INT8 DP4A recurrence.
  tensor   - float64 matmul on exact lattices (a library routine), the
             reference's tolerance/op-count golden values, the E2M1 table and
             packing known answers, FP8 E4M3FN decoding against torch's
             float8_e4m3fn, E8M0 scale doubling; the elementwise GEMM rule
             against torch.testing.assert_close and known answers a normwise
             rule would get wrong; the FP32/FP64 probe operands against the
             TF32/BF16/FP16/FP32 roundings they must expose.
"""
