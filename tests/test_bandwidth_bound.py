"""CPU tests of the copy's read/write bound helpers (bench_bandwidth.rw_bound, check_fill, --mode bound)."""

import math
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from triton_chip_benchmarks_amd import bench_bandwidth  # noqa: E402


def test_rw_bound_is_the_time_weighted_mean_of_equal_byte_streams():
    # Equal bytes at rates r and w take B/r + B/w; 2B over that time is the harmonic mean.
    read, write = 7405.3, 7073.7
    nbytes = 2**30
    expected = 2 * nbytes / (nbytes / read + nbytes / write)
    assert math.isclose(bench_bandwidth.rw_bound(read, write), expected, rel_tol=1e-12)
    assert bench_bandwidth.rw_bound(5000.0, 5000.0) == pytest.approx(5000.0)
    assert min(read, write) < bench_bandwidth.rw_bound(read, write) < max(read, write)


def test_check_fill_accepts_the_pattern_and_names_a_wrong_word():
    import torch

    words = torch.full((1024,), 1.0, dtype=torch.float32)
    assert bench_bandwidth.check_fill(words)["correctness"].startswith("passed")
    words[517] = 2.0
    with pytest.raises(AssertionError, match="1 of 1024 words"):
        bench_bandwidth.check_fill(words)
    high = torch.full((8,), -1, dtype=torch.int32)  # 0xFFFFFFFF: a pattern with the sign bit set
    assert bench_bandwidth.check_fill(high, pattern=0xFFFFFFFF)


def test_bound_mode_measures_copy_read_and_write():
    args = bench_bandwidth.parse_args(["--mode", "bound"])
    assert args.mode == "bound"
    args = bench_bandwidth.parse_args([])
    assert args.mode == "all"  # the reference's default: copy and read only
