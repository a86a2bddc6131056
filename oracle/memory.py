"""Oracle for the memory rows: copy identity, read block sums, accounting.

Follows bench_bandwidth.py (reference): copy_kernel 36-40, read_kernel 50-59,
check_read 81-110, eligibility 181-188, traffic 212-214.
"""

from __future__ import annotations

import math

import numpy as np

FLOAT32_EPS = float(np.finfo(np.float32).eps)


def copy(src: np.ndarray) -> np.ndarray:
    """dst[i] = src[i] for every element (bench_bandwidth.py:36-40)."""
    return np.array(src, copy=True)


def copy_traffic_bytes(buffer_bytes: int) -> int:
    """Copy reads and writes the buffer once each (bench_bandwidth.py:203, 212)."""
    return 2 * buffer_bytes


def read_traffic_bytes(buffer_bytes: int, elements: int, block: int) -> int:
    """Read traffic = buffer + the float32 sink (bench_bandwidth.py:210-212)."""
    return buffer_bytes + 4 * (-(-elements // block))


def gbps(traffic_bytes: int, milliseconds: float) -> float:
    """Decimal GB/s (bench_bandwidth.py:213-214)."""
    return traffic_bytes / (milliseconds * 1e6)


def block_sums(src: np.ndarray, block: int) -> np.ndarray:
    """Exact-as-float64 per-block sums, last block clipped (bench_bandwidth.py:50-59, 92-98)."""
    values = np.asarray(src, dtype=np.float64).reshape(-1)
    rows = -(-values.size // block)
    padded = np.zeros(rows * block, dtype=np.float64)
    padded[:values.size] = values
    return padded.reshape(rows, block).sum(axis=1)


def read_tolerance(src: np.ndarray, block: int) -> np.ndarray:
    """Per-block bound 2*eps32*max(1, log2 B)*sum|x| + 1e-6 (bench_bandwidth.py:87, 99)."""
    rounding = 2 * FLOAT32_EPS * max(1, math.log2(block))
    return block_sums(np.abs(np.asarray(src, dtype=np.float64)), block) * rounding + 1e-6


def check_read(src: np.ndarray, sink: np.ndarray, block: int) -> float:
    """Maximum error of `sink` against the float64 block sums; raises past the bound."""
    reference = block_sums(src, block)
    tolerance = read_tolerance(src, block)
    actual = np.asarray(sink, dtype=np.float64)[:reference.size]
    error = np.abs(actual - reference)
    if not np.all(error <= tolerance):  # also rejects NaN
        raise AssertionError(f"read block sums differ: max_abs_error={np.nanmax(error):.6g}")
    return float(error.max()) if error.size else 0.0


def cache_regime(buffer_bytes: int, cache_bytes: int, quick: bool) -> tuple[str, bool]:
    """(regime, peak_eligible) by the 4x-cache rule (bench_bandwidth.py:181-183)."""
    regime = ("unknown_l2" if not cache_bytes else
              "larger_than_l2" if buffer_bytes >= 4 * cache_bytes else "cache_sensitive")
    return regime, regime == "larger_than_l2" and not quick
