#!/usr/bin/env python3
"""Command-line entry point kept at the reference's path: `python bench_vector.py ...`.

The implementation is triton_chip_benchmarks_amd/bench_vector.py.
"""

import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

from triton_chip_benchmarks_amd.bench_vector import main  # noqa: E402

if __name__ == "__main__":
    raise SystemExit(main())
