"""Shared pytest configuration: the `gpu` marker and repository import paths."""

from pathlib import Path
import sys

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (an MI355X) and the built library")


@pytest.fixture(scope="session")
def gpu():
    """cuda:0 with libmi355x_bench.so loaded; GPU tests fail loudly without them."""
    import torch

    from triton_chip_benchmarks_amd import _native

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    torch.cuda.set_device(0)
    _native.load()
    return torch.device("cuda", 0)
