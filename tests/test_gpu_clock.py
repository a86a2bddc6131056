"""GPU tests of the engine-clock witness (mb_clock_witness) that bench.py uses to report each row's clock.

The witness counts shader clock cycles (s_memtime) against the 100 MHz real-time counter over a requested
interval. Checked here: the interval is honoured, the clock it reports lies within the device's range
(the runtime's peak engine clock bounds it from above), two back-to-back measurements of an idle device
agree, and bad arguments are refused before anything is launched.
"""

import ctypes

import pytest

pytestmark = pytest.mark.gpu


def test_witness_measures_a_plausible_clock_over_the_requested_interval(gpu):
    import torch

    from triton_chip_benchmarks_amd import _native

    wall_khz = _native.wall_clock_khz()
    peak_mhz = _native.device_query(0)["clock_khz"] / 1000
    assert wall_khz > 0 and peak_mhz > 0
    out = torch.zeros(4, dtype=torch.int64, device="cuda")
    side = torch.cuda.Stream()
    clocks = []
    for microseconds in (20000, 20000):
        print(f"clock witness {microseconds} us", flush=True)
        out.zero_()
        _native.clock_witness(out, microseconds, side)
        torch.cuda.synchronize()
        cycles, ticks, polls, start = (int(v) for v in out.tolist())
        assert ticks >= microseconds * wall_khz // 1000, (ticks, microseconds)
        assert ticks < 10 * microseconds * wall_khz // 1000  # ended by the interval, not much later
        assert polls > 0 and start > 0
        clocks.append(cycles / ticks * wall_khz / 1000)
    assert all(100 < mhz <= peak_mhz * 1.02 for mhz in clocks), (clocks, peak_mhz)
    assert abs(clocks[0] - clocks[1]) <= 0.1 * max(clocks), clocks


def test_witness_refuses_bad_arguments(gpu):
    import torch

    from triton_chip_benchmarks_amd import _native

    library = _native.load()
    out = torch.zeros(4, dtype=torch.int64, device="cuda")
    assert library.mb_clock_witness(None, 32, 10, None) == _native.MB_ERR_INVALID
    assert library.mb_clock_witness(ctypes.c_void_p(out.data_ptr()), 24, 10, None) == _native.MB_ERR_INVALID
    assert library.mb_clock_witness(ctypes.c_void_p(out.data_ptr()), 32, 0, None) == _native.MB_ERR_INVALID
    assert library.mb_clock_witness(ctypes.c_void_p(out.data_ptr()), 32, 10000001, None) == _native.MB_ERR_INVALID
    assert library.mb_clock_witness(ctypes.c_void_p(out.data_ptr() + 4), 32, 10, None) == _native.MB_ERR_ALIGNMENT
    assert "mb_clock_witness" in _native.last_error()
