"""CPU tests of common.measure against a simulated device clock.

The harness times batches of launches between two device events, optionally
replayed from one captured graph (reference common.py:295-534). A stand-in
for torch.cuda advances a device clock by a fixed kernel time per launch and
quantises event differences to a chosen timer resolution, so each rule can be
checked exactly: per-launch time = batch time / launches, calibration grows
batches until the timer resolves them, a coarse timer sets a floor of 20
ticks per batch, graph failures fall back to event batches only in `auto`,
invalid timestamps are rejected, and the host clock is never read.
"""

from __future__ import annotations

import argparse
import contextlib
import io
import math
import time
import types

import pytest

from triton_chip_benchmarks_amd import common


class FakeDevice:
    def __init__(self, kernel_ms, resolution_ms=0.0, graphs=True, replay_time=True, bad_elapsed=None):
        self.kernel_ms = kernel_ms
        self.resolution_ms = resolution_ms
        self.graphs = graphs
        self.replay_time = replay_time
        self.bad_elapsed = bad_elapsed
        self.now = 0.0
        self.launches = 0
        self.capture = None
        self.synchronizations = 0

    def launch(self):
        if self.capture is not None:
            self.capture.append(self.kernel_ms)
        else:
            self.now += self.kernel_ms
            self.launches += 1

    def module(self):
        device = self

        class Event:
            def __init__(self, enable_timing=False):
                assert enable_timing
                self.time = None

            def record(self):
                self.time = device.now

            def elapsed_time(self, end):
                if device.bad_elapsed is not None:
                    return device.bad_elapsed
                delta = end.time - self.time
                if device.resolution_ms:
                    delta = math.floor(delta / device.resolution_ms + 1e-9) * device.resolution_ms
                return delta

        class Graph:
            def __init__(self):
                if not device.graphs:
                    raise RuntimeError("graph capture is not supported by this stand-in")
                self.recorded = []

            def replay(self):
                if device.replay_time:
                    device.now += sum(self.recorded)
                device.launches += len(self.recorded)

        @contextlib.contextmanager
        def graph(g):
            device.capture = g.recorded
            try:
                yield
            finally:
                device.capture = None

        def synchronize():
            device.synchronizations += 1

        cuda = types.SimpleNamespace(Event=Event, Stream=lambda: object(),
                                     stream=lambda s: contextlib.nullcontext(), synchronize=synchronize,
                                     CUDAGraph=Graph, graph=graph)
        return types.SimpleNamespace(cuda=cuda)


def _args(timing="auto", warmup=5.0, rep=50.0, batch_ms=5.0, rounds=10):
    return argparse.Namespace(timing=timing, warmup=warmup, rep=rep, batch_ms=batch_ms, rounds=rounds)


def _measure(monkeypatch, device, args):
    monkeypatch.setattr(common, "_torch", device.module)
    with contextlib.redirect_stdout(io.StringIO()):
        return common.measure(device.launch, args)


@pytest.mark.parametrize("timing", ["events", "graph", "auto"])
def test_exact_clock_gives_the_kernel_time(monkeypatch, timing):
    device = FakeDevice(kernel_ms=0.25)
    result = _measure(monkeypatch, device, _args(timing))
    assert result["timing_method"] == ("events" if timing == "events" else "graph")
    assert result["median_ms"] == pytest.approx(0.25)
    assert result["min_ms"] == pytest.approx(0.25)
    assert result["sample_count"] >= 10
    assert result["launches_per_batch"] == math.ceil(5.0 / 0.25)
    assert result["measured_total_ms"] >= 50.0 - 1e-9
    assert result["timing_fallback_reason"] is None


def test_resolved_first_estimate_does_not_force_calibration_sized_batches(monkeypatch):
    device = FakeDevice(kernel_ms=2.0)
    result = _measure(monkeypatch, device, _args("events", batch_ms=1.0))
    assert result["calibration_launches"] == common.INITIAL_CALIBRATION_LAUNCHES
    assert result["launches_per_batch"] == 1


def test_coarse_timer_grows_the_calibration_batch_and_sets_a_resolution_floor(monkeypatch):
    device = FakeDevice(kernel_ms=0.01, resolution_ms=1.0)
    result = _measure(monkeypatch, device, _args("events", batch_ms=10.0, rep=200.0))
    # 5 launches read 0 ms; doubling reaches 160 launches = 1.6 ms -> one tick.
    assert result["calibration_launches"] == 160
    assert result["minimum_resolved_batch_ms"] == pytest.approx(20.0)
    assert all(sample >= 20.0 for sample in result["batch_samples_ms"])
    # Quantisation can only shorten a batch, by less than one tick.
    assert result["median_ms"] == pytest.approx(0.01, rel=1.0 / 20)


def test_timer_too_coarse_for_any_batch_is_rejected(monkeypatch):
    device = FakeDevice(kernel_ms=1e-6, resolution_ms=1000.0)
    with pytest.raises(RuntimeError, match="0 ms|too coarse"):
        _measure(monkeypatch, device, _args("events"))


def test_auto_falls_back_to_event_batches_when_capture_fails(monkeypatch):
    device = FakeDevice(kernel_ms=0.5, graphs=False)
    result = _measure(monkeypatch, device, _args("auto"))
    assert result["timing_method"] == "events"
    assert "capture" in result["timing_fallback_reason"]
    assert result["median_ms"] == pytest.approx(0.5)


def test_explicit_graph_request_never_changes_method(monkeypatch):
    device = FakeDevice(kernel_ms=0.5, graphs=False)
    with pytest.raises(common.GraphUnavailable):
        _measure(monkeypatch, device, _args("graph"))


def test_zero_graph_timestamps_fall_back_in_auto(monkeypatch):
    device = FakeDevice(kernel_ms=0.5, replay_time=False)
    result = _measure(monkeypatch, device, _args("auto"))
    assert result["timing_method"] == "events"
    assert result["median_ms"] == pytest.approx(0.5)


@pytest.mark.parametrize("bad", [float("nan"), -1.0, float("inf") * -1])
def test_invalid_device_timestamps_are_rejected(monkeypatch, bad):
    device = FakeDevice(kernel_ms=0.5, bad_elapsed=bad)
    with pytest.raises(RuntimeError, match="Invalid device event time"):
        _measure(monkeypatch, device, _args("events"))


def test_host_clock_is_never_read(monkeypatch):
    def forbidden(*_):
        raise AssertionError("host clock read during device timing")

    for name in ("time", "perf_counter", "perf_counter_ns", "monotonic", "monotonic_ns", "process_time"):
        monkeypatch.setattr(time, name, forbidden)
    device = FakeDevice(kernel_ms=0.3)
    result = _measure(monkeypatch, device, _args("graph"))
    assert result["median_ms"] == pytest.approx(0.3)


def test_every_launch_is_counted_and_warmup_runs(monkeypatch):
    device = FakeDevice(kernel_ms=1.0)
    result = _measure(monkeypatch, device, _args("events", warmup=20.0, rep=40.0, batch_ms=4.0, rounds=5))
    batch = result["launches_per_batch"]
    assert batch == 4
    # first launch + calibration (5) + sizing batch + >= 20 ms of warmup + timed batches
    timed = result["sample_count"] * batch
    assert device.launches >= 1 + 5 + batch + 20 + timed
    assert result["sample_count"] == max(5, math.ceil(40.0 / 4.0))
