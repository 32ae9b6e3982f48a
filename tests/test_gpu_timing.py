"""The launch-timing hook (``hmx_time_launches``): events armed before a call
are recorded by that call's own kernels -- the start event as the first kernel
begins, the stop event as the last one ends -- so their elapsed time is the
kernels' GPU time, within the span of plain events recorded around the call.
Disarmed calls leave the events alone, and timed results equal untimed ones."""

from __future__ import annotations

import pytest
import torch

import helion_mlir_utils as U
from helion_mlir_backend._compiler import native

pytestmark = pytest.mark.gpu


def _events(n: int) -> list[torch.cuda.Event]:
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for ev in evs:
        ev.record()  # creates the event
    torch.cuda.synchronize()
    return evs


def _timed(fn):
    """(result, armed ms, bracketing ms) of one call of ``fn``."""
    outer_start, start, stop, outer_stop = _events(4)
    outer_start.record()
    native.time_launches(start, stop)
    try:
        out = fn()
    finally:
        native.time_launches(None, None)
    outer_stop.record()
    torch.cuda.synchronize()
    return out, start.elapsed_time(stop), outer_start.elapsed_time(outer_stop)


def test_armed_events_span_one_kernel(gpu_device) -> None:
    x = torch.randn(32768, 4096, device=gpu_device, dtype=torch.bfloat16)
    U.softmax(x)
    y, armed, outer = _timed(lambda: U.softmax(x))
    # A 512 MB pass takes tens of microseconds; events left as recorded at
    # creation would span almost nothing.
    assert 0.25 * outer < armed <= outer
    assert torch.equal(y, U.softmax(x))


def test_armed_events_span_split_k_kernels(gpu_device) -> None:
    a = torch.rand(4, 256, 16384, device=gpu_device) * 2 - 1
    b = torch.rand(4, 16384, 256, device=gpu_device) * 2 - 1
    U.bmm(a, b, splits=8)
    c, armed, outer = _timed(lambda: U.bmm(a, b, splits=8))
    assert 0.25 * outer < armed <= outer
    assert torch.equal(c, U.bmm(a, b, splits=8))


def test_disarmed_calls_leave_events_alone(gpu_device) -> None:
    x = torch.randn(4096, 4096, device=gpu_device, dtype=torch.bfloat16)
    start, stop = _events(2)
    before = start.elapsed_time(stop)
    native.time_launches(start, stop)
    native.time_launches(None, None)
    U.softmax(x)
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) == before


def test_arming_needs_created_events(gpu_device) -> None:
    with pytest.raises(ValueError):
        native.time_launches(torch.cuda.Event(enable_timing=True), None)
