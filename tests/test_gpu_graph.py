"""Prepared launches under HIP graph capture (the hipGraph option of the
reference's prepared runs, ``native/call.cpp:703-830``): the library's calls
launch on torch's current stream with no host synchronisation or memset, so a
prepared ``linear``, a split-K ``bmm`` and the row kernels record into a
``torch.cuda.CUDAGraph``. Every replay -- with new inputs copied into the
captured buffers and eager work and synchronisations in between -- must equal
the eager result bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import helion_mlir_utils as U
from tests.helpers import tensor

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(11)


def _capture(fn):
    """Warm ``fn`` on a side stream (torch's recipe), then capture it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def _replays_match(graph, out, inputs, eager, replays=4):
    for _ in range(replays):
        for t in inputs:
            t.copy_(torch.from_numpy(RNG.uniform(-1, 1, tuple(t.shape)).astype(np.float32)).to(t.dtype))
        graph.replay()
        torch.cuda.synchronize()
        expect = eager()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, expect)


def test_prepared_linear_replays(gpu_device) -> None:
    layer = torch.nn.Linear(512, 768).to(device=gpu_device, dtype=torch.bfloat16)
    x = tensor(RNG.normal(0, 1, (256, 512)).astype(np.float32), "bf16", gpu_device)
    with torch.no_grad():
        _, cache = U.linear(x, layer, F.silu)
        assert cache.call is not None
        prepared = cache.call[1]
        graph, out = _capture(lambda: U.linear(x, layer, F.silu, cache=cache)[0])
        _replays_match(graph, out, [x], lambda: U.linear(x, layer, F.silu, cache=cache)[0])
    assert prepared.calls >= 6  # warm-up, capture and eager calls all took the prepared launch


def test_split_k_bmm_replays(gpu_device) -> None:
    a = tensor(RNG.uniform(-1, 1, (2, 64, 4096)).astype(np.float32), "f32", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (2, 4096, 96)).astype(np.float32), "f32", gpu_device)
    graph, out = _capture(lambda: U.bmm(a, b, splits=8))
    _replays_match(graph, out, [a, b], lambda: U.bmm(a, b, splits=8))


def test_row_kernels_replay(gpu_device) -> None:
    x = tensor(RNG.normal(0, 2, (1024, 4096)).astype(np.float32), "bf16", gpu_device)
    w = tensor(RNG.uniform(0.5, 1.5, 4096).astype(np.float32), "bf16", gpu_device)
    graph, out = _capture(lambda: U.rms_norm(U.softmax(x), w, 1e-6))
    _replays_match(graph, out, [x], lambda: U.rms_norm(U.softmax(x), w, 1e-6))


def test_native_switch_sends_prepared_calls_to_the_fallback(gpu_device) -> None:
    # set_native_call(False): a prepared linear takes its fallback (the
    # general entry point, same kernel and plan: the same bits) and counts no
    # native call; a linear prepared while off holds no prepared call.
    import helion_mlir_backend as B

    layer = torch.nn.Linear(512, 768).to(device=gpu_device, dtype=torch.bfloat16)
    x = tensor(RNG.normal(0, 1, (256, 512)).astype(np.float32), "bf16", gpu_device)
    with torch.no_grad():
        y, cache = U.linear(x, layer, F.silu)
        prepared = cache.call[1]
        assert isinstance(prepared, B.PreparedCall)
        before = prepared.native_calls
        try:
            B.set_native_call(False)
            y_off, _ = U.linear(x, layer, F.silu, cache=cache)
            assert prepared.native_calls == before
            _, fresh = U.linear(x, layer, F.silu)
            assert not isinstance(fresh.call[1], B.PreparedCall)
        finally:
            B.set_native_call(True)
        y_on, _ = U.linear(x, layer, F.silu, cache=cache)
        assert prepared.native_calls == before + 1
        torch.cuda.synchronize()
    assert torch.equal(y, y_off) and torch.equal(y, y_on)


def test_explain_on_the_gpu(gpu_device) -> None:
    # explain (the reference's call_trace.explain) on ROCm tensors: matmul runs
    # natively with the plan gemm_plan gives; a prepared linear reports its
    # native calls, and a call it would refuse names the argument and why.
    import helion_mlir_backend as B

    a = tensor(RNG.normal(0, 1, (1024, 512)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.normal(0, 1, (512, 768)).astype(np.float32), "bf16", gpu_device)
    e = B.explain(U.matmul, a, b)
    assert (e.run, e.reason) == ("native", None)
    assert e.config == U.gemm_plan(torch.bfloat16, 1024, 768, 512)
    assert B.explain(U.matmul, a, b.float()).run == "unsupported"
    layer = torch.nn.Linear(512, 768).to(device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        _, cache = U.linear(a, layer, F.silu)
        _, cache = U.linear(a, layer, F.silu, cache=cache)
    prepared = cache.call[1]
    e = B.explain(prepared, a)
    assert e.run == "native" and e.native_calls == prepared.native_calls >= 1
    assert e.config["splits"] >= 1 and e.config["tile_m"] in (128, 256)
    e = B.explain(prepared, a[:512])
    assert e.run == "general" and "varying argument 0" in e.reason
