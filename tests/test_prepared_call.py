"""``prepared_call`` with the reference's signature
(``_compiler/mlir/driver.py:748-788``) and the native-call switch
(``native/__init__.py:84-95``), on the host: the binding logic is exercised
with a CPU stand-in for a ``GpuLaunch`` (the gpu target's launch objects), so
no kernel runs. The cases follow the reference's own prepared-call tests
(``tests/test_native_call.py:700-910``): views of the argument and the
result, the bound tensors' current storage, metadata changes that send a
call to the fallback, sizes that views may not change, and the switch."""

from __future__ import annotations

import pytest
import torch

import helion_mlir_backend as B
from helion_mlir_backend._compiler import native


class AddRows(B.GpuLaunch):
    """CPU stand-in for a bound launch: ``x + y`` into a fresh tensor."""

    __slots__ = ("launches",)

    def __init__(self) -> None:
        self.launches = 0

    def __call__(self, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        self.launches += 1
        return (x + y).contiguous()


@pytest.fixture
def native_switch():
    before = native.enabled()
    yield B.set_native_call
    B.set_native_call(before)


def test_positional_signature_and_native_calls() -> None:
    x, y = torch.randn(16, 8), torch.randn(16, 8)
    kernel = AddRows()
    used: list[int] = []

    def fallback(a: torch.Tensor) -> str:
        used.append(1)
        return "fallback"

    prepared = B.prepared_call(kernel, (x, y), [0], fallback)
    assert isinstance(prepared, B.PreparedCall)
    x2 = torch.randn(16, 8)
    assert torch.equal(prepared(x2), x2 + y)
    assert prepared.native_calls == 1 and kernel.launches == 1 and not used
    # Another shape, dtype or strided layout: the fallback.
    for other in (torch.randn(8, 8), x2.double(), torch.randn(8, 16).t()):
        assert prepared(other) == "fallback"
    assert len(used) == 3 and prepared.native_calls == 1


def test_objects_without_a_native_run_return_none() -> None:
    x = torch.randn(4, 4)
    assert B.prepared_call(lambda a, b: a + b, (x, x), [0], lambda a: a) is None
    assert B.prepared_call(object(), (x, x), [0], lambda a: a) is None


def test_views_of_the_argument_and_the_result() -> None:
    x3, y3 = torch.randn(16, 4, 2), torch.randn(16, 4, 2)
    kernel = AddRows()
    calls: list[torch.Tensor] = []

    def fallback(x: torch.Tensor) -> torch.Tensor:
        calls.append(x)
        return (x.reshape(16, 8) + y3.view(16, 8)).view(128)

    prepared = B.prepared_call(kernel, (x3.view(16, 8), y3.view(16, 8)), [0], fallback,
                               views=[(16, 4, 2)], result_shape=(128,))
    assert prepared is not None
    x3 = torch.randn(16, 4, 2)
    out = prepared(x3)
    assert prepared.native_calls == 1 and not calls
    assert out.shape == (128,) and out.is_contiguous()
    assert torch.equal(out, (x3 + y3).view(128))
    for other in (x3.view(16, 8), x3.transpose(0, 1).contiguous().transpose(0, 1)):
        assert torch.equal(prepared(other), (other.reshape(16, 8) + y3.view(16, 8)).view(128))
    assert len(calls) == 2 and prepared.native_calls == 1


def test_bound_tensors_current_storage_is_read() -> None:
    x, y = torch.randn(24, 8), torch.randn(24, 8)
    prepared = B.prepared_call(AddRows(), (x, y), [0], lambda a: a + y)
    assert torch.equal(prepared(x), x + y)
    y.set_(torch.randn(24, 8))  # the bound tensor's storage changes
    assert torch.equal(prepared(x), x + y)
    assert prepared.native_calls == 2
    y.set_(torch.randn(8, 24).t())  # its metadata changes: the fallback
    assert torch.equal(prepared(x), x + y)
    assert prepared.native_calls == 2


def test_views_that_change_the_size_take_the_fallback() -> None:
    x, y = torch.randn(40, 8), torch.randn(40, 8)
    calls: list[int] = []

    def fallback(a: torch.Tensor) -> torch.Tensor:
        calls.append(1)
        return a[:40] + y

    prepared = B.prepared_call(AddRows(), (x, y), [0], fallback, views=[(80, 8)])
    big = torch.randn(80, 8)
    prepared(big)
    assert torch.equal(prepared(big), big[:40] + y)
    assert len(calls) == 2 and prepared.native_calls == 0


def test_bad_positions_are_refused() -> None:
    x = torch.randn(4, 4)
    with pytest.raises(ValueError, match="varying positions"):
        B.prepared_call(AddRows(), (x, x), [2], lambda a: a)
    with pytest.raises(ValueError, match="not a tensor"):
        B.prepared_call(AddRows(), (x, 3), [1], lambda a: a)
    with pytest.raises(ValueError, match="one view"):
        B.prepared_call(AddRows(), (x, x), [0], lambda a: a, views=[(4, 4), (4, 4)])


def test_switch_off_applies_to_prepared_calls(native_switch) -> None:
    # Off takes effect at once for every prepared call (each checks it), and
    # prepared_call made while off has no native run.
    x, y = torch.randn(16, 16), torch.randn(16, 16)
    kernel = AddRows()
    prepared = B.prepared_call(kernel, (x, y), [0], lambda a: a + y)
    expected = x + y
    assert torch.equal(prepared(x), expected) and prepared.native_calls == 1
    native_switch(False)
    for _ in range(2):
        assert torch.equal(prepared(x), expected)
    assert prepared.native_calls == 1 and kernel.launches == 1
    assert B.prepared_call(kernel, (x, y), [0], lambda a: a + y) is None
    native_switch(True)
    assert torch.equal(prepared(x), expected)
    assert prepared.native_calls == 2


def test_switch_environment_is_read_at_import() -> None:
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    code = ("import sys; sys.path[:0] = [%r, %r]; import helion_mlir_backend as B; "
            "from helion_mlir_backend._compiler import native; print(native.enabled())"
            % (str(root), str(root / "helion-mlir-xsmm_amd")))
    env = dict(os.environ, HELION_MLIR_NATIVE_CALL="0")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True)
    assert out.stdout.strip() == "False"


# ---------------------------------------------------------------------------
# explain (the reference's _compiler/call_trace.py:220-270): what a call would
# do, without running it, over this target's kernels.


def test_explain_a_prepared_call_and_its_refusals(native_switch) -> None:
    x, y = torch.randn(16, 8), torch.randn(16, 8)
    kernel = AddRows()
    prepared = B.prepared_call(kernel, (x, y), [0], lambda a: "fallback")
    e = B.explain(prepared, torch.randn(16, 8))
    assert isinstance(e, B.CallExplanation)
    assert (e.dispatch, e.run, e.reason, e.planned, e.native_calls) == ("direct", "native", None, True, 0)
    assert kernel.launches == 0  # explain runs nothing
    e = B.explain(prepared, torch.randn(8, 8))
    assert e.run == "general" and "shape (8, 8)" in e.reason and "(16, 8)" in e.reason
    # Calls that take the fallback are counted by kind, the last in full.
    prepared(torch.randn(8, 8))
    prepared(torch.randn(16, 8).double())
    prepared(torch.randn(16, 8))
    e = B.explain(prepared, torch.randn(16, 8))
    assert e.native_calls == 1 and e.run == "native"
    assert e.refusals == {"a varying argument differs from the prepared one": 2}
    assert "torch.float64" in e.last_refusal
    native_switch(False)
    e = B.explain(prepared, torch.randn(16, 8))
    assert e.run == "general" and "set_native_call(False)" in e.reason
    assert "general run" in str(e) and "took the fallback 2 times" in str(e)


def test_explain_entry_points_and_other_objects() -> None:
    import helion_mlir_utils as U

    a, b = torch.randn(64, 32), torch.randn(32, 16)
    e = B.explain(U.matmul, a, b)
    assert (e.kernel, e.dispatch, e.run) == ("matmul", "bind", "unsupported")
    assert "tensors on cpu" in e.reason
    assert B.explain(U.softmax).reason == "no tensor arguments"
    e = B.explain(AddRows())
    assert (e.dispatch, e.run) == ("direct", "native")
    info = B.explain()  # no kernel: the process report
    assert {"library", "native_calls", "jit", "output_pool"} <= set(info)
    with pytest.raises(TypeError, match="not a kernel of this backend"):
        B.explain(object())


def test_native_module_and_load_error(native_switch) -> None:
    # native.module() / load_error() as the reference's tests use them
    # (``native.module() is None`` to skip): the loaded library, or None
    # while native calls are off.
    if native.available():
        assert native.module() is native.lib() and native.load_error() is None
    native_switch(False)
    assert native.module() is None
