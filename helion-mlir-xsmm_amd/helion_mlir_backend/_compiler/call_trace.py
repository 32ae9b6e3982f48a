"""What a call on the gpu target would do: :func:`explain` and
:class:`CallExplanation`, the reference's interface for it
(``_compiler/call_trace.py:85-116,220-270``) over this target's kernels.

The reference explains calls of ``@helion.kernel(backend="mlir")`` kernels
and their bound kernels: which dispatch, which run (native, the plan-recording
first call, the general Python path, or a compile), and which check refuses
the native run. This target runs the ``helion_mlir_utils`` entry points, the
prepared calls :func:`~helion_mlir_backend.prepared_call` returns and the
bound launches behind them, so those are what it explains, in the same record.
``explain`` runs, compiles and caches nothing.
"""

from __future__ import annotations

import dataclasses
import inspect

import torch

from . import native
from .prepared import GpuLaunch, PreparedCall

_NO_KERNEL = object()


@dataclasses.dataclass(frozen=True)
class CallExplanation:
    """What a call would do (:func:`explain`); the reference's fields.

    ``dispatch``: ``direct`` (a prepared call or a bound launch was given) or
    ``bind`` (an entry point, which plans and binds its launch on the call).
    ``run``: ``native`` (the library's kernels), ``general`` (a prepared
    call's fallback), ``compile`` (a Helion kernel, which this target does not
    compile) or ``unsupported`` (the entry point refuses these arguments: the
    call raises). ``reason``: why the run is not ``native``. ``config``: the
    launch plan where one is known (splits, tile, workspace). ``refusals`` and
    ``last_refusal``: a prepared call's calls that took its fallback, by kind,
    and the last one's reason in full."""

    kernel: str
    backend: str | None
    dispatch: str
    dispatch_reason: str | None
    run: str
    reason: str | None
    config: object
    planned: bool
    native_calls: int
    refusals: dict[str, int]
    last_refusal: str | None

    def __str__(self) -> str:
        out = [f"{self.kernel}: {self.run} run, {self.dispatch} dispatch"]
        for label, text in (("dispatch", self.dispatch_reason), ("why", self.reason), ("plan", self.config)):
            if text:
                out.append(f"  {label}: {text}")
        out.append(f"  planned {self.planned}; {self.native_calls} native calls so far")
        out += [f"  took the fallback {n} times: {why}" for why, n in self.refusals.items()]
        if self.last_refusal:
            out.append(f"  last: {self.last_refusal}")
        return "\n".join(out)


def _tensors(args: tuple, kwargs: dict) -> list[torch.Tensor]:
    return [v for v in (*args, *kwargs.values()) if isinstance(v, torch.Tensor)]


def _entry_point_run(fn, args: tuple, kwargs: dict) -> tuple[str, str | None, object]:
    """(run, reason, plan) of a ``helion_mlir_utils`` entry point's call."""
    tensors = _tensors(args, kwargs)
    if not tensors:
        return "unsupported", "no tensor arguments", None
    devices = {t.device for t in tensors}
    if any(d.type != "cuda" for d in devices):
        where = ", ".join(sorted(str(d) for d in devices))
        return "unsupported", f"tensors on {where}: the gpu target runs tensors on a ROCm device (the call raises)", None
    if len(devices) > 1:
        return "unsupported", "tensors on more than one device (the call raises)", None
    if not native.available():
        return "unsupported", f"{native.library_path()} is not built (the call raises)", None
    import helion_mlir_utils as U

    if fn is U.matmul and len(args) >= 2:
        a, b = args[0], args[1]
        try:
            bound = inspect.signature(U.matmul).bind(*args, **kwargs)
        except TypeError as e:
            return "unsupported", f"arguments do not bind: {e}", None
        opts = bound.arguments
        ta, tb = bool(opts.get("trans_a", False)), bool(opts.get("trans_b", False))
        if not U.supports(a, b, ta, tb):
            return "unsupported", "supports() is False for these operands (the call raises ValueError)", None
        m = a.shape[1] if ta else a.shape[0]
        k = a.shape[0] if ta else a.shape[1]
        n = b.shape[0] if tb else b.shape[1]
        plan = U.gemm_plan(a.dtype, m, n, k, trans_b=tb, block_sizes=opts.get("block_sizes"))
        return "native", None, plan
    return "native", None, None


def explain(kernel: object = _NO_KERNEL, *args: object, **kwargs: object) -> CallExplanation | dict[str, object]:
    """What ``kernel(*args, **kwargs)`` would do now on this target; runs,
    compiles and caches nothing (``_compiler/call_trace.py:220-270`` of the
    reference). ``kernel`` is a prepared call, a bound launch, a
    ``helion_mlir_utils`` entry point or a Helion kernel. Without arguments:
    what the native path has done in this process -- the library, native
    calls, run-time compilations and the output pool (this target's own
    report)."""
    if kernel is _NO_KERNEL:
        from . import output_pool

        return {
            "library": str(native.library_path()),
            "library_built": native.available(),
            "native_calls": native.native_calls(),
            "jit": native.jit_info() if native.available() else None,
            "output_pool": output_pool.output_pool_stats(),
        }
    if isinstance(kernel, PreparedCall):
        why = kernel.refusal(args)
        plan = getattr(kernel.kernel, "plan", None)
        return CallExplanation(
            type(kernel.kernel).__name__, "gpu", "direct", None, "general" if why else "native",
            why[1] if why else None, plan() if callable(plan) else None, True, kernel.native_calls,
            dict(kernel.refusals), kernel.last_refusal,
        )
    if isinstance(kernel, GpuLaunch):
        plan = getattr(kernel, "plan", None)
        return CallExplanation(type(kernel).__name__, "gpu", "direct", None, "native", None,
                               plan() if callable(plan) else None, True, getattr(kernel, "calls", 0), {}, None)
    if callable(kernel) and getattr(kernel, "__module__", "").startswith("helion_mlir_utils"):
        run, reason, plan = _entry_point_run(kernel, args, kwargs)
        return CallExplanation(kernel.__name__, "gpu", "bind", "an entry point plans and binds its launch per call",
                               run, reason, plan, False, 0, {}, None)
    if hasattr(kernel, "bind") and hasattr(kernel, "settings"):
        name = getattr(kernel, "name", type(kernel).__name__)
        return CallExplanation(str(name), getattr(kernel.settings, "backend", None), "bind", None, "compile",
                               "the gpu target does not compile @helion.kernel(backend=\"mlir\") kernels; the "
                               "helion_mlir_utils entry points run on it", None, False, 0, {}, None)
    raise TypeError(f"explain: a {type(kernel).__name__} is not a kernel of this backend")
