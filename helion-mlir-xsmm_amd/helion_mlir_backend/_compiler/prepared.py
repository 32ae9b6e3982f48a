"""Prepared launches: a kernel call with every argument but the varying ones
bound once, so that a call does no host work beyond a few checks and one
native launch.

Stands in for ``prepared_call`` / ``PreparedRun`` of the reference
(``_compiler/mlir/driver.py:748-788``, ``native/call.cpp:703-830``), with its
signature: ``prepared_call(bound_kernel, args, varying, fallback, *,
views=None, result_shape=None)``. On the gpu target a kernel with a native
run is a :class:`GpuLaunch` (a ``hmx_*`` launch with its plan and non-tensor
arguments bound, e.g. ``helion_mlir_utils.matmul.GemmLaunch``); for anything
else -- a Helion ``BoundKernel``, a plain callable -- ``prepared_call``
returns ``None``, as the reference does for kernels without a native run.

A prepared call checks its varying tensors (dtype, device, shape and
strides as in ``args``, or a contiguous tensor of ``views[k]``'s shape) and
the bound tensors' metadata (shape, strides, dtype, device, storage offset:
their data is read afresh on every call, so a bound tensor whose storage was
replaced with ``set_`` is followed); any other call takes ``fallback`` (the
general entry point, which raises for what it cannot take), as the
reference's ``PreparedRun`` does. ``set_native_call(False)`` sends every
prepared call to its fallback from then on, and ``prepared_call`` made while
off returns ``None`` (``native/__init__.py:84-95`` of the reference).
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

from . import native


class GpuLaunch:
    """Base of the gpu target's launch objects: a ``libhmx`` kernel launch
    whose plan and non-tensor arguments are bound. ``launch(*tensors)`` runs
    it on the tensors' current data and returns the result tensor."""

    __slots__ = ()

    def __call__(self, *tensors: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


# The kinds of refusal a prepared call counts.
REFUSALS = (
    "native calls are off",
    "a view changes the element count",
    "the number of varying arguments differs",
    "a varying argument differs from the prepared one",
    "a bound argument changed",
)


def _meta(t: torch.Tensor) -> tuple[object, ...]:
    return (tuple(t.shape), tuple(t.stride()), t.dtype, t.device, t.storage_offset())


class PreparedCall:
    """``bound_kernel(*args with the varying positions replaced)`` for
    varying tensors like the examples; anything else takes ``fallback``.
    ``native_calls`` counts the calls that launched the kernel directly."""

    __slots__ = ("_kernel", "_args", "_varying", "_fallback", "_views", "_result_shape", "_specs",
                 "_bound_meta", "_off", "native_calls", "refusals", "last_refusal")

    def __init__(
        self,
        bound_kernel: GpuLaunch,
        args: Sequence[object],
        varying: Sequence[int],
        fallback: Callable[..., object],
        views: Sequence[tuple[int, ...] | None],
        result_shape: tuple[int, ...] | None,
    ) -> None:
        self._kernel = bound_kernel
        self._args = list(args)
        self._varying = tuple(varying)
        self._fallback = fallback
        self._views = tuple(views)
        self._result_shape = result_shape
        # What each varying argument must look like: (shape, strides, dtype,
        # device) of the example, or the view's contiguous shape.
        self._specs = tuple(
            (tuple(view), None, args[i].dtype, args[i].device) if view is not None
            else (tuple(args[i].shape), tuple(args[i].stride()), args[i].dtype, args[i].device)
            for i, view in zip(self._varying, self._views)
        )
        self._bound_meta = tuple(
            (i, _meta(a)) for i, a in enumerate(self._args)
            if i not in self._varying and isinstance(a, torch.Tensor)
        )
        self._off = False
        self.native_calls = 0
        # Calls that took the fallback, by kind of refusal, and the last
        # one's reason in full (what ``explain`` reports, as the reference's
        # KernelRun.refusals / .last_refusal).
        self.refusals: dict[str, int] = {}
        self.last_refusal: str | None = None

    def disable(self) -> None:
        """Send every call to the fallback from now on."""
        self._off = True

    @property
    def calls(self) -> int:
        """The number of native calls (also ``native_calls``)."""
        return self.native_calls

    def matches(self, values: Sequence[object]) -> bool:
        """Whether a call with ``values`` launches the kernel directly."""
        if self._off or len(values) != len(self._specs):
            return False
        for t, (shape, strides, dtype, device) in zip(values, self._specs):
            if (
                not isinstance(t, torch.Tensor)
                or t.dtype is not dtype
                or t.device != device
                or tuple(t.shape) != shape
            ):
                return False
            if strides is None:
                if not t.is_contiguous():
                    return False
            elif tuple(t.stride()) != strides:
                return False
        return all(_meta(self._args[i]) == meta for i, meta in self._bound_meta)

    @property
    def kernel(self) -> GpuLaunch:
        """The bound launch this call runs natively."""
        return self._kernel

    def refusal(self, values: Sequence[object]) -> tuple[str, str] | None:
        """Why a call with ``values`` would take the fallback -- (kind, the
        reason in full) -- or None when it would launch natively."""
        if not native.enabled():
            return REFUSALS[0], "native calls are off (set_native_call(False))"
        if self._off:
            return REFUSALS[1], "a view changes its argument's element count: every call takes the fallback"
        if len(values) != len(self._specs):
            return REFUSALS[2], f"{len(values)} varying arguments, prepared with {len(self._specs)}"
        for k, (t, (shape, strides, dtype, device)) in enumerate(zip(values, self._specs)):
            if not isinstance(t, torch.Tensor):
                return REFUSALS[3], f"varying argument {k} is a {type(t).__name__}, not a tensor"
            got = (t.dtype, t.device, tuple(t.shape))
            if got != (dtype, device, shape):
                return REFUSALS[3], (f"varying argument {k} is {t.dtype} of shape {tuple(t.shape)} on {t.device}, "
                                     f"prepared {dtype} of shape {shape} on {device}")
            if strides is None and not t.is_contiguous():
                return REFUSALS[3], f"varying argument {k} is not contiguous (strides {tuple(t.stride())})"
            if strides is not None and tuple(t.stride()) != strides:
                return REFUSALS[3], f"varying argument {k} has strides {tuple(t.stride())}, prepared {strides}"
        for i, meta in self._bound_meta:
            if _meta(self._args[i]) != meta:
                return REFUSALS[4], (f"bound argument {i} changed shape, strides, dtype, device or storage "
                                     f"offset since the call was prepared")
        return None

    def __call__(self, *values: object) -> object:
        if not native.enabled() or not self.matches(values):
            why = self.refusal(values)
            if why is not None:
                self.refusals[why[0]] = self.refusals.get(why[0], 0) + 1
                self.last_refusal = why[1]
            return self._fallback(*values)
        full = list(self._args)
        for i, value, view in zip(self._varying, values, self._views):
            full[i] = value if view is None else value.view(self._args[i].shape)
        self.native_calls += 1
        out = self._kernel(*full)
        return out if self._result_shape is None else out.view(self._result_shape)


def prepared_call(
    bound_kernel: object,
    args: Sequence[object],
    varying: Sequence[int],
    fallback: Callable[..., object],
    *,
    views: Sequence[Sequence[int] | None] | None = None,
    result_shape: Sequence[int] | None = None,
) -> PreparedCall | None:
    """``lambda *v: bound_kernel(*args with v at the varying positions)``,
    launched natively when the varying tensors and the bound ones look as
    when prepared; any other call returns ``fallback(*v)``. ``None`` if
    ``bound_kernel`` has no native run on this target (it is not a
    :class:`GpuLaunch`) or native calls are off.

    ``views[k]`` (optional, per varying argument): the caller passes a
    contiguous tensor of that shape, standing for its contiguous view of the
    argument's shape. ``result_shape``: the result is returned as
    ``result.view(result_shape)``. Neither may change the element count: a
    view that does sends every call to ``fallback``, as in the reference."""
    if not isinstance(bound_kernel, GpuLaunch) or not native.enabled():
        return None
    args = list(args)
    varying = [int(i) for i in varying]
    if len(set(varying)) != len(varying) or any(not 0 <= i < len(args) for i in varying):
        raise ValueError(f"prepared_call: varying positions {varying} do not index {len(args)} arguments")
    for i in varying:
        if not isinstance(args[i], torch.Tensor):
            raise ValueError(f"prepared_call: varying argument {i} is not a tensor")
    if views is None:
        views_t: list[tuple[int, ...] | None] = [None] * len(varying)
    else:
        if len(views) != len(varying):
            raise ValueError("prepared_call: one view (or None) per varying argument")
        views_t = [None if v is None else tuple(int(d) for d in v) for v in views]
    shape = None if result_shape is None else tuple(int(d) for d in result_shape)
    prepared = PreparedCall(bound_kernel, args, varying, fallback, views_t, shape)
    # A view must stand for the argument's contiguous data: one that changes
    # the element count (or of a strided argument) leaves only the fallback.
    for i, view in zip(varying, views_t):
        if view is not None and (not args[i].is_contiguous() or _numel(view) != args[i].numel()):
            prepared.disable()
    return prepared


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n
