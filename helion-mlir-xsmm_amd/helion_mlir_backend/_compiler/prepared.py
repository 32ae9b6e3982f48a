"""Prepared launches: a kernel call with every argument but the varying ones
bound once, so that a call does no host work beyond a few checks and one
native launch.

Stands in for ``prepared_call`` / ``PreparedRun`` of the reference
(``_compiler/mlir/driver.py:748-788``, ``native/call.cpp:703-830``). A prepared
call checks its varying tensors' shape, dtype, device and contiguity; any
other call takes ``fallback`` (the general entry point, which raises for what
it cannot take), as the reference's ``PreparedRun`` does.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch


class PreparedCall:
    """``launch(*varying)`` for tensors like ``examples``; else ``fallback``."""

    __slots__ = ("_launch", "_fallback", "_specs", "calls")

    def __init__(
        self,
        launch: Callable[..., torch.Tensor],
        examples: Sequence[torch.Tensor],
        fallback: Callable[..., torch.Tensor],
    ) -> None:
        self._launch = launch
        self._fallback = fallback
        self._specs = tuple((tuple(t.shape), t.dtype, t.device) for t in examples)
        self.calls = 0

    def matches(self, args: Sequence[torch.Tensor]) -> bool:
        if len(args) != len(self._specs):
            return False
        for t, (shape, dtype, device) in zip(args, self._specs):
            if (
                not isinstance(t, torch.Tensor)
                or t.dtype is not dtype
                or t.device != device
                or tuple(t.shape) != shape
                or not t.is_contiguous()
            ):
                return False
        return True

    def __call__(self, *args: torch.Tensor) -> torch.Tensor:
        if self.matches(args):
            self.calls += 1
            return self._launch(*args)
        return self._fallback(*args)


def prepared_call(
    launch: Callable[..., torch.Tensor],
    examples: Sequence[torch.Tensor],
    fallback: Callable[..., torch.Tensor],
) -> PreparedCall:
    """A :class:`PreparedCall` of ``launch`` for arguments like ``examples``."""
    return PreparedCall(launch, examples, fallback)
