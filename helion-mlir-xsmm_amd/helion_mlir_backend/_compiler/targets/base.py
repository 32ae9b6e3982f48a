"""The device-specific half of running a kernel.

Mirrors ``MLIRTarget`` of the reference (``_compiler/targets/base.py:54-212``):
a target owns its pipelines, the device checks around a call and the name
that keys caches. Targets hold no per-kernel state: one instance serves
every kernel.
"""

from __future__ import annotations

import abc
from typing import ClassVar

import torch


class MLIRTarget(abc.ABC):
    """A device the backend runs kernels on."""

    name: ClassVar[str]
    pipelines: ClassVar[tuple[str, ...]]
    config_keys: ClassVar[frozenset[str]] = frozenset()
    device_type: ClassVar[str]
    buffer_alignment: ClassVar[int] = 64

    @abc.abstractmethod
    def default_pipeline(self) -> str:
        """The pipeline of configs that name none."""

    def resolve_pipeline(self, pipeline: str | None) -> str:
        """``pipeline``, or the default for ``None``; ``ValueError`` if the
        target has no such pipeline."""
        if pipeline is None:
            return self.default_pipeline()
        if pipeline not in self.pipelines:
            raise ValueError(
                f"unknown pipeline {pipeline!r} for the MLIR target {self.name!r}; "
                f"expected one of {self.pipelines}"
            )
        return pipeline

    @abc.abstractmethod
    def hardware_name(self) -> str:
        """What the target runs on (keys autotune caches)."""

    def validate_environment(self) -> None:
        """Raise if this process cannot run the target's kernels."""

    def check_tensor(self, name: str, tensor: torch.Tensor) -> None:
        """Raise ``NotImplementedError`` for a tensor on another device."""
        if tensor.device.type != self.device_type:
            raise NotImplementedError(
                f"{name} is on {tensor.device}; only {self.device_type.upper()} is "
                f"supported by the MLIR target {self.name!r}"
            )
