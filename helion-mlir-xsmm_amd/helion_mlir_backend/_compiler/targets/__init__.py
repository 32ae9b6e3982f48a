"""Device targets and how a kernel's target is chosen.

As in the reference (``_compiler/targets/__init__.py:1-85``), the target is the
one named by the caller, else ``HELION_MLIR_TARGET``, else the one of the device
of the kernel's tensors (``auto``). This build registers ``gpu`` beside
``cpu`` and maps ROCm devices (``torch.device("cuda")``) to it.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from ..support.debug import target_override
from ..support.errors import UnsupportedTargetError
from .base import MLIRTarget
from .cpu import CpuTarget
from .gpu import GpuTarget

if TYPE_CHECKING:
    from collections.abc import Callable

    import torch

__all__ = [
    "CpuTarget",
    "GpuTarget",
    "MLIRTarget",
    "get_target",
    "resolve_target",
    "target_config_keys",
]

_FACTORIES: dict[str, Callable[[], MLIRTarget]] = {"cpu": CpuTarget, "gpu": GpuTarget}
_TARGET_CLASSES: tuple[type[MLIRTarget], ...] = (CpuTarget, GpuTarget)
_DEVICE_TARGETS = {"cpu": "cpu", "cuda": "gpu"}
"""The target of each ``torch.device`` type under ``auto``."""
_INSTANCES: dict[str, MLIRTarget] = {}


def target_config_keys() -> frozenset[str]:
    return frozenset().union(*(cls.config_keys for cls in _TARGET_CLASSES))


def get_target(name: str) -> MLIRTarget:
    """The target named ``name`` (``cpu`` or ``gpu``)."""
    if name not in _FACTORIES:
        raise ValueError(f"unknown MLIR target {name!r}; expected one of {tuple(_FACTORIES)}")
    if (target := _INSTANCES.get(name)) is None:
        target = _INSTANCES[name] = _FACTORIES[name]()
    return target


def resolve_target(device: torch.device | None = None, override: str | None = None) -> MLIRTarget:
    """The target running a kernel whose tensors are on ``device`` (``None``:
    the CPU). ``override`` names the target (``auto``: follow the device); if it
    is ``None``, ``HELION_MLIR_TARGET`` may."""
    name = override if override is not None else target_override()
    if name is not None and name != "auto":
        return get_target(name)
    device_type = "cpu" if device is None else device.type
    if device_type == "meta":
        raise UnsupportedTargetError(
            "MLIR compilation for meta tensors",
            reason="meta tensors have no device to pick the target from",
            alternatives=["target='cpu'", "target='gpu'", "HELION_MLIR_TARGET"],
        )
    if device_type not in _DEVICE_TARGETS:
        raise UnsupportedTargetError(
            f"MLIR compilation for device '{device_type}'",
            reason="the MLIR backend runs on CPU and ROCm (gfx950) tensors",
        )
    return get_target(_DEVICE_TARGETS[device_type])
