"""Target selection: which device target runs a kernel.

The public functions keep the reference's names, precedence and errors
(``_compiler/targets/__init__.py:30-85``): an explicit target name wins,
then ``HELION_MLIR_TARGET``, then the device the kernel's tensors live on
(``auto``). Here the device rule is read off the target classes themselves
-- each declares the ``torch.device`` type it serves -- so the ``gpu``
target (ROCm devices, ``torch.device("cuda")``) joins ``cpu`` by being
listed in ``_TARGETS`` and nothing else.
"""

from __future__ import annotations

import threading
from typing import TYPE_CHECKING

from ..support.debug import target_override
from ..support.errors import UnsupportedTargetError
from .base import MLIRTarget
from .cpu import CpuTarget
from .gpu import GpuTarget

if TYPE_CHECKING:
    import torch

__all__ = [
    "CpuTarget",
    "GpuTarget",
    "MLIRTarget",
    "get_target",
    "resolve_target",
    "target_config_keys",
]


class _TargetTable:
    """The known target classes, looked up by name or by the device type
    they serve; each target is built on first use and shared afterwards
    (targets carry no per-kernel state)."""

    def __init__(self, classes: tuple[type[MLIRTarget], ...]) -> None:
        self._by_name = {cls.name: cls for cls in classes}
        self._name_for_device = {cls.device_type: cls.name for cls in classes}
        self._built: dict[str, MLIRTarget] = {}
        self._lock = threading.Lock()

    def names(self) -> tuple[str, ...]:
        return tuple(self._by_name)

    def config_keys(self) -> frozenset[str]:
        keys: set[str] = set()
        for cls in self._by_name.values():
            keys |= cls.config_keys
        return frozenset(keys)

    def build(self, name: str) -> MLIRTarget:
        cls = self._by_name.get(name)
        if cls is None:
            raise ValueError(f"unknown MLIR target {name!r}; expected one of {self.names()}")
        target = self._built.get(name)
        if target is None:
            with self._lock:
                target = self._built.setdefault(name, cls())
        return target

    def name_for_device(self, device_type: str) -> str | None:
        return self._name_for_device.get(device_type)

    def device_types(self) -> tuple[str, ...]:
        return tuple(self._name_for_device)


# cpu serves torch.device("cpu"); gpu serves ROCm devices ("cuda" under torch).
_TARGETS = _TargetTable((CpuTarget, GpuTarget))


def target_config_keys() -> frozenset[str]:
    """Config keys any target's lowering understands (``MLIRTarget.config_keys``)."""
    return _TARGETS.config_keys()


def get_target(name: str) -> MLIRTarget:
    """The target called ``name`` (``cpu`` or ``gpu``); ``ValueError`` for
    any other name."""
    return _TARGETS.build(name)


def resolve_target(device: torch.device | None = None, override: str | None = None) -> MLIRTarget:
    """The target for a kernel whose tensors are on ``device`` (``None`` means
    the CPU). A name in ``override`` -- or, when ``override`` is ``None``, in
    ``HELION_MLIR_TARGET`` -- selects that target; ``auto`` (or no name)
    follows the device."""
    name = target_override() if override is None else override
    if name not in (None, "auto"):
        return get_target(name)
    kind = "cpu" if device is None else device.type
    if kind == "meta":
        raise UnsupportedTargetError(
            "MLIR compilation for meta tensors",
            reason="meta tensors have no device to pick the target from",
            alternatives=["target='cpu'", "target='gpu'", "HELION_MLIR_TARGET"],
        )
    chosen = _TARGETS.name_for_device(kind)
    if chosen is None:
        served = ", ".join(_TARGETS.device_types())
        raise UnsupportedTargetError(
            f"MLIR compilation for device '{kind}'",
            reason=f"the MLIR backend runs on {served} tensors (ROCm devices are 'cuda' under torch)",
        )
    return get_target(chosen)
