"""The CPU target of the reference (``_compiler/targets/cpu.py:66-118``): the
x86 AMX/AVX-512 lowering through lighthouse. This build keeps its name and
device mapping so that target resolution behaves as in the reference, but the
lowering itself is not part of the build: running a kernel on it raises."""

from __future__ import annotations

import platform

from ..support import debug
from ..support.errors import UnsupportedTargetError
from .base import MLIRTarget


class CpuTarget(MLIRTarget):
    name = "cpu"
    pipelines = debug.PIPELINES
    device_type = "cpu"

    def default_pipeline(self) -> str:
        return debug.default_pipeline()

    def hardware_name(self) -> str:
        return platform.processor() or platform.machine()

    def validate_environment(self) -> None:
        try:
            import helion  # noqa: F401
            import lighthouse  # noqa: F401
        except ImportError as exc:
            raise UnsupportedTargetError(
                "MLIR target 'cpu'",
                reason=f"the CPU lowering needs Helion and lighthouse ({exc})",
                alternatives=["tensors on a gfx950 GPU (target 'gpu')"],
            ) from exc
