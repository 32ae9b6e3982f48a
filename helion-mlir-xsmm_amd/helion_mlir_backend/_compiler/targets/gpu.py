"""The ``gpu`` target: hand-written gfx950 (MI355X) kernels behind ``libhmx.so``.

New in this build (the reference registers only ``cpu``,
``_compiler/targets/__init__.py:30-36``). It has one pipeline, ``hip``: the
``helion_mlir_utils`` entry points dispatch to its kernels directly, and
``Config.block_sizes`` picks the workgroup tile of its GEMMs.
"""

from __future__ import annotations

import torch

from .. import native
from ..support import debug
from ..support.errors import UnsupportedTargetError
from .base import MLIRTarget


class GpuTarget(MLIRTarget):
    name = "gpu"
    pipelines = debug.GPU_PIPELINES
    device_type = "cuda"  # ROCm devices under torch
    buffer_alignment = 256

    def default_pipeline(self) -> str:
        return "hip"

    def hardware_name(self) -> str:
        if torch.cuda.is_available():
            return torch.cuda.get_device_properties(0).gcnArchName
        return "gfx950"

    def validate_environment(self) -> None:
        if not torch.cuda.is_available():
            raise UnsupportedTargetError(
                "MLIR target 'gpu'", reason="no ROCm device is visible to torch"
            )
        native.lib()
        native.ensure_device(torch.device("cuda", torch.cuda.current_device()))
