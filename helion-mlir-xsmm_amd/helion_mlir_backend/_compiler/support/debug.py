"""Environment-driven options, read in one place.

``HELION_MLIR_TARGET`` of the reference (``mlir/support/debug.py:11,62-68``)
accepts ``auto`` and ``cpu``; this build adds ``gpu``, which ``auto`` selects
for tensors on a ROCm device (``torch.device("cuda")`` under ROCm torch).
"""

from __future__ import annotations

import os

PIPELINES = ("opt", "scalar")
"""The CPU target's lighthouse pipelines (names kept for the reference's API)."""
GPU_PIPELINES = ("hip",)
"""The gpu target's only pipeline: the hand-written gfx950 kernels."""
TARGETS = ("auto", "cpu", "gpu")
"""``HELION_MLIR_TARGET`` values; ``auto`` follows the device."""
PIPELINE_CONFIG_KEY = "mlir_pipeline"


def target_override() -> str | None:
    """``HELION_MLIR_TARGET``; ``None`` if unset or ``auto``."""
    target = os.environ.get("HELION_MLIR_TARGET", "").strip() or "auto"
    if target not in TARGETS:
        raise ValueError(f"HELION_MLIR_TARGET={target!r}; expected one of {TARGETS}")
    return None if target == "auto" else target


def default_pipeline() -> str:
    """``HELION_MLIR_PIPELINE`` (``opt`` or ``scalar``); ``opt`` if unset."""
    pipeline = os.environ.get("HELION_MLIR_PIPELINE", "").strip() or "opt"
    if pipeline not in PIPELINES:
        raise ValueError(f"HELION_MLIR_PIPELINE={pipeline!r}; expected one of {PIPELINES}")
    return pipeline
