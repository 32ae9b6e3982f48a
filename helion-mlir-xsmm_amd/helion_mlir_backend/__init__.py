"""Helion ``mlir`` backend with an MI355X (gfx950) execution target.

The reference (adam-smnk/helion-mlir-xsmm, ``helion_mlir_backend/__init__.py:1-38``)
registers an external Helion backend whose kernels JIT-compile for x86 CPUs.
This build keeps the package name and public API and adds the ``gpu`` target:
``HELION_MLIR_TARGET=gpu``, or ``auto`` with tensors on a ROCm device, runs
the ``helion_mlir_utils`` hot path on hand-written gfx950 kernels
(``libhmx.so``) through ``_compiler.native``.
"""

from __future__ import annotations

from ._compiler import output_pool as output_pool
from ._compiler.call_trace import CallExplanation as CallExplanation
from ._compiler.call_trace import explain as explain
from ._compiler.native import set_native_call as set_native_call
from ._compiler.output_pool import set_output_pool as set_output_pool
from ._compiler.prepared import GpuLaunch as GpuLaunch
from ._compiler.prepared import PreparedCall as PreparedCall
from ._compiler.prepared import prepared_call as prepared_call
from ._compiler.support.errors import UnsupportedTargetError as UnsupportedTargetError
from ._compiler.targets import get_target as get_target
from ._compiler.targets import resolve_target as resolve_target
from .api import compile_mlir as compile_mlir
from .api import generate_mlir as generate_mlir
from .api import lower_mlir as lower_mlir
from .inject import install as install
from .language import InlineMLIRHint as InlineMLIRHint
from .language import inline_mlir as inline_mlir


__all__ = [
    "CallExplanation",
    "GpuLaunch",
    "InlineMLIRHint",
    "PreparedCall",
    "UnsupportedTargetError",
    "compile_mlir",
    "explain",
    "generate_mlir",
    "get_target",
    "inline_mlir",
    "install",
    "lower_mlir",
    "output_pool",
    "prepared_call",
    "resolve_target",
    "set_native_call",
    "set_output_pool",
]

# Import-time side effect, as in the reference: register backend "mlir" with
# Helion when it is present.
install()
