"""Public compile API of the backend: ``generate_mlir``, ``compile_mlir`` and
``lower_mlir`` (reference ``helion_mlir_backend/api.py:16-148``).

These compile arbitrary ``@helion.kernel(backend="mlir")`` kernels through the
reference's Helion -> Linalg -> x86 pipeline, which this build does not
contain (Helion, MLIR and lighthouse are not part of it). On the ``gpu``
target the hot-path kernels are reached through ``helion_mlir_utils``; these
functions raise ``UnsupportedTargetError`` naming that alternative.
"""

from __future__ import annotations

from typing import Any

from ._compiler.support.errors import UnsupportedTargetError
from ._compiler.targets import resolve_target


def _device_of(args: list[object]) -> Any:
    import torch

    for arg in args:
        if isinstance(arg, torch.Tensor):
            return arg.device
    return None


def _unsupported(what: str, args: list[object], target: str | None) -> UnsupportedTargetError:
    chosen = resolve_target(_device_of(args), target)
    return UnsupportedTargetError(
        f"{what} for the MLIR target '{chosen.name}'",
        reason=(
            "this build runs the helion_mlir_utils hot path on hand-written gfx950 "
            "kernels; compiling arbitrary Helion kernels needs the reference's "
            "Helion/MLIR/lighthouse CPU pipeline, which is not part of it"
        ),
        alternatives=["helion_mlir_utils.matmul / linear / bmm / softmax / rms_norm / ..."],
    )


def generate_mlir(kernel: object, args: list[object], *, config: object | None = None, target: str | None = None) -> Any:
    raise _unsupported("generate_mlir", args, target)


def compile_mlir(
    kernel: object,
    args: list[object],
    *,
    config: object | None = None,
    target: str | None = None,
    pipeline: str | None = None,
) -> Any:
    raise _unsupported("compile_mlir", args, target)


def lower_mlir(kernel: object, args: list[object], *, config: object | None = None, target: str | None = None, **_: object) -> Any:
    raise _unsupported("lower_mlir", args, target)
