"""``inline_mlir`` (reference ``helion_mlir_backend/language.py:26-80``): MLIR
text snippets inside Helion kernels. MLIR snippets have no meaning on
hand-written HIP kernels; the function is kept for the API and raises."""

from __future__ import annotations

from ._compiler.support.errors import UnsupportedOperationError


class InlineMLIRHint:
    """Placeholder of the reference's snippet hint type."""


def inline_mlir(*args: object, **kwargs: object) -> object:
    raise UnsupportedOperationError(
        "inline_mlir",
        reason="MLIR snippets need the Helion -> MLIR CPU compiler, which this build does not contain",
    )
