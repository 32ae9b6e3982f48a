"""Error types of the backend.

Mirrors ``helion_mlir_backend/_compiler/mlir/support/errors.py:18-60`` of the
reference: every error derives from ``helion.exc.BaseError`` when Helion is
importable, else from ``Exception`` (Helion is optional for the ``gpu``
target, whose kernels do not go through Helion's compiler).
"""

from __future__ import annotations

try:  # pragma: no cover - depends on the environment
    import helion.exc as _helion_exc

    _Base: type[Exception] = _helion_exc.BaseError
except ImportError:  # Helion absent: the gpu target still works.
    _Base = Exception


class MLIRBackendError(_Base):  # type: ignore[misc, valid-type]
    """Base exception for all backend errors."""

    message = "{0}"


class UnsupportedOperationError(MLIRBackendError):
    """Raised when an unsupported operation is encountered."""

    def __init__(
        self,
        op_name: str,
        reason: str | None = None,
        alternatives: list[str] | None = None,
    ) -> None:
        msg = f"Unsupported operation: {op_name}"
        if reason:
            msg += f"\nReason: {reason}"
        if alternatives:
            msg += f"\nAlternatives: {', '.join(alternatives)}"
        super().__init__(msg)
        self.op_name = op_name
        self.reason = reason
        self.alternatives = alternatives

    def __reduce__(self) -> tuple:
        args = (self.op_name, self.reason, self.alternatives)
        return type(self), args, self.__dict__


class UnsupportedTargetError(UnsupportedOperationError, NotImplementedError):
    """Raised for a device (or target name) no target compiles for. Also a
    :class:`NotImplementedError`, as in the reference."""
