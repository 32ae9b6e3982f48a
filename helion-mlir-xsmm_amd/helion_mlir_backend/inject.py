"""Backend registration (reference ``helion_mlir_backend/inject.py:22-56``).

``install()`` registers the backend name ``"mlir"`` with Helion when Helion is
importable and returns ``True``; without Helion it returns ``False``, as the
reference does on ``ImportError``. The gpu target's kernels do not need
Helion: ``helion_mlir_utils`` reaches them directly.
"""

from __future__ import annotations

import logging

log = logging.getLogger(__name__)

_installed = [False]


def install() -> bool:
    """Register the ``mlir`` backend into Helion's registry if Helion is present."""
    if _installed[0]:
        return True
    try:
        from helion._compiler.backend_registry import register_compiler_backend  # noqa: F401
    except ImportError as exc:
        log.debug("Helion is not importable; the mlir backend is not registered: %s", exc)
        return False
    # A Helion is present, but the Helion -> Linalg compiler is not part of this
    # build: nothing to register a compile function for.
    log.info("Helion found; generic @helion.kernel(backend='mlir') compilation is not part of this build")
    return False
