"""Kernels of one body that differ by tile config (reference
``helion_mlir_utils/kernels.py:14-31``): ``@per_config(backend="mlir")`` makes
a body's name take a hashable ``block_sizes`` and return that config's
``helion.Kernel``. It needs Helion; on the gpu target ``block_sizes`` reaches
the kernels as the ``block_sizes`` argument of ``matmul``."""

from __future__ import annotations

import functools
from typing import Callable

from helion_mlir_backend._compiler.support.errors import UnsupportedOperationError


def per_config(**kernel_args: object) -> Callable[[Callable[..., object]], Callable[[tuple[int, ...]], object]]:
    def wrap(body: Callable[..., object]) -> Callable[[tuple[int, ...]], object]:
        @functools.cache
        def for_config(block_sizes: tuple[int, ...]) -> object:
            try:
                import helion
            except ImportError as exc:
                raise UnsupportedOperationError(
                    "per_config", reason=f"Helion kernels need Helion, which is not importable ({exc})"
                ) from exc
            return helion.kernel(body, config=helion.Config(block_sizes=list(block_sizes)), **kernel_args)

        for_config.body = body  # type: ignore[attr-defined]
        return for_config

    return wrap
