"""Elementwise ops of the gpu target (reference ``helion_mlir_utils/elementwise.py:14-56``):
16-byte vectors per lane, one read and one write per element."""

from __future__ import annotations

from torch import Tensor

from helion_mlir_backend import output_pool
from helion_mlir_backend._compiler import native

from ._gpu import SUPPORTED_DTYPES, is_gpu, on_device

__all__ = ["leaky_relu", "relu", "scalar_mul"]


def _run(name: str, op: int, x: Tensor, arg: float) -> Tensor:
    if not is_gpu(x) or x.dtype not in SUPPORTED_DTYPES:
        raise ValueError(
            f"{name}() runs float32/bfloat16 tensors on a ROCm device, got {x.dtype} on {x.device}"
        )
    x = x.contiguous()
    out = output_pool.empty_like(x)
    if x.numel() == 0:
        return out
    with on_device(x.device) as stream:
        native.call("hmx_elementwise", op, native.dtype_code(x.dtype), x.data_ptr(), out.data_ptr(),
                    x.numel(), float(arg), stream)
    return out


def relu(x: Tensor) -> Tensor:
    """Elementwise ``max(x, 0)`` (NaN stays NaN)."""
    return _run("relu", native.ELT_RELU, x, 0.0)


def leaky_relu(x: Tensor, negative_slope: float = 0.01) -> Tensor:
    """Elementwise LeakyReLU: ``x if x > 0 else x * negative_slope``."""
    return _run("leaky_relu", native.ELT_LEAKY_RELU, x, negative_slope)


def scalar_mul(a: Tensor, s: float | Tensor) -> Tensor:
    """Elementwise ``a * s``."""
    if isinstance(s, Tensor):
        s = float(s)
    return _run("scalar_mul", native.ELT_SCALE, a, s)
