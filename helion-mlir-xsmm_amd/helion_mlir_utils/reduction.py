"""Row/column reductions and gemv of the gpu target.

Reference: ``helion_mlir_utils/reduction.py`` (``matvec`` 24-67, ``row_sum``
79-121, ``column_sum`` 124-163, ``row_dot`` 166-212). Memory-bound: each
element of ``x`` is read once, f32 accumulation, one rounding.
"""

from __future__ import annotations

import ctypes
from typing import Callable

import torch
from torch import Tensor

from helion_mlir_backend import output_pool
from helion_mlir_backend._compiler import native

from ._gpu import SUPPORTED_DTYPES, epilogue_code, identity_epilogue, is_gpu, on_device

__all__ = ["column_sum", "matvec", "row_dot", "row_sum", "supports_matvec"]


def _check(name: str, x: Tensor) -> None:
    if x.dim() != 2:
        raise ValueError(f"{name}() expects a 2-D tensor, got {tuple(x.shape)}")
    if not is_gpu(x) or x.dtype not in SUPPORTED_DTYPES:
        raise ValueError(
            f"{name}() runs float32/bfloat16 tensors on a ROCm device, got {x.dtype} on {x.device}"
        )


def supports_matvec(a: Tensor, b: Tensor) -> bool:
    """Whether :func:`matvec` can run this pair on the gpu target."""
    if a.dtype != b.dtype or a.dtype not in SUPPORTED_DTYPES:
        return False
    if not is_gpu(a, b) or a.device != b.device:
        return False
    if a.dim() != 2 or b.dim() != 2 or b.shape[1] != 1:
        return False
    return a.shape[1] == b.shape[0]


def matvec(a: Tensor, b: Tensor) -> Tensor:
    """``A @ b`` for ``A: [M, K]``, ``b: [K, 1]`` -> ``[M, 1]``; raises
    ``ValueError`` if unsupported (see :func:`supports_matvec`)."""
    if not supports_matvec(a, b):
        raise ValueError(
            f"matvec() does not support these operands: a.shape={tuple(a.shape)} "
            f"a.dtype={a.dtype} a.device={a.device}, b.shape={tuple(b.shape)} "
            f"b.dtype={b.dtype} b.device={b.device}. b must be K-by-1, dtype must be "
            "float32 or bfloat16, both on one ROCm device. Check supports_matvec() before "
            "calling, or use torch.matmul directly for unsupported cases."
        )
    m, k = map(int, a.shape)
    a = a.contiguous()
    x = b.reshape(k).contiguous()
    out = output_pool.empty((m, 1), dtype=a.dtype, device=a.device)
    if m == 0:
        return out
    with on_device(a.device) as stream:
        native.call("hmx_matvec", native.dtype_code(a.dtype), a.data_ptr(), x.data_ptr(), out.data_ptr(), m, k, stream)
    return out


def row_sum(x: Tensor, epilogue: Callable[[Tensor], Tensor] = identity_epilogue) -> Tensor:
    """``epilogue(x.sum(1, keepdim=True))`` of a 2-D ``x``, summed in f32."""
    _check("row_sum", x)
    code, arg, program = epilogue_code(epilogue)
    m, n = map(int, x.shape)
    x = x.contiguous()
    out = output_pool.empty((m, 1), dtype=x.dtype, device=x.device)
    if m == 0:
        return out
    with on_device(x.device) as stream:
        native.call("hmx_row_sum", native.dtype_code(x.dtype), x.data_ptr(), out.data_ptr(), m, n, code, arg,
                    native.program_arg(program), stream)
    return out


def column_sum(x: Tensor) -> Tensor:
    """``x.sum(0)`` of a 2-D ``x`` in f32 (an f32 ``[N]``)."""
    _check("column_sum", x)
    m, n = map(int, x.shape)
    x = x.contiguous()
    out = output_pool.empty((n,), dtype=torch.float32, device=x.device)
    if n == 0:
        return out
    ws_bytes = ctypes.c_int64()
    native.check(native.lib().hmx_column_sum_plan(m, n, ctypes.byref(ws_bytes)), "hmx_column_sum_plan")
    # Row-chunk partials (kept alive by `ws` until the call is enqueued; torch's
    # stream-ordered allocator keeps them until the kernels have run).
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=x.device) if ws_bytes.value else None
    with on_device(x.device) as stream:
        native.call("hmx_column_sum", native.dtype_code(x.dtype), x.data_ptr(), out.data_ptr(), m, n,
                    native.ptr(ws), ws_bytes.value, stream)
    return out


def row_dot(x: Tensor, v: Tensor, epilogue: Callable[[Tensor], Tensor] = identity_epilogue) -> Tensor:
    """``epilogue(x @ v)`` of a 2-D ``x`` and an f32 ``[N]``, in f32 and
    rounded once, as ``[M, 1]``."""
    if x.dim() != 2 or v.dim() != 1 or x.shape[1] != v.shape[0]:
        raise ValueError(
            f"row_dot() expects [M, N] and [N], got {tuple(x.shape)}, {tuple(v.shape)}"
        )
    if v.dtype != torch.float32:
        raise ValueError(f"row_dot() expects an f32 vector, got {v.dtype}")
    _check("row_dot", x)
    code, arg, program = epilogue_code(epilogue)
    m, n = map(int, x.shape)
    x = x.contiguous()
    v = v.to(x.device).contiguous()
    out = output_pool.empty((m, 1), dtype=x.dtype, device=x.device)
    if m == 0:
        return out
    with on_device(x.device) as stream:
        native.call("hmx_row_dot", native.dtype_code(x.dtype), x.data_ptr(), v.data_ptr(), out.data_ptr(),
                    m, n, code, arg, native.program_arg(program), stream)
    return out
