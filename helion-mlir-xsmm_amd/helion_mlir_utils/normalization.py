"""Row normalizations of the gpu target: softmax, RMSNorm, GroupNorm/LayerNorm.

Reference: ``helion_mlir_utils/normalization.py`` (softmax ``28-87, 138-153``,
GroupNorm ``94-123, 156-196``). Each row (or (row, group) unit) is owned by
one wave64, read once from HBM into registers, reduced in f32 across the
wave and written once, rounded to the input dtype. RMSNorm is new API: the
reference has none.
"""

from __future__ import annotations

import operator
from typing import Callable

import torch
from torch import Tensor

from helion_mlir_backend import output_pool
from helion_mlir_backend._compiler import native

from ._gpu import SUPPORTED_DTYPES, epilogue_code, is_gpu, on_device

__all__ = ["group_norm", "layer_norm", "rms_norm", "softmax"]


def _check(name: str, x: Tensor) -> None:
    if x.dim() != 2:
        raise ValueError(f"{name}() expects a 2-D tensor, got {tuple(x.shape)}")
    if not is_gpu(x) or x.dtype not in SUPPORTED_DTYPES:
        raise ValueError(
            f"{name}() runs float32/bfloat16 tensors on a ROCm device, got {x.dtype} on {x.device}"
        )


def _target(x: Tensor, in_place: bool) -> tuple[Tensor, Tensor]:
    """(input, output): in place writes into a contiguous ``x``."""
    x = x.contiguous() if not in_place else x
    if in_place and not x.is_contiguous():
        x = x.contiguous()
    return x, (x if in_place else output_pool.empty_like(x))


def softmax(x: Tensor, in_place: bool = False) -> Tensor:
    """Softmax over the last dim of a 2-D ``x``, f32 inside: ``exp(x - max) *
    (1 / sum)`` rounded once (``normalization.py:138-153``). A row with a NaN or
    +inf gives NaN, one column gives 1 (NaN for NaN/inf), as torch. ``in_place``
    may overwrite a contiguous ``x``; use the result, not ``x``."""
    _check("softmax", x)
    m, n = map(int, x.shape)
    x, y = _target(x, in_place)
    if m == 0 or n == 0:
        return y
    with on_device(x.device) as stream:
        native.call("hmx_softmax_rows", native.dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), m, n, stream)
    return y


def rms_norm(x: Tensor, weight: Tensor | None = None, eps: float = 1e-6, in_place: bool = False) -> Tensor:
    """RMSNorm of the rows of a 2-D ``x``: ``x * rsqrt(mean(x**2) + eps) *
    weight`` in f32, rounded once to ``x.dtype``. ``weight`` is ``[N]`` (any of
    f32/bf16) or ``None``."""
    _check("rms_norm", x)
    m, n = map(int, x.shape)
    if weight is not None:
        if weight.dim() != 1 or int(weight.shape[0]) != n:
            raise ValueError(f"rms_norm() weight must have shape ({n},), got {tuple(weight.shape)}")
        if weight.dtype not in SUPPORTED_DTYPES:
            weight = weight.float()
        weight = weight.to(x.device).contiguous()
    x, y = _target(x, in_place)
    if m == 0 or n == 0:
        return y
    w_dtype = native.dtype_code(weight.dtype) if weight is not None else native.DTYPE_F32
    with on_device(x.device) as stream:
        native.call("hmx_rmsnorm_rows", native.dtype_code(x.dtype), x.data_ptr(), native.ptr(weight),
                    w_dtype, y.data_ptr(), m, n, float(eps), stream)
    return y


def _second_operand(y: Tensor, extra: Tensor) -> Tensor:
    return y


_EXTRA_OPS: dict[object, int] = {
    _second_operand: native.EXTRA_NONE,
    torch.add: native.EXTRA_ADD,
    operator.add: native.EXTRA_ADD,
    torch.mul: native.EXTRA_MUL,
    operator.mul: native.EXTRA_MUL,
}


def _extra_op(epilogue: Callable[[Tensor, Tensor], Tensor]) -> tuple[int, int, float, native.Program | None]:
    """(extra op, activation, activation arg, program) fused for a group-norm
    epilogue: ``_second_operand`` (y), ``torch.add``/``torch.mul`` with the
    extra operand, ``GroupNormEpilogue``, or any other elementwise
    ``epilogue(y, extra)`` traced into an epilogue program (extra op none: the
    program reads the extra operand itself)."""
    from ._program import traced_epilogue

    if isinstance(epilogue, GroupNormEpilogue) and epilogue.activation[0] != native.EPI_PROGRAM:
        return epilogue.extra_op, epilogue.activation[0], epilogue.activation[1], None
    if epilogue in _EXTRA_OPS:
        return _EXTRA_OPS[epilogue], native.EPI_IDENTITY, 0.0, None
    program = traced_epilogue(epilogue, 2)
    if program is None:
        return native.EXTRA_NONE, native.EPI_IDENTITY, 0.0, None
    return native.EXTRA_NONE, native.EPI_PROGRAM, 0.0, program.struct


class GroupNormEpilogue:
    """A group-norm epilogue the gpu kernel fuses: ``act(y op extra)`` with
    ``op`` one of ``None`` (ignore extra), ``"add"``, ``"mul"`` and ``act`` a
    fusable activation (see ``matmul``'s epilogues)."""

    def __init__(self, op: str | None = None, activation: Callable[[Tensor], Tensor] | None = None) -> None:
        from ._gpu import identity_epilogue

        self.op = op
        self.extra_op = {None: native.EXTRA_NONE, "add": native.EXTRA_ADD, "mul": native.EXTRA_MUL}[op]
        self.fn = activation or identity_epilogue
        self.activation = epilogue_code(self.fn)

    def __call__(self, y: Tensor, extra: Tensor) -> Tensor:
        if self.op == "add":
            y = y + extra
        elif self.op == "mul":
            y = y * extra
        return self.fn(y)


def group_norm(
    x: Tensor,
    num_groups: int,
    weight: Tensor,
    bias: Tensor,
    eps: float,
    epilogue: Callable[[Tensor, Tensor], Tensor] = _second_operand,
    extra: Tensor | None = None,
    in_place: bool = False,
) -> Tensor:
    """``epilogue(GroupNorm(x), extra)`` of ``x`` ``[M, C]`` (``normalization.py:156-196``):
    per (row, group) f32 mean and centered variance, ``(x - mean) * rsqrt(var +
    eps) * weight + bias``, the epilogue, one rounding. ``extra`` is an optional
    per-channel ``[C]`` operand of the epilogue."""
    if x.dim() != 2 or num_groups <= 0 or x.shape[1] % num_groups:
        raise ValueError(
            f"group_norm() expects [M, C] with C divisible by {num_groups} groups, "
            f"got {tuple(x.shape)}"
        )
    _check("group_norm", x)
    m, c = map(int, x.shape)
    extra_op, act, act_arg, program = _extra_op(epilogue)
    reads_extra = extra_op != native.EXTRA_NONE or act == native.EPI_PROGRAM
    if reads_extra and extra is None:
        extra = weight  # the reference's default extra operand (normalization.py:190-192)
    vecs = []
    for name, v in (("weight", weight), ("bias", bias), ("extra", extra if reads_extra else None)):
        if v is None:
            vecs.append(None)
            continue
        if v.numel() != c:
            raise ValueError(f"group_norm() {name} must have {c} elements, got {tuple(v.shape)}")
        vecs.append(v.reshape(-1).to(device=x.device, dtype=torch.float32).contiguous())
    x, y = _target(x, in_place)
    if m == 0 or c == 0:
        return y
    with on_device(x.device) as stream:
        native.call("hmx_group_norm_rows", native.dtype_code(x.dtype), x.data_ptr(),
                    native.ptr(vecs[0]), native.ptr(vecs[1]), native.ptr(vecs[2]), native.DTYPE_F32,
                    y.data_ptr(), m, num_groups, c // num_groups, float(eps), extra_op, act, act_arg,
                    native.program_arg(program), stream)
    return y


def layer_norm(x: Tensor, weight: Tensor, bias: Tensor, eps: float = 1e-5, in_place: bool = False) -> Tensor:
    """LayerNorm over the last dim of a 2-D ``x``: :func:`group_norm` with one group."""
    return group_norm(x, 1, weight, bias, eps, in_place=in_place)
