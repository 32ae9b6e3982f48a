"""Shared host-side pieces of the gpu entry points: device checks, the launch
stream, dtype codes and epilogue resolution."""

from __future__ import annotations

import contextlib
import functools
from typing import Callable, Iterator, Optional, Tuple

import torch
import torch.nn.functional as F

from helion_mlir_backend._compiler import native

SUPPORTED_DTYPES = (torch.bfloat16, torch.float32)


def is_gpu(*tensors: torch.Tensor | None) -> bool:
    """Whether every given tensor is on a ROCm device (torch's "cuda")."""
    return all(t is None or t.device.type == "cuda" for t in tensors)


@contextlib.contextmanager
def on_device(device: torch.device) -> Iterator[int]:
    """Make ``device`` current and yield its current stream (``hipStream_t``)."""
    native.ensure_device(device)
    if device.index is None or device.index == torch.cuda.current_device():
        yield native.stream_of(device)
        return
    with torch.cuda.device(device):
        yield native.stream_of(device)


def identity_epilogue(x: torch.Tensor) -> torch.Tensor:
    return x


class Activation:
    """An epilogue the gpu kernels fuse by code, callable on a tensor like the
    torch function it names (so it serves every target): ``Activation("silu")``,
    ``Activation("leaky_relu", 0.2)``, ``Activation("gelu_tanh")``."""

    _CODES = {
        "identity": native.EPI_IDENTITY,
        "relu": native.EPI_RELU,
        "silu": native.EPI_SILU,
        "sigmoid": native.EPI_SIGMOID,
        "gelu": native.EPI_GELU,
        "gelu_tanh": native.EPI_GELU_TANH,
        "tanh": native.EPI_TANH,
        "leaky_relu": native.EPI_LEAKY_RELU,
    }

    def __init__(self, name: str, arg: float = 0.01) -> None:
        if name not in self._CODES:
            raise ValueError(f"unknown activation {name!r}; expected one of {tuple(self._CODES)}")
        self.name = name
        self.arg = float(arg)
        self.code = self._CODES[name]

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.name == "identity":
            return x
        if self.name == "gelu_tanh":
            return F.gelu(x, approximate="tanh")
        if self.name == "leaky_relu":
            return F.leaky_relu(x, self.arg)
        return getattr(F, self.name)(x) if self.name != "tanh" else torch.tanh(x)

    def __repr__(self) -> str:
        return f"Activation({self.name!r})" if self.name != "leaky_relu" else f"Activation('leaky_relu', {self.arg})"


_KNOWN: dict[object, tuple[int, float]] = {
    identity_epilogue: (native.EPI_IDENTITY, 0.0),
    torch.relu: (native.EPI_RELU, 0.0),
    F.relu: (native.EPI_RELU, 0.0),
    F.silu: (native.EPI_SILU, 0.0),
    torch.sigmoid: (native.EPI_SIGMOID, 0.0),
    F.sigmoid: (native.EPI_SIGMOID, 0.0),
    F.gelu: (native.EPI_GELU, 0.0),
    torch.tanh: (native.EPI_TANH, 0.0),
    F.tanh: (native.EPI_TANH, 0.0),
    F.leaky_relu: (native.EPI_LEAKY_RELU, 0.01),
}


def register_epilogue(fn: Callable[[torch.Tensor], torch.Tensor], name: str, arg: float = 0.01) -> None:
    """Let the gpu kernels fuse ``fn`` as the activation ``name`` (a callable
    the caller guarantees computes it, e.g. a module's own alias)."""
    act = Activation(name, arg)
    _KNOWN[fn] = (act.code, act.arg)


# What the kernels fuse for an epilogue: (activation code, its argument, the
# epilogue program for code EPI_PROGRAM, else None).
Epilogue = Tuple[int, float, Optional[native.Program]]
IDENTITY: Epilogue = (native.EPI_IDENTITY, 0.0, None)

# Single-operation programs that are one of the named activations: those
# keep the kernels' register epilogues.
_NAMED_PROGRAMS = {
    native.OP["relu"]: native.EPI_RELU,
    native.OP["silu"]: native.EPI_SILU,
    native.OP["sigmoid"]: native.EPI_SIGMOID,
    native.OP["gelu"]: native.EPI_GELU,
    native.OP["gelu_tanh"]: native.EPI_GELU_TANH,
    native.OP["tanh"]: native.EPI_TANH,
    native.OP["leaky_relu"]: native.EPI_LEAKY_RELU,
}


def epilogue_code(epilogue: Callable[[torch.Tensor], torch.Tensor]) -> Epilogue:
    """What the kernels fuse for ``epilogue``: one of the named activations,
    or any other elementwise callable traced into an epilogue program
    (:func:`compile_epilogue`).

    Raises ``ValueError`` for a callable they cannot fuse: an epilogue is
    never run as a separate eager pass behind the caller's back."""
    from ._program import traced_epilogue

    if isinstance(epilogue, Activation):
        return epilogue.code, epilogue.arg, None
    if epilogue in _KNOWN:
        return (*_KNOWN[epilogue], None)
    if isinstance(epilogue, functools.partial) and not epilogue.args:
        kwargs = epilogue.keywords
        if epilogue.func is F.leaky_relu and set(kwargs) <= {"negative_slope"}:
            return native.EPI_LEAKY_RELU, float(kwargs.get("negative_slope", 0.01)), None
        if epilogue.func is F.gelu and set(kwargs) <= {"approximate"}:
            approx = kwargs.get("approximate", "none")
            return (native.EPI_GELU_TANH if approx == "tanh" else native.EPI_GELU), 0.0, None
    if epilogue is identity_epilogue or getattr(epilogue, "__name__", None) == "identity_epilogue":
        return IDENTITY
    program = traced_epilogue(epilogue, 1)
    if program is None:
        return IDENTITY
    if (len(program.code) == 1 and program.code[0].a == 0 and program.result == program.code[0].dst
            and program.code[0].op in _NAMED_PROGRAMS):
        ins = program.code[0]
        return _NAMED_PROGRAMS[ins.op], ins.c0, None
    return native.EPI_PROGRAM, 0.0, program.struct
