"""Epilogue programs: arbitrary elementwise epilogues on the gpu target.

The reference applies any callable to the f32 accumulator inside its Helion
kernels (``helion_mlir_utils/matmul.py:321-327``; group_norm's
``epilogue(y, extra)``, ``normalization.py:121``), because Helion traces the
callable into the kernel. The gfx950 kernels are compiled ahead of time, so
here a callable is traced once with ``torch.fx`` into a straight-line program
of elementwise f32 operations (``hmx_program`` in ``include/hmx.h``) that the
kernels interpret on each value before the single rounding:
``compile_epilogue(lambda x: F.silu(x) * 2)``, ``lambda x: x * 3``,
``F.hardswish``, ``nn.Sequential(nn.GELU(), nn.Hardtanh(-2, 2))`` ...

A callable is accepted when every operation it applies is one of the
elementwise torch operations listed in ``_FUNCTIONS`` / ``_METHODS`` on its
input(s) and Python scalars; anything else (a captured tensor, a reduction,
data-dependent control flow, more than ``PROGRAM_MAX`` instructions or
``PROGRAM_REGS`` live values) raises ``ValueError`` -- never a silent eager
pass. The trace is taken at call time, so scalars a closure captures are read
then.
"""

from __future__ import annotations

import math
import operator
import weakref
from typing import Callable, NamedTuple

import torch
import torch.fx as fx
import torch.nn.functional as F

from helion_mlir_backend._compiler import native

__all__ = ["EpilogueProgram", "compile_epilogue", "traced_epilogue"]

_OP = native.OP


class Instr(NamedTuple):
    op: int
    dst: int
    a: int
    b: int = 0
    c0: float = 0.0
    c1: float = 0.0


_SELU_ALPHA = 1.6732632423543772848170429916717
_SELU_SCALE = 1.0507009873554804934193349852946


def _f32(v: float) -> float:
    """A Python scalar as the f32 value torch uses with an f32 tensor."""
    return float(torch.tensor(float(v), dtype=torch.float32))


class EpilogueProgram:
    """A traced elementwise epilogue: ``arity`` inputs (the value, and for
    group_norm the extra operand) in registers 0 and 1, ``code`` over
    ``PROGRAM_REGS`` f32 registers, the result in register ``result``.

    Calling it evaluates the same operations with torch on any tensors (the
    program's meaning, on every target); passing it as an epilogue hands the
    program to the kernels unchanged."""

    def __init__(self, code: list[Instr], result: int, arity: int, source: object = None) -> None:
        if not 1 <= len(code) <= native.PROGRAM_MAX:
            raise ValueError(f"an epilogue program holds 1..{native.PROGRAM_MAX} instructions, got {len(code)}")
        self.code = list(code)
        self.result = result
        self.arity = arity
        self.source = source
        prog = native.Program()
        prog.count = len(code)
        prog.result = result
        for i, ins in enumerate(code):
            prog.code[i] = native.Instr(ins.op, ins.dst, ins.a, ins.b, ins.c0, ins.c1)
        self.struct = prog

    def __repr__(self) -> str:
        names = native.OPCODES
        body = "; ".join(f"r{i.dst} = {names[i.op]}(r{i.a}, r{i.b}, {i.c0:g}, {i.c1:g})" for i in self.code)
        return f"EpilogueProgram([{body}] -> r{self.result})"

    def __call__(self, *values: torch.Tensor) -> torch.Tensor:
        if len(values) != self.arity:
            raise TypeError(f"this epilogue program takes {self.arity} operand(s), got {len(values)}")
        first = values[0].float()
        regs: list[torch.Tensor] = [torch.zeros_like(first) for _ in range(native.PROGRAM_REGS)]
        regs[0] = first
        if self.arity > 1:
            regs[1] = values[1].float().expand_as(first) if values[1].dim() else values[1].float()
        for ins in self.code:
            regs[ins.dst] = _evaluate(ins, regs[ins.a], regs[ins.b])
        return regs[self.result]


def _evaluate(ins: Instr, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """One instruction with torch's f32 operations (the kernels' formulas)."""
    name = native.OPCODES[ins.op]
    c0, c1 = ins.c0, ins.c1
    unary = {
        "copy": lambda: a.clone(), "neg": lambda: -a, "abs": lambda: a.abs(), "relu": lambda: torch.relu(a),
        "sigmoid": lambda: torch.sigmoid(a), "tanh": lambda: torch.tanh(a), "silu": lambda: F.silu(a),
        "gelu": lambda: F.gelu(a), "gelu_tanh": lambda: F.gelu(a, approximate="tanh"),
        "exp": lambda: a.exp(), "log": lambda: a.log(), "sqrt": lambda: a.sqrt(), "rsqrt": lambda: a.rsqrt(),
        "recip": lambda: a.reciprocal(), "erf": lambda: torch.erf(a), "sin": lambda: a.sin(),
        "cos": lambda: a.cos(), "log1p": lambda: a.log1p(), "expm1": lambda: a.expm1(),
        "floor": lambda: a.floor(), "ceil": lambda: a.ceil(), "trunc": lambda: a.trunc(),
        "round": lambda: a.round(), "softplus": lambda: F.softplus(a, c0, c1), "mish": lambda: F.mish(a),
        "hardswish": lambda: F.hardswish(a), "hardsigmoid": lambda: F.hardsigmoid(a),
        "elu": lambda: _elu(a, c0, c1),
        "leaky_relu": lambda: F.leaky_relu(a, c0), "clamp": lambda: a.clamp(c0, c1),
        "add_c": lambda: a + c0, "mul_c": lambda: a * c0, "div_c": lambda: a / c0,
        "rsub_c": lambda: c0 - a, "rdiv_c": lambda: c0 / a, "pow_c": lambda: a.pow(c0),
        "add": lambda: a + b, "sub": lambda: a - b, "mul": lambda: a * b, "div": lambda: a / b,
        "max": lambda: torch.maximum(a, b), "min": lambda: torch.minimum(a, b), "pow": lambda: a.pow(b),
    }
    return unary[name]()


def _elu(a: torch.Tensor, alpha: float, scale: float) -> torch.Tensor:
    if scale == 1.0:
        return F.elu(a, alpha)
    if (alpha, scale) == (_f32(_SELU_ALPHA), _f32(_SELU_SCALE)):
        return F.selu(a)
    return F.elu(a, alpha) * scale


# ---------------------------------------------------------------------------
# Tracing.


class _Tracer(fx.Tracer):
    """Traces through every module (activation modules become the functional
    calls their forward makes), including modules the root does not own."""

    def is_leaf_module(self, m: torch.nn.Module, module_qualified_name: str) -> bool:
        return False

    def path_of_module(self, mod: torch.nn.Module) -> str:
        try:
            return super().path_of_module(mod)
        except NameError:
            return ""


def _trace(fn: Callable[..., torch.Tensor], arity: int) -> fx.Graph:
    if arity == 1:
        def root(x):
            return fn(x)
    else:
        def root(y, extra):
            return fn(y, extra)
    return _Tracer().trace(root)


class _Emitter:
    """Builds the instruction list, allocating registers as values die."""

    def __init__(self, arity: int, last_use: dict[fx.Node, int]) -> None:
        self.code: list[Instr] = []
        self.reg: dict[fx.Node, int] = {}
        self.free = [r for r in range(native.PROGRAM_REGS - 1, arity - 1, -1)]
        self.last_use = last_use

    def take(self) -> int:
        if not self.free:
            raise ValueError(f"the epilogue keeps more than {native.PROGRAM_REGS} values live")
        return self.free.pop()

    def release_dead(self, inputs: list[fx.Node], index: int) -> None:
        for arg in set(inputs):
            if self.last_use.get(arg) == index and arg in self.reg:
                self.free.append(self.reg.pop(arg))

    def emit(self, op: str, dst: int, a: int, b: int = 0, c0: float = 0.0, c1: float = 0.0) -> None:
        self.code.append(Instr(_OP[op], dst, a, b, _f32(c0), _f32(c1)))


def _scalar(v: object) -> bool:
    return isinstance(v, (int, float, bool)) and not isinstance(v, torch.Tensor)


def _float_args(name: str, values: list[object]) -> list[float]:
    out = []
    for v in values:
        if not _scalar(v):
            raise ValueError(f"the gpu epilogue needs a Python scalar for {name}'s parameter, got {v!r}")
        out.append(float(v))
    return out


def _bind(name: str, args: tuple, kwargs: dict, params: tuple[str, ...], defaults: dict[str, object]) -> list:
    """Positional + keyword arguments of a call as a list in ``params`` order."""
    if len(args) > len(params):
        raise ValueError(f"{name}: too many arguments for the gpu epilogue")
    bound = dict(zip(params, args))
    for key, value in kwargs.items():
        if key == "inplace" or key == "out" and value is None:
            continue
        if key not in params or key in bound:
            raise ValueError(f"{name}: argument {key!r} is not supported in a gpu epilogue")
        bound[key] = value
    missing = [p for p in params if p not in bound and p not in defaults]
    if missing:
        raise ValueError(f"{name}: missing {missing}")
    return [bound.get(p, defaults.get(p)) for p in params]


# Unary operations: name -> (params after the input, defaults, emitter of
# (emitter, dst, a, *params)).
def _unary(op: str) -> Callable:
    return lambda e, dst, a: e.emit(op, dst, a)


def _pow_const(e: _Emitter, dst: int, a: int, c: float) -> None:
    # torch's f32 pow by a scalar: x*x, x*x*x, sqrt, rsqrt, 1/x, 1/(x*x) for
    # those exponents, the general power otherwise.
    if c == 1.0:
        e.emit("copy", dst, a)
    elif c == 2.0:
        e.emit("mul", dst, a, a)
    elif c == 3.0:
        e.emit("mul", dst, a, a)
        e.emit("mul", dst, dst, a)
    elif c == 0.5:
        e.emit("sqrt", dst, a)
    elif c == -0.5:
        e.emit("rsqrt", dst, a)
    elif c == -1.0:
        e.emit("recip", dst, a)
    elif c == -2.0:
        e.emit("mul", dst, a, a)
        e.emit("recip", dst, dst)
    else:
        e.emit("pow_c", dst, a, 0, c)


def _clamp(e: _Emitter, dst: int, a: int, lo: object, hi: object) -> None:
    lo_f = -math.inf if lo is None else _float_args("clamp", [lo])[0]
    hi_f = math.inf if hi is None else _float_args("clamp", [hi])[0]
    e.emit("clamp", dst, a, 0, lo_f, hi_f)


_UNARY: dict[str, tuple[tuple[str, ...], dict[str, object], Callable]] = {
    "relu": ((), {}, _unary("relu")),
    "sigmoid": ((), {}, _unary("sigmoid")),
    "tanh": ((), {}, _unary("tanh")),
    "silu": ((), {}, _unary("silu")),
    "neg": ((), {}, _unary("neg")),
    "abs": ((), {}, _unary("abs")),
    "exp": ((), {}, _unary("exp")),
    "log": ((), {}, _unary("log")),
    "sqrt": ((), {}, _unary("sqrt")),
    "rsqrt": ((), {}, _unary("rsqrt")),
    "reciprocal": ((), {}, _unary("recip")),
    "erf": ((), {}, _unary("erf")),
    "sin": ((), {}, _unary("sin")),
    "cos": ((), {}, _unary("cos")),
    "log1p": ((), {}, _unary("log1p")),
    "expm1": ((), {}, _unary("expm1")),
    "floor": ((), {}, _unary("floor")),
    "ceil": ((), {}, _unary("ceil")),
    "trunc": ((), {}, _unary("trunc")),
    "mish": ((), {}, _unary("mish")),
    "hardswish": ((), {}, _unary("hardswish")),
    "hardsigmoid": ((), {}, _unary("hardsigmoid")),
    "square": ((), {}, lambda e, dst, a: e.emit("mul", dst, a, a)),
    "identity": ((), {}, lambda e, dst, a: e.emit("copy", dst, a)),
    "round": (("decimals",), {"decimals": 0}, lambda e, dst, a, d: _round(e, dst, a, d)),
    "gelu": (("approximate",), {"approximate": "none"}, lambda e, dst, a, approx: _gelu(e, dst, a, approx)),
    "softplus": (("beta", "threshold"), {"beta": 1.0, "threshold": 20.0},
                 lambda e, dst, a, beta, thr: e.emit("softplus", dst, a, 0, *_float_args("softplus", [beta, thr]))),
    "elu": (("alpha",), {"alpha": 1.0},
            lambda e, dst, a, alpha: e.emit("elu", dst, a, 0, _float_args("elu", [alpha])[0], 1.0)),
    "selu": ((), {}, lambda e, dst, a: e.emit("elu", dst, a, 0, _SELU_ALPHA, _SELU_SCALE)),
    "leaky_relu": (("negative_slope",), {"negative_slope": 0.01},
                   lambda e, dst, a, s: e.emit("leaky_relu", dst, a, 0, _float_args("leaky_relu", [s])[0])),
    "relu6": ((), {}, lambda e, dst, a: e.emit("clamp", dst, a, 0, 0.0, 6.0)),
    "hardtanh": (("min_val", "max_val"), {"min_val": -1.0, "max_val": 1.0},
                 lambda e, dst, a, lo, hi: _clamp(e, dst, a, lo, hi)),
    "clamp": (("min", "max"), {"min": None, "max": None}, lambda e, dst, a, lo, hi: _clamp(e, dst, a, lo, hi)),
    "clamp_min": (("min",), {}, lambda e, dst, a, lo: _clamp(e, dst, a, lo, None)),
    "clamp_max": (("max",), {}, lambda e, dst, a, hi: _clamp(e, dst, a, None, hi)),
}
_UNARY["clip"] = _UNARY["clamp"]


def _round(e: _Emitter, dst: int, a: int, decimals: object) -> None:
    if decimals != 0:
        raise ValueError("round(decimals != 0) is not supported in a gpu epilogue")
    e.emit("round", dst, a)


def _gelu(e: _Emitter, dst: int, a: int, approximate: object) -> None:
    if approximate not in ("none", "tanh"):
        raise ValueError(f"gelu(approximate={approximate!r}) is not supported")
    e.emit("gelu_tanh" if approximate == "tanh" else "gelu", dst, a)


# Binary operations: register/register opcode, and the forms with a scalar.
_BINARY = {"add", "sub", "mul", "div", "pow", "maximum", "minimum"}


def _binary(e: _Emitter, name: str, dst: int, x: object, y: object, reg: Callable[[object], int | None]) -> None:
    rx, ry = reg(x), reg(y)
    if rx is not None and ry is not None:
        op = {"maximum": "max", "minimum": "min"}.get(name, name)
        e.emit(op, dst, rx, ry)
        return
    if rx is None and ry is None:
        raise ValueError(f"{name} of two constants in a gpu epilogue")
    if name in ("maximum", "minimum"):
        raise ValueError(f"torch.{name} takes two tensors")
    if rx is not None:
        (c,) = _float_args(name, [y])
        if name == "add":
            e.emit("add_c", dst, rx, 0, c)
        elif name == "sub":
            e.emit("add_c", dst, rx, 0, -c)
        elif name == "mul":
            e.emit("mul_c", dst, rx, 0, c)
        elif name == "div":
            e.emit("div_c", dst, rx, 0, c)
        else:
            _pow_const(e, dst, rx, c)
    else:
        (c,) = _float_args(name, [x])
        if name == "add":
            e.emit("add_c", dst, ry, 0, c)
        elif name == "sub":
            e.emit("rsub_c", dst, ry, 0, c)
        elif name == "mul":
            e.emit("mul_c", dst, ry, 0, c)
        elif name == "div":
            e.emit("rdiv_c", dst, ry, 0, c)
        else:
            raise ValueError("a scalar raised to a tensor power is not supported in a gpu epilogue")


# Call targets: function object -> operation name.
_FUNCTIONS: dict[object, str] = {
    operator.add: "add", torch.add: "add",
    operator.sub: "sub", torch.sub: "sub", torch.subtract: "sub",
    operator.mul: "mul", torch.mul: "mul", torch.multiply: "mul",
    operator.truediv: "div", torch.div: "div", torch.divide: "div", torch.true_divide: "div",
    operator.pow: "pow", torch.pow: "pow",
    torch.maximum: "maximum", torch.minimum: "minimum",
    operator.neg: "neg", torch.neg: "neg", torch.negative: "neg",
    operator.pos: "identity", operator.abs: "abs", torch.abs: "abs", torch.absolute: "abs",
    torch.relu: "relu", F.relu: "relu",
    torch.sigmoid: "sigmoid", F.sigmoid: "sigmoid", torch.special.expit: "sigmoid",
    torch.tanh: "tanh", F.tanh: "tanh",
    F.silu: "silu", F.gelu: "gelu", F.mish: "mish", F.hardswish: "hardswish", F.hardsigmoid: "hardsigmoid",
    F.softplus: "softplus", F.elu: "elu", F.selu: "selu", F.leaky_relu: "leaky_relu",
    F.relu6: "relu6", F.hardtanh: "hardtanh",
    torch.exp: "exp", torch.log: "log", torch.sqrt: "sqrt", torch.rsqrt: "rsqrt",
    torch.reciprocal: "reciprocal", torch.erf: "erf", torch.special.erf: "erf",
    torch.sin: "sin", torch.cos: "cos", torch.log1p: "log1p", torch.special.log1p: "log1p",
    torch.expm1: "expm1", torch.special.expm1: "expm1",
    torch.floor: "floor", torch.ceil: "ceil", torch.trunc: "trunc", torch.round: "round",
    torch.square: "square", torch.clamp: "clamp", torch.clip: "clip",
    torch.clamp_min: "clamp_min", torch.clamp_max: "clamp_max",
}
# Tensor methods: method name -> operation name.
_METHODS = {
    **{name: name for name in ("add", "sub", "mul", "div", "pow", "maximum", "minimum", "neg", "abs", "relu",
                               "sigmoid", "tanh", "exp", "log", "sqrt", "rsqrt", "reciprocal", "erf", "sin",
                               "cos", "log1p", "expm1", "floor", "ceil", "trunc", "round", "square", "clamp",
                               "clip", "clamp_min", "clamp_max")},
    "subtract": "sub", "multiply": "mul", "divide": "div", "true_divide": "div", "negative": "neg",
    "absolute": "abs", "float": "identity", "contiguous": "identity",
}


def _lower_call(e: _Emitter, node: fx.Node, name: str, dst: int, reg: Callable[[object], int | None]) -> None:
    args, kwargs = tuple(node.args), dict(node.kwargs)
    if name in _BINARY:
        if name == "div" and kwargs.pop("rounding_mode", None) is not None:
            raise ValueError("div(rounding_mode=...) is not supported in a gpu epilogue")
        alpha = kwargs.pop("alpha", 1)
        params = ("input", "exponent") if name == "pow" else ("input", "other")
        x, y = _bind(name, args, kwargs, params, {})
        if alpha != 1:
            if name not in ("add", "sub"):
                raise ValueError(f"{name}: alpha is not supported")
            ry = reg(y)
            if ry is None:
                y = float(y) * float(alpha)
            else:
                e.emit("mul_c", dst, ry, 0, float(alpha))
                rx = reg(x)
                if rx is None:
                    raise ValueError(f"{name} with alpha and a scalar input")
                e.emit(name, dst, rx, dst)
                return
        _binary(e, name, dst, x, y, reg)
        return
    params, defaults, emitter = _UNARY[name]
    if name == "identity":
        args = args[:1]
        kwargs = {}
    bound = _bind(name, args, kwargs, ("input",) + params, defaults)
    a = reg(bound[0])
    if a is None:
        raise ValueError(f"{name} of a constant in a gpu epilogue")
    emitter(e, dst, a, *bound[1:])


def _op_name(node: fx.Node) -> str:
    if node.op == "call_function":
        name = _FUNCTIONS.get(node.target)
    elif node.op == "call_method":
        name = _METHODS.get(node.target)
        if node.target == "to":
            dtypes = [v for v in list(node.args[1:]) + list(node.kwargs.values()) if isinstance(v, torch.dtype)]
            if all(d == torch.float32 for d in dtypes):
                return "identity"
            raise ValueError("an epilogue rounds once, to the output dtype: .to() another dtype is not fused")
    else:
        name = None
    if name is None:
        raise ValueError(f"the gpu target cannot fuse {node.op} {node.target!r} in an epilogue")
    return name


# Programs traced so far, by callable object and arity. Tracing (torch.fx)
# takes hundreds of microseconds, more than many GEMMs; the reference likewise
# binds an epilogue once and keeps the bound kernel in an LRU keyed by the
# epilogue object (helion_mlir_utils/matmul.py:487-489). Entries go with the
# callable; a full table is cleared.
_TRACED: "weakref.WeakKeyDictionary[Callable[..., torch.Tensor], dict[int, EpilogueProgram | None]]" = (
    weakref.WeakKeyDictionary()
)
_TRACED_MAX = 256


def traced_epilogue(fn: Callable[..., torch.Tensor], arity: int = 1) -> EpilogueProgram | None:
    """:func:`compile_epilogue`, traced once per callable object: later calls
    with the same object reuse its program (a closure's captured scalars are
    read when it is first traced; pass a new callable to change them).
    Callables that cannot be weakly referenced are traced every time."""
    try:
        known = _TRACED.get(fn)
    except TypeError:
        return compile_epilogue(fn, arity)
    if known is not None and arity in known:
        return known[arity]
    program = compile_epilogue(fn, arity)
    if len(_TRACED) >= _TRACED_MAX:
        _TRACED.clear()
    try:
        _TRACED.setdefault(fn, {})[arity] = program
    except TypeError:
        pass
    return program


def compile_epilogue(fn: Callable[..., torch.Tensor], arity: int = 1) -> EpilogueProgram | None:
    """Trace ``fn`` (of ``arity`` tensors: the value, and for group_norm the
    extra operand) into an :class:`EpilogueProgram`; ``None`` when it returns
    its first input unchanged. Raises ``ValueError`` if it is not fusable."""
    if isinstance(fn, EpilogueProgram):
        if fn.arity != arity:
            raise ValueError(f"the epilogue program takes {fn.arity} operand(s), this epilogue {arity}")
        return fn
    try:
        graph = _trace(fn, arity)
    except Exception as exc:  # tracing runs user code: any failure means "not fusable"
        raise ValueError(f"the gpu target cannot fuse the epilogue {fn!r}: tracing it failed ({exc})") from exc
    nodes = list(graph.nodes)
    # Operations that return their input (.float(), .contiguous(), +x) are
    # aliases: uses of them are uses of the value they alias.
    alias: dict[fx.Node, fx.Node] = {}
    names: dict[fx.Node, str] = {}
    for node in nodes:
        if node.op in ("call_function", "call_method"):
            names[node] = _op_name(node)
            if names[node] == "identity" and node.args and isinstance(node.args[0], fx.Node):
                alias[node] = alias.get(node.args[0], node.args[0])
        elif node.op == "get_attr":
            raise ValueError(f"the gpu epilogue reads the tensor {node.target!r}: only scalars are fusable")

    def source(v: object) -> object:
        return alias.get(v, v) if isinstance(v, fx.Node) else v

    # In-place activations (``F.relu(x, inplace=True)`` and the like) write
    # their input: every later use of that value, or of an alias of it, reads
    # the activation's result. Rewrite those uses to the activation's node,
    # then recompute the aliases.
    rewritten = False
    for i, node in enumerate(nodes):
        if node.op not in ("call_function", "call_method") or node.kwargs.get("inplace") is not True:
            continue
        if not node.args or not isinstance(node.args[0], fx.Node):
            raise ValueError(f"the gpu epilogue cannot fuse in-place {node.target!r} of a constant")
        written = source(node.args[0])
        for later in nodes[i + 1:]:
            for arg in list(later.all_input_nodes):
                if source(arg) is written:
                    later.replace_input_with(arg, node)
        rewritten = True
    # Operations whose result nothing reads (a discarded activation) are dead:
    # dropped, so they cost no instruction.
    changed = True
    while changed:
        changed = False
        for node in reversed(list(graph.nodes)):
            if node.op in ("call_function", "call_method") and not node.users:
                graph.erase_node(node)
                names.pop(node, None)
                changed = rewritten = True
    if rewritten:
        nodes = list(graph.nodes)
        alias.clear()
        for node in nodes:
            if names.get(node) == "identity" and node.args and isinstance(node.args[0], fx.Node):
                alias[node] = alias.get(node.args[0], node.args[0])

    last_use: dict[fx.Node, int] = {}
    for i, node in enumerate(nodes):
        for arg in node.all_input_nodes:
            last_use[source(arg)] = i
    e = _Emitter(arity, last_use)
    placeholders = [n for n in nodes if n.op == "placeholder"]
    for r, node in enumerate(placeholders):
        e.reg[node] = r

    def reg(v: object) -> int | None:
        if isinstance(v, fx.Node):
            return e.reg[source(v)]
        if _scalar(v):
            return None
        raise ValueError(f"the gpu epilogue reads {v!r}: only its inputs and Python scalars are fusable")

    result = None
    for i, node in enumerate(nodes):
        if node.op == "placeholder" or node in alias:
            continue
        if node.op == "output":
            out = node.args[0]
            if not isinstance(out, fx.Node):
                raise ValueError(f"the epilogue must return one tensor, got {out!r}")
            result = e.reg[source(out)]
            break
        # dst is taken while the inputs still hold their registers (lowerings
        # of several instructions write dst before reading the inputs again);
        # inputs used for the last time are freed after.
        dst = e.take()
        _lower_call(e, node, names[node], dst, reg)
        e.release_dead([source(a) for a in node.all_input_nodes], i)
        e.reg[node] = dst
    if result is None:
        raise ValueError("the epilogue returned nothing")
    if not e.code:
        if result != 0:
            raise ValueError("the epilogue returns its extra operand, not the value")
        return None
    if len(e.code) > native.PROGRAM_MAX:
        raise ValueError(f"the epilogue needs {len(e.code)} instructions; at most {native.PROGRAM_MAX} fuse")
    return EpilogueProgram(e.code, result, arity, fn)
