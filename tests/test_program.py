"""Epilogue programs on the host: tracing callables into the kernels'
elementwise programs (helion_mlir_utils/_program.py), checked on the CPU.

A program evaluated with torch (EpilogueProgram.__call__, one torch operation
per instruction) must give what the callable itself gives: that pins the
translation -- operand order of sub/div, scalar placement, pow
specialisations, register allocation across a DAG -- without a GPU. The GPU
tests then compare the kernels' interpretation of the same programs with the
oracle.
"""

from __future__ import annotations

import functools
import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import helion_mlir_utils as U
from helion_mlir_backend._compiler import native
from helion_mlir_utils._program import compile_epilogue


def _values() -> torch.Tensor:
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4096, generator=g) * 4
    special = torch.tensor([0.0, -0.0, 1.0, -1.0, 3.0, -3.0, 20.0, 25.0, -25.0, 88.0, -104.0,
                            float("inf"), float("-inf"), float("nan"), 1e-30, -1e-30])
    return torch.cat([x, special])


# (name, callable): every supported operation, as functions, methods,
# operators and modules, alone and composed.
EPILOGUES = [
    ("scale", lambda x: x * 3),
    ("rscale", lambda x: 3 * x),
    ("shift", lambda x: x + 0.5),
    ("sub", lambda x: x - 0.25),
    ("rsub", lambda x: 1.5 - x),
    ("div", lambda x: x / 7),
    ("rdiv", lambda x: 2 / x),
    ("neg", lambda x: -x),
    ("abs", torch.abs),
    ("pow2", lambda x: x ** 2),
    ("pow3", lambda x: x.pow(3)),
    ("pow_half", lambda x: torch.pow(x, 0.5)),
    ("pow_m1", lambda x: x ** -1),
    ("pow_m2", lambda x: x ** -2),
    ("pow_1_5", lambda x: x.abs() ** 1.5),
    ("silu_x2", lambda x: F.silu(x) * 2),
    ("x_sigmoid", lambda x: x * torch.sigmoid(x)),
    ("hardswish", F.hardswish),
    ("hardsigmoid", F.hardsigmoid),
    ("mish", F.mish),
    ("softplus", F.softplus),
    ("softplus_beta", functools.partial(F.softplus, beta=2.0, threshold=5.0)),
    ("elu", functools.partial(F.elu, alpha=0.7)),
    ("selu", F.selu),
    ("relu6", F.relu6),
    ("hardtanh", lambda x: F.hardtanh(x, -2.0, 2.5)),
    ("clamp", lambda x: x.clamp(min=-1.0, max=2.0)),
    ("clamp_min", lambda x: torch.clamp(x, min=0.5)),
    ("clip", lambda x: torch.clip(x, None, 1.0)),
    ("exp", torch.exp),
    ("log_abs", lambda x: torch.log(x.abs() + 1)),
    ("sqrt_abs", lambda x: x.abs().sqrt()),
    ("rsqrt", lambda x: torch.rsqrt(x * x + 1)),
    ("recip", torch.reciprocal),
    ("erf", torch.erf),
    ("sin_cos", lambda x: torch.sin(x) + torch.cos(x)),
    ("log1p_expm1", lambda x: torch.log1p(x.abs()) - torch.expm1(-x.abs())),
    ("rounding", lambda x: torch.floor(x) + torch.ceil(x) * 2 + torch.trunc(x) * 3 + torch.round(x) * 5),
    ("square", torch.square),
    ("max_min", lambda x: torch.maximum(x, x * 0.5) - torch.minimum(x, -x)),
    ("add_alpha", lambda x: torch.add(x, F.relu(x), alpha=0.5)),
    ("gelu_tanh_method", lambda x: F.gelu(x * 1.1, approximate="tanh").float()),
    ("modules", nn.Sequential(nn.GELU(), nn.Hardtanh(-2.0, 2.0))),
    ("module_leaky", nn.LeakyReLU(0.3)),
    ("deep", lambda x: (x * 2 + F.silu(x)) * torch.sigmoid(x * 3) - x / 4 + torch.tanh(x) * F.relu(x - 1)),
]


@pytest.mark.parametrize(("name", "fn"), EPILOGUES, ids=[e[0] for e in EPILOGUES])
def test_program_computes_what_the_callable_computes(name: str, fn) -> None:
    program = compile_epilogue(fn)
    assert program is not None and 1 <= len(program.code) <= native.PROGRAM_MAX
    x = _values()
    with torch.no_grad():
        want = fn(x.clone())
        got = program(x.clone())
    # The same torch operations in the same order: equal, NaN where NaN. A
    # rewrite that changes rounding (x - c as x + (-c), x / c) is exact too.
    assert torch.equal(torch.isnan(got), torch.isnan(want)), name
    finite = ~torch.isnan(want)
    torch.testing.assert_close(got[finite], want[finite], rtol=0, atol=0, msg=name)


def test_group_norm_programs_take_the_extra_operand() -> None:
    fn = lambda y, e: F.silu(y * e + 1) - e  # noqa: E731
    program = compile_epilogue(fn, 2)
    assert program.arity == 2
    y = _values()[:4096]
    e = torch.randn(4096)
    torch.testing.assert_close(program(y, e), fn(y, e), rtol=0, atol=0)
    # The default group-norm epilogue returns y: no program.
    assert compile_epilogue(lambda y, e: y, 2) is None
    with pytest.raises(ValueError, match="extra operand"):
        compile_epilogue(lambda y, e: e, 2)


def test_closure_scalars_are_read_when_traced() -> None:
    s = 2.0
    fn = lambda x: x * s  # noqa: E731
    assert compile_epilogue(fn).code[0].c0 == 2.0
    s = 3.0
    assert compile_epilogue(fn).code[0].c0 == 3.0


def test_registers_are_reused_as_values_die() -> None:
    # 15 instructions in a chain that keeps at most three values live.
    def chain(x):
        for i in range(5):
            x = torch.tanh(x) * (i + 1) + x
        return x

    program = compile_epilogue(chain)
    assert len(program.code) == 15
    assert max(max(i.dst, i.a, i.b) for i in program.code) < native.PROGRAM_REGS
    x = _values()
    torch.testing.assert_close(program(x), chain(x), rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize(
    ("fn", "message"),
    [
        (lambda x: x.sum(), "cannot fuse"),
        (lambda x: x * torch.ones(3), "only scalars are fusable"),
        (lambda x: x if x.sum() > 0 else -x, "tracing it failed"),
        (lambda x: x.to(torch.bfloat16), "rounds once"),
        (lambda x: torch.div(x, 2, rounding_mode="floor"), "rounding_mode"),
        (lambda x: 2 ** x, "scalar raised"),
        (lambda x: functools.reduce(lambda a, _: torch.tanh(a), range(17), x), "at most 16"),
    ],
)
def test_unfusable_epilogues_are_refused(fn, message: str) -> None:
    with pytest.raises(ValueError, match=message):
        compile_epilogue(fn)


def test_too_many_live_values_are_refused() -> None:
    def wide(x):
        parts = [x * (i + 1) for i in range(8)]
        return functools.reduce(torch.add, parts)

    with pytest.raises(ValueError, match="live"):
        compile_epilogue(wide)


def test_programs_pass_through_as_epilogues() -> None:
    program = U.compile_epilogue(lambda x: F.hardswish(x) + 1)
    code, arg, struct = U._gpu.epilogue_code(program)
    assert code == native.EPI_PROGRAM and struct is program.struct
    assert struct.count == 2 and struct.result == program.result
    # The structure the library reads holds the instructions as traced.
    assert [(struct.code[i].op, struct.code[i].dst) for i in range(2)] == [(i.op, i.dst) for i in program.code]
    assert math.isclose(struct.code[1].c0, 1.0)


def test_a_callable_is_traced_once() -> None:
    # Tracing takes longer than many GEMMs: the program of a callable object
    # is kept with it (as the reference keeps a bound kernel per epilogue
    # object), a new callable is traced anew.
    s = 2.0
    fn = lambda x: F.silu(x) * s  # noqa: E731
    first = U._gpu.epilogue_code(fn)
    s = 3.0
    again = U._gpu.epilogue_code(fn)
    assert again[2] is first[2] and first[2].code[1].c0 == 2.0
    other = U._gpu.epilogue_code(lambda x: F.silu(x) * s)
    assert other[2] is not first[2] and other[2].code[1].c0 == 3.0
    # The public compiler traces every time.
    assert compile_epilogue(fn).code[1].c0 == 3.0


def _relu_inplace_then_scale(x):
    F.relu(x, inplace=True)
    return x * 2


def _silu_inplace_plus_input(x):
    y = F.silu(x, inplace=True)
    return y + x


def _alias_then_leaky_inplace(x):
    y = x.float()  # an alias of x: the in-place op below writes it too
    F.leaky_relu(x, 0.1, inplace=True)
    return y - 1


def _hardtanh_inplace(x):
    F.hardtanh(x, -0.5, 0.5, inplace=True)
    return x


@pytest.mark.parametrize("fn", [_relu_inplace_then_scale, _silu_inplace_plus_input, _alias_then_leaky_inplace,
                                _hardtanh_inplace])
def test_inplace_activations_write_their_input(fn) -> None:
    # An in-place activation changes the value every later use reads; the
    # program must give what eager torch gives on a fresh copy.
    x = _values()
    program = compile_epilogue(fn)
    assert program is not None
    torch.testing.assert_close(program(x.clone()), fn(x.clone()), rtol=0, atol=0, equal_nan=True)


def test_discarded_results_cost_nothing() -> None:
    # A result nothing reads is dead code: the identity stays the identity,
    # and one in-place activation returned as its input is that activation.
    def discard(x):
        torch.relu(x)
        return x

    def relu_inplace(x):
        F.relu(x, inplace=True)
        return x

    assert compile_epilogue(discard) is None
    assert U._gpu.epilogue_code(discard)[0] == native.EPI_IDENTITY
    assert U._gpu.epilogue_code(relu_inplace)[0] == native.EPI_RELU
