"""Parity of arbitrary elementwise epilogues on the GPU: callables traced into
epilogue programs (helion_mlir_utils/_program.py) and the named activations,
on every GEMM kernel family -- the direct-to-LDS kernels run them fused in
their LDS-staged epilogue; the register-staged bf16 and f32 kernels, split-K
and the skinny shapes leave them to the split-K reduction -- and on
group_norm, row_sum and row_dot.

The oracle applies the same callable with torch to its f32 values, as the
reference applies ``epilogue(acc)`` to its f32 accumulator
(helion_mlir_utils/matmul.py:321-327) and ``epilogue(y, extra)`` in group_norm
(normalization.py:121). Tolerances: bf16-in / f32-accumulate rtol 1e-2 plus an
atol scaled by sqrt(K), times the epilogues' largest slope (3); f32 rtol 1e-4.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import helion_mlir_utils as U
from helion_mlir_backend._compiler import native
from oracle import restate as R
from tests.helpers import assert_close, bf16_gemm_atol, tensor, to_np

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(23)

EPILOGUES = {
    "scale3": lambda x: x * 3,
    "hardswish": F.hardswish,
    "mish": F.mish,
    "silu_mix": lambda x: F.silu(x) * 2 - x / 4,
    "softplus": lambda x: F.softplus(x, beta=2.0, threshold=3.0),
    "selu": F.selu,
    "clamp": lambda x: torch.clamp(x, -0.5, 0.5),
    "gelu_named": F.gelu,
    "sigmoid_named": torch.sigmoid,
    "module": nn.Sequential(nn.Hardtanh(-2.0, 2.0), nn.ELU(0.5)),
}


def _operands(m, n, k, trans_a, trans_b, dtype, device):
    a = tensor(RNG.normal(0, 1, (k, m) if trans_a else (m, k)).astype(np.float32), dtype, device)
    b = tensor(RNG.normal(0, 1, (n, k) if trans_b else (k, n)).astype(np.float32), dtype, device)
    return a, b


def _check(got, ref, k, a, b, out):
    if out == "f32":
        assert_close(got, ref, 1e-4, 3e-5 * np.sqrt(k))
    else:
        assert_close(got, ref, 1e-2, 3 * bf16_gemm_atol(k, a, b))


# Shapes that reach each kernel family (planned for the device's CUs):
# (m, n, k, trans_a, trans_b, dtype).
SHAPES = {
    "dma_256": (4096, 4096, 128, False, False, "bf16"),   # 256 x 256 tiles, eight waves
    "dma_256_nk": (4096, 4096, 128, False, True, "bf16"),  # B [N, K]
    "dma_k32": (4096, 4096, 96, False, False, "bf16"),    # 32-wide K stages
    "dma_ragged": (4000, 4100, 128, False, True, "bf16"),  # ragged M and N
    "dma_trans_a": (4096, 4096, 128, True, False, "bf16"),
    "dma_128": (512, 512, 256, False, False, "bf16"),     # 128 x 128 tiles
    "bf16_general": (300, 200, 100, False, False, "bf16"),  # K not whole stages: reduction finishes
    "split_k": (256, 256, 8192, False, False, "bf16"),    # split-K: reduction finishes
    "skinny_shape": (32, 1024, 256, False, True, "bf16"),  # never the skinny kernel with a program
    "f32": (300, 200, 130, False, False, "f32"),
    "f32_split": (512, 512, 512, False, False, "f32"),
}


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("epi", ["scale3", "hardswish", "silu_mix", "gelu_named", "module"])
def test_matmul_epilogues_on_every_kernel(gpu_device, shape: str, epi: str) -> None:
    m, n, k, ta, tb, dtype = SHAPES[shape]
    fn = EPILOGUES[epi]
    a, b = _operands(m, n, k, ta, tb, dtype, gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), dtype, gpu_device)
    got = to_np(U.matmul(a, b, trans_a=ta, trans_b=tb, bias=bias, epilogue=fn))
    ref = R.matmul(to_np(a), to_np(b), ta, tb, to_np(bias), act=fn, out=dtype)
    _check(got, ref, k, to_np(a), to_np(b), dtype)


@pytest.mark.parametrize("epi", list(EPILOGUES))
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_each_epilogue_with_scale_shift_and_f32_output(gpu_device, epi: str, out: str) -> None:
    m, n, k = 4096, 4096, 64
    fn = EPILOGUES[epi]
    a, b = _operands(m, n, k, False, True, "bf16", gpu_device)
    scale = torch.from_numpy(RNG.uniform(0.5, 1.5, n).astype(np.float32)).to(gpu_device)
    shift = torch.from_numpy(RNG.normal(0, 0.5, n).astype(np.float32)).to(gpu_device)
    got = to_np(U.matmul(a, b, trans_b=True, epilogue=fn, scale=scale, shift=shift,
                         out_dtype=torch.float32 if out == "f32" else None))
    ref = R.matmul(to_np(a), to_np(b), False, True, None, to_np(scale), to_np(shift), act=fn, out=out)
    if out == "f32":
        # bf16 operands, f32 accumulation in different orders: the tolerance
        # of the products themselves, not of f32 operands.
        assert_close(got, ref, 1e-4, 2 * 3 * bf16_gemm_atol(k, to_np(a), to_np(b)))
    else:
        _check(got, ref, k, to_np(a), to_np(b), out)


def test_special_values_through_a_program(gpu_device) -> None:
    # NaN / inf accumulators through max/min/clamp-based programs: NaN stays
    # NaN (torch.clamp, torch.maximum), infinities saturate as torch's do.
    m, n, k = 256, 256, 64
    a = np.zeros((m, k), np.float32)
    b = np.zeros((k, n), np.float32)
    a[:, 0] = np.linspace(-3, 3, m)
    b[0, :] = 1.0
    a[0, 1], b[1, 0] = np.inf, 1.0   # C[0, 0] = +inf
    a[1, 1], b[1, 1] = np.nan, 1.0   # C[1, 1] = NaN
    a[2, 2], b[2, 2] = -np.inf, 1.0  # C[2, 2] = -inf
    fn = lambda x: torch.maximum(F.hardswish(x), x * 0.5).clamp(-1.0, 2.0)  # noqa: E731
    for dtype in ("bf16", "f32"):
        ta, tb = tensor(a, dtype, gpu_device), tensor(b, dtype, gpu_device)
        got = to_np(U.matmul(ta, tb, epilogue=fn))
        ref = R.matmul(to_np(ta), to_np(tb), act=fn, out=dtype)
        assert_close(got, ref, 1e-2 if dtype == "bf16" else 1e-5, 1e-6)


def test_prepacked_and_linear_take_programs(gpu_device) -> None:
    m, n, k = 512, 768, 256
    fn = EPILOGUES["silu_mix"]
    a, w = _operands(m, n, k, False, True, "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    ref = R.matmul(to_np(a), to_np(w), False, True, to_np(bias), act=fn, out="bf16")
    for panel in (64, 256):
        got = to_np(U.matmul_prepacked_b(a, U.pack_b_vnni_t(w, panel), n, bias, fn))
        _check(got, ref, k, to_np(a), to_np(w), "bf16")
    layer = nn.Linear(k, n, device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_(w)
        layer.bias.copy_(bias)
    y, cache = U.linear(a, layer, epilogue=fn)
    _check(to_np(y), ref, k, to_np(a), to_np(w), "bf16")
    y2, _ = U.linear(a, layer, epilogue=fn, cache=cache)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("groups", [1, 32])
@pytest.mark.parametrize("m,c", [(256, 4096), (3000, 2048), (64, 8192), (700, 320)])
def test_group_norm_programs(gpu_device, dtype: str, groups: int, m: int, c: int) -> None:
    # 3000 rows make the whole-row kernel walk several rows per block; 8192
    # channels take 512-thread workgroups (bf16) or the streaming kernel
    # (f32); 320 channels in 32 groups (10 per group) take the streaming kernel.
    x = tensor(RNG.normal(0, 2, (m, c)).astype(np.float32), dtype, gpu_device)
    w = torch.from_numpy(RNG.uniform(0.5, 1.5, c).astype(np.float32)).to(gpu_device)
    b = torch.from_numpy(RNG.normal(0, 0.5, c).astype(np.float32)).to(gpu_device)
    extra = torch.from_numpy(RNG.normal(0, 1, c).astype(np.float32)).to(gpu_device)
    fn = lambda y, e: F.silu(y * e + 1) - torch.abs(e)  # noqa: E731
    got = to_np(U.group_norm(x, groups, w, b, 1e-5, epilogue=fn, extra=extra))
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, to_np(extra), "callable", fn, out=dtype)
    assert_close(got, ref, 1e-2 if dtype == "bf16" else 1e-4, 5e-3 if dtype == "bf16" else 1e-4)
    # No extra operand: the epilogue's second operand is the weight.
    got = to_np(U.group_norm(x, groups, w, b, 1e-5, epilogue=lambda y, e: y * e))
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, None, "callable", lambda y, e: y * e, out=dtype)
    assert_close(got, ref, 1e-2 if dtype == "bf16" else 1e-4, 5e-3 if dtype == "bf16" else 1e-4)
    # GroupNormEpilogue with an activation that is a program.
    epi = U.GroupNormEpilogue("add", F.hardswish)
    got = to_np(U.group_norm(x, groups, w, b, 1e-5, epilogue=epi, extra=extra))
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, to_np(extra), "callable",
                       lambda y, e: F.hardswish(y + e), out=dtype)
    assert_close(got, ref, 1e-2 if dtype == "bf16" else 1e-4, 5e-3 if dtype == "bf16" else 1e-4)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_reduction_programs(gpu_device, dtype: str) -> None:
    m, n = 1000, 777
    x = tensor(RNG.normal(0, 1, (m, n)).astype(np.float32), dtype, gpu_device)
    v = torch.from_numpy(RNG.normal(0, 1, n).astype(np.float32)).to(gpu_device)
    fn = lambda s: F.softplus(s / 8) * 3  # noqa: E731
    tol = (1e-2, 1e-2) if dtype == "bf16" else (1e-4, 1e-4)
    assert_close(to_np(U.row_sum(x, fn)), R.row_sum(to_np(x), fn, out=dtype), *tol)
    assert_close(to_np(U.row_dot(x, v, fn)), R.row_dot(to_np(x), to_np(v), fn, out=dtype), *tol)


def test_noalloc_runs_programs(gpu_device) -> None:
    # The allocation-free entry point stages the program's f32 products in
    # its scratch when the kernel leaves the program to the reduction.
    m, n, k = 300, 200, 100
    fn = EPILOGUES["mish"]
    program = U.compile_epilogue(fn)
    a, b = _operands(m, n, k, False, False, "bf16", gpu_device)
    c = torch.empty(m, n, dtype=torch.bfloat16, device=gpu_device)
    stream = torch.cuda.current_stream(gpu_device).cuda_stream
    status = native.lib().hmx_gemm_noalloc(
        native.DTYPE_BF16, native.DTYPE_BF16, a.data_ptr(), k, 0, b.data_ptr(), n, native.B_ROW, 0, 0,
        c.data_ptr(), n, m, n, k, 1, 0, 0, 0, None, None, None, native.DTYPE_F32,
        native.EPI_PROGRAM, 0.0, ctypes.addressof(program.struct), 0, 0, 0, 0, stream)
    assert status == native.OK, native.last_error()
    torch.cuda.synchronize()
    ref = R.matmul(to_np(a), to_np(b), act=fn, out="bf16")
    _check(to_np(c), ref, k, to_np(a), to_np(b), "bf16")


def _exact_activation(name: str, x: np.ndarray) -> np.ndarray:
    """The named activations in float64 from their definitions (math.erf,
    tanh, exp): the accuracy bound the kernels' fast forms are held to."""
    import math

    x = x.astype(np.float64)
    if name == "silu":
        return x / (1.0 + np.exp(-x))
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if name == "tanh":
        return np.tanh(x)
    if name == "gelu":
        return 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))
    u = math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)
    # 1 + tanh(u) cancels in float64 too once u < -5; there it is
    # 2 / (1 + e^-2u), the same number without the cancellation.
    return np.where(u > -5.0, 0.5 * x * (1.0 + np.tanh(u)), x / (1.0 + np.exp(-2.0 * u)))


@pytest.mark.parametrize("name", ["silu", "sigmoid", "gelu", "gelu_tanh", "tanh"])
def test_fast_activations_accuracy(gpu_device, name: str) -> None:
    import math

    # C = I @ X passes X through the f32 GEMM exactly, so the epilogue sees
    # the values themselves. SiLU and sigmoid (hardware reciprocal), tanh
    # (series below 0.25, 1 - 2 / (1 + e^2|x|) above) and tanh-GELU
    # (x / (1 + e^-2u)) stay within 2e-6 relative over [-12, 12]
    # (e^x as v_exp_f32 of x log2 e loses up to ~1e-6 at |x| = 12); GELU's
    # erf by Abramowitz & Stegun 7.1.26 within its 1.5e-7 absolute bound on
    # erf, 0.5 |x| 1.5e-7 on GELU, plus the same relative rounding. A wrong
    # coefficient or branch fails these by orders of magnitude.
    x = np.linspace(-12.0, 12.0, 128 * 512, dtype=np.float32).reshape(128, 512)
    eye = torch.eye(128, device=gpu_device)
    fn = {"silu": F.silu, "sigmoid": torch.sigmoid, "gelu": F.gelu, "gelu_tanh": U.Activation("gelu_tanh"),
          "tanh": torch.tanh}[name]
    got = to_np(U.matmul(eye, torch.from_numpy(x).to(gpu_device), epilogue=fn)).astype(np.float64)
    exact = _exact_activation(name, x)
    err = np.abs(got - exact)
    if name == "gelu":
        assert (err <= 0.5 * np.abs(x) * 2e-7 + 2e-6 * np.abs(exact) + 1e-30).all(), float(err.max())
    elif name == "gelu_tanh":
        # u = sqrt(2/pi) (x + 0.044715 x^3) itself is an f32 value: its
        # rounding (~|u| 2^-24) moves e^(-2u) by a relative 2|u| 2^-24, which
        # far out on the negative side outweighs the rest. (torch, adding
        # tanh(u) to 1 in f32, returns 0 there.)
        u = np.abs(math.sqrt(2.0 / math.pi) * (x.astype(np.float64) + 0.044715 * x.astype(np.float64) ** 3))
        assert (err <= (2e-6 + 4e-7 * u) * np.abs(exact) + 1e-30).all(), float(err.max())
    else:
        # (Values below 1e-30, where f32 has underflowed as torch's does, are exempt.)
        assert (err <= 2e-6 * np.abs(exact) + 1e-30).all(), float((err / np.maximum(np.abs(exact), 1e-30)).max())


# Run-time compiled epilogues (hmx_jit.cpp): the 16x16x32 kernel with the
# program or named activation compiled into its register epilogue. Each
# shape reaches one of its variants: whole 256 x 256 tiles, ragged ones, the
# 256 x 128 round after whole rounds of 256 x 256, 128 x 128 tiles (K of 16+
# stages), and f32 C.
JIT_SHAPES = {
    "whole": (4096, 4096, 256, False, "bf16"),
    "ragged": (4000, 4104, 256, True, "bf16"),
    "round_tail": (4096, 4352, 256, True, "bf16"),
    "tiles_128": (512, 512, 1024, False, "bf16"),
    "f32_out": (4096, 4096, 256, True, "f32"),
}


def _jit_launches() -> int:
    return native.jit_info()["launches"]


@pytest.mark.parametrize("shape", list(JIT_SHAPES))
@pytest.mark.parametrize("epi", ["silu_mix", "hardswish", "gelu_named", "module"])
def test_jit_epilogues_run_compiled(gpu_device, monkeypatch, shape: str, epi: str) -> None:
    m, n, k, tb, out = JIT_SHAPES[shape]
    fn = EPILOGUES[epi]
    a, b = _operands(m, n, k, False, tb, "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    out_dtype = torch.float32 if out == "f32" else None
    start = native.jit_info()
    got = U.matmul(a, b, trans_b=tb, bias=bias, epilogue=fn, out_dtype=out_dtype)
    torch.cuda.synchronize()
    info = native.jit_info()
    assert info["failed"] == start["failed"], info["last_failure_log"]
    assert info["launches"] > start["launches"], "the compiled kernel did not run"
    if shape == "round_tail":
        # Whole rounds of 256 x 256 tiles and the 256 x 128 tail: one
        # compiled launch for both.
        assert info["launches"] - start["launches"] == 1
    ref = R.matmul(to_np(a), to_np(b), False, tb, to_np(bias), act=fn, out=out)
    if out == "f32":
        assert_close(to_np(got), ref, 1e-4, 2 * 3 * bf16_gemm_atol(k, to_np(a), to_np(b)))
    else:
        _check(to_np(got), ref, k, to_np(a), to_np(b), out)
    # With run-time compilation off the interpreter runs it; on whole tiles
    # it is the same 16x16x32 kernel, so the two agree bit for bit (the
    # compiled code evaluates each instruction with the interpreter's
    # formula).
    monkeypatch.setenv("HMX_JIT", "0")
    before = _jit_launches()
    again = U.matmul(a, b, trans_b=tb, bias=bias, epilogue=fn, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert _jit_launches() == before
    if shape in ("whole", "f32_out"):
        assert torch.equal(got, again)
    else:
        if out == "f32":
            assert_close(to_np(again), ref, 1e-4, 2 * 3 * bf16_gemm_atol(k, to_np(a), to_np(b)))
        else:
            _check(to_np(again), ref, k, to_np(a), to_np(b), out)


@pytest.mark.parametrize("act", [F.gelu, torch.tanh, torch.sigmoid, lambda x: F.leaky_relu(x, 0.2),
                                 lambda x: F.gelu(x, approximate="tanh")])
def test_jit_named_activations_match_the_staged_epilogue(gpu_device, monkeypatch, act) -> None:
    # Named activations the precompiled register epilogue does not carry run
    # compiled in; the staged epilogue they replace computes the same formula.
    m, n, k = 4096, 4096, 256
    a, b = _operands(m, n, k, False, True, "bf16", gpu_device)
    scale = torch.from_numpy(RNG.uniform(0.5, 1.5, n).astype(np.float32)).to(gpu_device)
    got = U.matmul(a, b, trans_b=True, epilogue=act, scale=scale)
    monkeypatch.setenv("HMX_JIT", "0")
    staged = U.matmul(a, b, trans_b=True, epilogue=act, scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(got, staged)
    ref = R.matmul(to_np(a), to_np(b), False, True, None, to_np(scale), act=act, out="bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("groups,c", [(32, 4096), (1, 4096), (1, 8192), (32, 2048)])
def test_jit_group_norm_programs(gpu_device, monkeypatch, dtype: str, groups: int, c: int) -> None:
    # Whole-row GroupNorm with the program compiled in: every row shape the
    # whole-row kernel takes (8192 f32 channels need 16 waves, which the
    # interpreter's kernels cannot hold: they take the streaming kernel).
    m = 600
    x = tensor(RNG.normal(0, 2, (m, c)).astype(np.float32), dtype, gpu_device)
    w = torch.from_numpy(RNG.uniform(0.5, 1.5, c).astype(np.float32)).to(gpu_device)
    b = torch.from_numpy(RNG.normal(0, 0.5, c).astype(np.float32)).to(gpu_device)
    extra = torch.from_numpy(RNG.normal(0, 1, c).astype(np.float32)).to(gpu_device)
    fn = lambda y, e: F.silu(y * e + 1) - e  # noqa: E731
    start = native.jit_info()
    got = U.group_norm(x, groups, w, b, 1e-5, epilogue=fn, extra=extra)
    torch.cuda.synchronize()
    info = native.jit_info()
    assert info["failed"] == start["failed"], info["last_failure_log"]
    assert info["launches"] > start["launches"], "the compiled kernel did not run"
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, to_np(extra), "callable", fn, out=dtype)
    assert_close(to_np(got), ref, 1e-2 if dtype == "bf16" else 1e-4, 5e-3 if dtype == "bf16" else 1e-4)
    monkeypatch.setenv("HMX_JIT", "0")
    again = U.group_norm(x, groups, w, b, 1e-5, epilogue=fn, extra=extra)
    torch.cuda.synchronize()
    if dtype == "bf16" or c <= 4096:
        # The same whole-row kernel with the interpreter: the same bits.
        assert torch.equal(got, again)
    else:
        assert_close(to_np(again), ref, 1e-4, 1e-4)


@pytest.mark.parametrize("layout", ["blocked_vnni", "vnni64", "vnni512", "panels64", "blocked"])
def test_jit_epilogues_on_packed_b(gpu_device, layout: str) -> None:
    # Whole 256 x 256 tiles with B in each packed layout: the 16x16x32 kernel
    # compiled with the program for that layout's loads, bit-equal to the
    # same product with plain B (the same K walk and the same compiled
    # epilogue), and to the oracle within the bf16 tolerance.
    m, n, k = 512, 1024, 384
    fn = EPILOGUES["silu_mix"]
    a, b = _operands(m, n, k, False, False, "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    bt = b.t().contiguous()
    packed = {"blocked_vnni": lambda: U.pack_b_blocked_vnni(b), "vnni64": lambda: U.pack_b_vnni_t(bt, 64),
              "vnni512": lambda: U.pack_b_vnni_t(bt, 512), "panels64": lambda: U.pack_b_panels(b, 64),
              "blocked": lambda: U.pack_b_blocked(b)}[layout]()
    start = native.jit_info()
    got = U.matmul_prepacked_b(a, packed, n, bias, fn)
    torch.cuda.synchronize()
    info = native.jit_info()
    assert info["failed"] == start["failed"], info["last_failure_log"]
    assert info["launches"] > start["launches"], "the compiled kernel did not run"
    assert torch.equal(got, U.matmul(a, b, bias=bias, epilogue=fn))
    ref = R.matmul(to_np(a), to_np(b), bias=to_np(bias), act=fn, out="bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


def test_no_run_time_compilation_failed(gpu_device) -> None:
    # Every kernel the tests above compiled at run time compiled: a failure
    # would have sent its GEMM to the interpreter without an error.
    info = native.jit_info()
    assert info["failed"] == 0, info["last_failure_log"]
