"""Parity of the gfx950 kernels on adversarial values: signed zeros, infinities,
NaN, the smallest normal and the largest finite value of the dtype, and the
dtype's neighbours of large and small constants (the kind of values the
reference's own tests use, tests/inputs.py:22-76), spread so that rows, lanes
and columns 16 or 64 apart all differ.

Each result is compared with the CPU oracle: the same NaNs and infinities
element for element, finite elements within the dtype's tolerance. Sums
(norms, reductions) leave out the largest finite value: whether such a sum
overflows depends on the order of its terms. The softmax rows of the
reference's formulation, ``exp(x - row_max)`` (normalization.py:61-72), stay
finite for any finite row: ``[1e10, 0]`` is ``[1, 0]`` and a one-column row
is ``x - x + 1`` (normalization.py:76-87), exactly 1 for every finite x.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import helion_mlir_utils as U
from oracle import restate as R
from tests.helpers import (
    assert_specials_close,
    max_rel_error,
    special_values,
    spread,
    tensor,
    to_np,
)

pytestmark = pytest.mark.gpu

DTYPES = ["f32", "bf16"]


def _tol(dtype: str) -> tuple[float, float]:
    return (1e-5, 1e-6) if dtype == "f32" else (1e-2, 1e-3)


# ---------------------------------------------------------------------------
# softmax


@pytest.mark.parametrize("dtype", DTYPES)
def test_softmax_large_finite_rows(gpu_device, dtype: str) -> None:
    rows = np.array([[1e10, 0.0], [-1e10, -1e10 + 2048.0], [3e38, -3e38], [-3e38, -3e38], [5e9, 5e9],
                     [-5e9, 1e-30]], np.float32)
    x = tensor(rows, dtype, gpu_device)
    got = to_np(U.softmax(x))
    exact = torch.softmax(x.double().cpu(), -1).numpy().astype(np.float32)
    # Every answer here is 0, 0.5 or 1 (or the bf16 rounding of the rows
    # makes a row's values equal): exact in any dtype.
    np.testing.assert_array_equal(got, exact)
    np.testing.assert_array_equal(got, R.softmax(to_np(x), dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows", [1, 5, 70])
def test_softmax_one_column_is_x_minus_x_plus_one(gpu_device, dtype: str, rows: int) -> None:
    values = special_values(dtype, (5e9, 3e9, 1e10, 0.5, 1e-30, 65504.0))
    x = tensor(spread(values, rows * len(values), 1), dtype, gpu_device)
    got = to_np(U.softmax(x))
    xs = to_np(x)
    expected = np.where(np.isfinite(xs), np.float32(1.0), np.float32(np.nan))
    np.testing.assert_array_equal(got, expected)
    np.testing.assert_array_equal(got, R.softmax(xs, dtype))


SOFTMAX_SETS = {
    "all": dict(constants=(1e10, 5e9, 0.5, 1.0, 88.0, 100.0)),
    "finite": dict(constants=(1e10, 5e9, 0.5, 1.0, 88.0, 100.0), finite=True),
    # rows whose maximum is a large finite value and whose others reach -inf
    "no_max": dict(constants=(1e10, 0.5, 1.0, 30.0), largest=False),
}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("values", list(SOFTMAX_SETS))
@pytest.mark.parametrize("cols", [2, 7, 64, 65, 129, 1024, 4100, 20000])
def test_softmax_specials(gpu_device, dtype: str, values: str, cols: int) -> None:
    vals = special_values(dtype, **SOFTMAX_SETS[values])
    if values == "no_max":
        vals = [v for v in vals if not (np.isnan(v) or v == float("inf"))]
    x = tensor(spread(vals, 37, cols), dtype, gpu_device)
    got = to_np(U.softmax(x))
    ref = R.softmax(to_np(x), dtype)
    assert_specials_close(got, ref, *_tol(dtype))
    fin = np.isfinite(ref).all(axis=1)
    if fin.any():
        assert max_rel_error(got[fin], ref[fin]) < (1e-6 if dtype == "f32" else 1e-2)
    # in place: the same bits
    y = x.clone()
    assert torch.equal(torch.nan_to_num(U.softmax(y, in_place=True), 7.0),
                       torch.nan_to_num(U.softmax(x), 7.0))


# ---------------------------------------------------------------------------
# RMSNorm: a square of the largest value is +inf in any order, so the sum of
# squares is +inf (the row's rsqrt 0) whatever order its terms are added in.


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "n"), [(21, 7), (9, 64), (7, 333), (4, 4096), (3, 20000)])
def test_rms_norm_specials(gpu_device, dtype: str, m: int, n: int) -> None:
    vals = special_values(dtype, (1e15, 0.5, 1.0, 3.0, 1e-20))
    x = tensor(spread(vals, m, n), dtype, gpu_device)
    # weight: finite specials, shifted against x's columns
    wv = special_values(dtype, (0.5, 2.0, 1e10), finite=True)
    w = tensor(spread(wv, 3, n)[2], dtype, gpu_device)
    xs, ws = to_np(x), to_np(w)
    for weight, wref in ((w, ws), (None, None)):
        got = to_np(U.rms_norm(x, weight, 1e-6))
        ref = R.rms_norm(xs, wref, 1e-6, dtype)
        assert_specials_close(got, ref, *_tol(dtype))


# ---------------------------------------------------------------------------
# GroupNorm / LayerNorm and the reductions: no +-max (order-dependent
# overflow of the sums); inf and NaN make a group or row NaN / inf in any
# order.


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "c", "groups"), [(23, 64, 4), (5, 4096, 1), (9, 96, 3), (2, 20000, 1), (13, 4096, 32)])
@pytest.mark.parametrize("finite", [True, False])
def test_group_norm_specials(gpu_device, dtype: str, m: int, c: int, groups: int, finite: bool) -> None:
    vals = special_values(dtype, (1e15, 0.5, 1.0, 3.0, 1e-20), finite=finite, largest=False)
    x = tensor(spread(vals, m, c), dtype, gpu_device)
    vv = special_values(dtype, (0.5, 2.0), finite=True, largest=False)
    w, b, e = (tensor(spread(vv, 5, c)[i], dtype, gpu_device) for i in (1, 2, 3))
    xs, ws, bs, es = map(to_np, (x, w, b, e))
    got = to_np(U.group_norm(x, groups, w, b, 1e-5))
    ref = R.group_norm(xs, groups, ws, bs, 1e-5, out=dtype)
    rtol, atol = _tol(dtype)
    assert_specials_close(got, ref, rtol * 10, atol * 10)
    got = to_np(U.group_norm(x, groups, w, b, 1e-5, U.GroupNormEpilogue("add", F.silu), e))
    ref = R.group_norm(xs, groups, ws, bs, 1e-5, es, "add", "silu", out=dtype)
    assert_specials_close(got, ref, rtol * 10, atol * 10)


def _sum_tol(terms: np.ndarray, axis: int, dtype: str) -> np.ndarray:
    """atol of a sum in another order: a few ulps of the sum of |terms|."""
    with np.errstate(invalid="ignore"):
        mag = np.where(np.isfinite(terms), np.abs(terms), 0.0).sum(axis=axis, keepdims=True)
    return mag * (2.0**-20 if dtype == "f32" else 2.0**-7) + 1e-30


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "n"), [(21, 5), (9, 64), (11, 513), (3, 4096)])
def test_reductions_specials(gpu_device, dtype: str, m: int, n: int) -> None:
    vals = special_values(dtype, (100.0, 0.5, 1.0, 3.0, 1e-20), largest=False)
    x = tensor(spread(vals, m, n), dtype, gpu_device)
    vv = special_values("f32", (0.5, 2.0), largest=False)
    v = torch.from_numpy(spread(vv, 2, n)[1]).to(gpu_device)
    xs, vs = to_np(x), to_np(v)
    rtol = 1e-5 if dtype == "f32" else 1e-2
    tol_rows = _sum_tol(xs.astype(np.float64), 1, dtype)
    assert_specials_close(to_np(U.row_sum(x)), R.row_sum(xs, out=dtype), rtol, tol_rows)
    assert_specials_close(to_np(U.row_sum(x, torch.relu)), R.row_sum(xs, "relu", out=dtype), rtol, tol_rows)
    assert_specials_close(to_np(U.column_sum(x)), R.column_sum(xs), 1e-5, _sum_tol(xs.astype(np.float64), 0, "f32")[0])
    with np.errstate(invalid="ignore"):
        prod = xs.astype(np.float64) * vs.astype(np.float64)[None, :]
    assert_specials_close(to_np(U.row_dot(x, v)), R.row_dot(xs, vs, out=dtype), rtol, _sum_tol(prod, 1, dtype))
    xv = tensor(vs, dtype, gpu_device)
    xvs = to_np(xv)
    with np.errstate(invalid="ignore"):
        prod = xs.astype(np.float64) * xvs.astype(np.float64)[None, :]
    assert_specials_close(to_np(U.matvec(x, xv.reshape(n, 1))), R.matvec(xs, xvs, out=dtype), rtol,
                          _sum_tol(prod, 1, dtype))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("numel", [9, 4096, 100003])
def test_elementwise_specials_bit_exact(gpu_device, dtype: str, numel: int) -> None:
    vals = special_values(dtype, (1e10, 0.5, 1.0, 1e-30))
    x = tensor(spread(vals, 1, numel)[0], dtype, gpu_device)
    xs = to_np(x)
    for got, ref in (
        (U.relu(x), R.relu(xs, dtype)),
        (U.leaky_relu(x, 0.1), R.leaky_relu(xs, 0.1, dtype)),
        (U.scalar_mul(x, 2.5), R.scalar_mul(xs, 2.5, dtype)),
        (U.scalar_mul(x, -1e30), R.scalar_mul(xs, -1e30, dtype)),
    ):
        g = to_np(got)
        # bit for bit, signed zeros included; NaN by position
        assert np.array_equal(np.isnan(g), np.isnan(ref))
        keep = ~np.isnan(ref)
        assert np.array_equal(g[keep].view(np.uint32), ref[keep].view(np.uint32))


# ---------------------------------------------------------------------------
# GEMM epilogues: small-integer operands make every accumulator exact in f32,
# so the kernel and the oracle apply the epilogue to the same values; bias,
# scale and shift carry the special values.

ACTS = {"identity": U.identity_epilogue, "relu": torch.relu, "silu": F.silu, "sigmoid": torch.sigmoid,
        "gelu": F.gelu, "gelu_tanh": U.Activation("gelu_tanh"), "tanh": torch.tanh,
        "leaky_relu": U.Activation("leaky_relu", 0.2)}

RNG = np.random.default_rng(2024)


def _int_operand(shape: tuple[int, int], dtype: str, device) -> torch.Tensor:
    return tensor(RNG.integers(-3, 4, shape).astype(np.float32), dtype, device)


# (m, n, k, trans_b): whole 256 x 256 tiles (direct-to-LDS), 128 x 128
# tiles, ragged edges, a decode-shaped product (skinny kernel) and a long-K
# product that splits K (the reduction kernel applies the epilogue).
EPI_SHAPES = [(256, 256, 128, False), (512, 512, 128, True), (70, 45, 130, False),
              (32, 320, 128, True), (64, 64, 2048, False)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("act", list(ACTS))
@pytest.mark.parametrize("shape", EPI_SHAPES)
def test_gemm_epilogue_specials(gpu_device, dtype: str, act: str, shape) -> None:
    m, n, k, trans_b = shape
    a = _int_operand((m, k), dtype, gpu_device)
    b = _int_operand((n, k) if trans_b else (k, n), dtype, gpu_device)
    vals = special_values("f32", (0.5, 1e10, 2.0, 1e-30))
    bias, scale, shift = (torch.from_numpy(spread(vals, 4, n)[i]).to(gpu_device) for i in (1, 2, 3))
    got = to_np(U.matmul(a, b, trans_b=trans_b, bias=bias, scale=scale, shift=shift, epilogue=ACTS[act]))
    arg = 0.2 if act == "leaky_relu" else 0.01
    ref = R.matmul(to_np(a), to_np(b), False, trans_b, to_np(bias), to_np(scale), to_np(shift), act, arg, out=dtype)
    rtol, atol = (1e-5, 1e-6) if dtype == "f32" else (1e-2, 1e-6)
    assert_specials_close(got, ref, rtol, atol)


# ---------------------------------------------------------------------------
# GEMM operands holding inf and NaN: a product of inf and 0 is NaN and +inf
# meeting -inf is NaN, so a kernel that lets padding or a neighbouring row or
# column into a sum (a K tail read past the end, a clamped edge load that is
# stored) shows up in the NaN / inf pattern of C. The expected C is summed
# element by element in float64 (IEEE semantics throughout; no BLAS).


def _ieee_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):
        return (a.astype(np.float64)[:, :, None] * b.astype(np.float64)[None, :, :]).sum(axis=1)


def _sparse_specials(shape: tuple[int, int], dtype: str, every: int) -> np.ndarray:
    x = RNG.integers(-3, 4, shape).astype(np.float32)
    vals = [np.inf, -np.inf, np.nan, 0.0, -0.0]
    flat = x.reshape(-1)
    pos = np.arange(0, flat.size, every)
    flat[pos] = np.asarray(vals, np.float32)[np.arange(pos.size) % len(vals)]
    # The first and last column of some rows, and the first and last row of
    # some columns: what a K tail read past the end of a row, or a read of a
    # neighbouring row, would pick up.
    x[5::13, 0] = np.inf
    x[9::13, -1] = np.nan
    x[0, 7::17] = -np.inf
    x[-1, 3::19] = np.nan
    return x


OPERAND_SHAPES = [(70, 96, 130, False), (37, 45, 70, True), (256, 256, 192, False), (300, 260, 192, False),
                  (300, 260, 192, True), (64, 64, 4096, False), (16, 256, 128, True), (128, 128, 96, True)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", OPERAND_SHAPES)
def test_gemm_operand_specials(gpu_device, dtype: str, shape) -> None:
    m, n, k, trans_b = shape
    a_np = _sparse_specials((m, k), dtype, 997 if m * k < 50000 else 30011)
    b_np = _sparse_specials((n, k) if trans_b else (k, n), dtype, 1009 if n * k < 50000 else 30013)
    a, b = tensor(a_np, dtype, gpu_device), tensor(b_np, dtype, gpu_device)
    got = to_np(U.matmul(a, b, trans_b=trans_b))
    exact = _ieee_matmul(to_np(a), to_np(b).T if trans_b else to_np(b))
    ref = R.round_to(exact.astype(np.float32), dtype)
    # small-integer finite terms: every finite element is exact
    assert_specials_close(got, ref, 0.0, 0.0)
