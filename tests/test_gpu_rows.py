"""Parity of the gfx950 row kernels with the CPU oracle: softmax, RMSNorm,
GroupNorm/LayerNorm, row/column reductions, gemv and elementwise ops.

Tolerances: the reference's own for softmax (max-normalised error < 1e-6 for
f32, < 1e-2 for bf16; tests/test_cpu_utils_softmax.py:18-34); rtol 1e-4 for
f32 and one bf16 rounding (rtol 1e-2) for bf16 elsewhere. The full config-2
size is checked on sampled rows against the oracle plus a whole-tensor
invariant (softmax rows sum to 1).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helion_mlir_utils as U
from helion_mlir_backend._compiler import native
import hmx_workloads as W
from oracle import restate as R
from tests.helpers import assert_close, max_rel_error, tensor, to_np

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(99)


def _tol(dtype: str) -> tuple[float, float]:
    return (1e-4, 1e-5) if dtype == "f32" else (1e-2, 1e-3)


# ---------------------------------------------------------------------------
# softmax


@pytest.mark.parametrize(
    ("m", "n", "shift"),
    [(130, 515, 0.0), (4, 129, -50.0), (2, 200, -50.0), (4, 256, -50.0), (3, 47, 0.0),
     (7, 4096, 0.0), (5, 4097, 3.0), (3, 9000, 0.0), (64, 1, 0.0), (1, 64, 0.0), (33, 8, 100.0),
     # one row per workgroup of 2..16 waves (whole and ragged), then the streaming kernel
     (3, 1024, 0.0), (2, 2048, 0.0), (2, 2056, 0.0), (2, 16384, 0.0), (2, 16388, 0.0), (2, 33000, 0.0)],
)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_matches_oracle(gpu_device, m: int, n: int, shift: float, dtype: str) -> None:
    x = RNG.normal(0, 1, (m, n)).astype(np.float32) + np.float32(shift)
    xt = tensor(x, dtype, gpu_device)
    got = to_np(U.softmax(xt))
    ref = R.softmax(to_np(xt), dtype)
    assert max_rel_error(got, ref) < (1e-6 if dtype == "f32" else 1e-2)
    f64 = torch.softmax(xt.double().cpu(), -1).numpy()
    assert max_rel_error(got, f64) < (1e-6 if dtype == "f32" else 1e-2)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_nonfinite_and_one_column(gpu_device, dtype: str) -> None:
    col = np.array([[0.5], [-3e4], [np.nan], [np.inf], [-np.inf]], np.float32)
    col = np.concatenate([col, RNG.normal(0, 1, (60, 1)).astype(np.float32)])
    got = to_np(U.softmax(tensor(col, dtype, gpu_device)))
    ref = R.softmax(col, dtype)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    rows = np.array([[1.0, np.nan, 2.0], [1.0, np.inf, 2.0], [-np.inf] * 3, [1.0, -np.inf, 1.0]], np.float32)
    got = to_np(U.softmax(tensor(rows, dtype, gpu_device)))
    ref = R.softmax(rows, dtype)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_allclose(got[3], [0.5, 0.0, 0.5], rtol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(32, 128), (64, 256), (16, 129), (33, 257), (2, 65), (1, 127), (5, 2),
                                   (4, 4096), (2, 9000)])
def test_softmax_in_place_is_the_out_of_place_result(gpu_device, shape, dtype: str) -> None:
    # test_cpu_utils_softmax.py:58-76: in place is bit-equal, the input of the
    # out-of-place call is left alone.
    x = tensor(RNG.normal(0, 3, shape).astype(np.float32), dtype, gpu_device)
    before = x.clone()
    out = U.softmax(x)
    assert torch.equal(x, before)
    y = x.clone()
    pointer = y.data_ptr()
    inplace = U.softmax(y, in_place=True)
    assert inplace.data_ptr() == pointer
    assert torch.equal(inplace, out)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_softmax_config2_full_size(gpu_device, dtype: str) -> None:
    cfg = W.config2(torch.bfloat16 if dtype == "bf16" else torch.float32)
    x = cfg["x"].to(gpu_device)
    y = U.softmax(x)
    torch.cuda.synchronize()
    sums = y.double().sum(-1)
    assert torch.allclose(sums, torch.ones_like(sums), atol=(1e-5 if dtype == "f32" else 2e-2))
    rows = np.sort(RNG.choice(x.shape[0], 256, replace=False))
    got = to_np(y[torch.from_numpy(rows).to(gpu_device)])
    ref = R.softmax(to_np(cfg["x"][torch.from_numpy(rows)]), dtype)
    assert max_rel_error(got, ref) < (1e-6 if dtype == "f32" else 1e-2)


# ---------------------------------------------------------------------------
# RMSNorm


@pytest.mark.parametrize(("m", "n"), [(17, 333), (8, 4096), (3, 5000), (64, 64), (5, 3), (2, 12000),
                                     (4, 1024), (3, 16384), (2, 16400)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("scale", [2.0, 1e-4])
def test_rms_norm_matches_oracle(gpu_device, m: int, n: int, dtype: str, scale: float) -> None:
    x = tensor(RNG.normal(0, scale, (m, n)).astype(np.float32), dtype, gpu_device)
    w = tensor(RNG.uniform(0.5, 1.5, n).astype(np.float32), dtype, gpu_device)
    got = to_np(U.rms_norm(x, w, 1e-6))
    ref = R.rms_norm(to_np(x), to_np(w), 1e-6, dtype)
    rtol, atol = _tol(dtype)
    assert_close(got, ref, rtol, atol * (1 if scale > 1 else 1e-2))
    got_nw = to_np(U.rms_norm(x, None, 1e-6))
    assert_close(got_nw, R.rms_norm(to_np(x), None, 1e-6, dtype), rtol, atol)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_rms_norm_config2_full_size(gpu_device, dtype: str) -> None:
    cfg = W.config2(torch.bfloat16 if dtype == "bf16" else torch.float32)
    x, w = cfg["x"].to(gpu_device), cfg["weight"].to(gpu_device)
    y = U.rms_norm(x, w, cfg["eps"])
    torch.cuda.synchronize()
    rows = np.sort(RNG.choice(x.shape[0], 256, replace=False))
    idx = torch.from_numpy(rows)
    got = to_np(y[idx.to(gpu_device)])
    ref = R.rms_norm(to_np(cfg["x"][idx]), to_np(cfg["weight"]), cfg["eps"], dtype)
    assert_close(got, ref, *_tol(dtype))
    y2 = U.rms_norm(x.clone(), w, cfg["eps"], in_place=True)
    assert torch.equal(y2, y)


# ---------------------------------------------------------------------------
# GroupNorm / LayerNorm


@pytest.mark.parametrize(("m", "c", "groups"), [(32, 256, 16), (33, 256, 4), (64, 512, 512), (5, 96, 3), (2, 65, 5), (4, 8192, 1),
                                                 (3, 2048, 2), (2, 16384, 1), (2, 20000, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_group_norm_matches_oracle(gpu_device, m: int, c: int, groups: int, dtype: str) -> None:
    x = tensor((RNG.normal(0, 3, (m, c)) + 1.5).astype(np.float32), dtype, gpu_device)
    w = tensor(RNG.normal(0, 1, c).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.normal(0, 1, c).astype(np.float32), dtype, gpu_device)
    got = to_np(U.group_norm(x, groups, w, b, 1e-5))
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, out=dtype)
    rtol, atol = _tol(dtype)
    assert_close(got, ref, rtol, atol * 10)
    y = x.clone()
    pointer = y.data_ptr()
    inplace = U.group_norm(y, groups, w, b, 1e-5, in_place=True)
    assert inplace.data_ptr() == pointer
    assert torch.equal(inplace, U.group_norm(x, groups, w, b, 1e-5))


@pytest.mark.parametrize("groups", [32, 64, 512])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_group_norm_lane_groups(gpu_device, groups: int, dtype: str) -> None:
    # Groups of 128, 64 and 8 channels: several groups per wave (lane groups of
    # 4-32 lanes), 1001 rows so the last wave is partly filled.
    m, c = 1001, 4096
    x = tensor((RNG.normal(0, 3, (m, c)) + 1.5).astype(np.float32), dtype, gpu_device)
    w = tensor(RNG.normal(0, 1, c).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.normal(0, 1, c).astype(np.float32), dtype, gpu_device)
    got = to_np(U.group_norm(x, groups, w, b, 1e-5))
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, out=dtype)
    rtol, atol = _tol(dtype)
    assert_close(got, ref, rtol, atol * 10)


@pytest.mark.parametrize(
    ("m", "c", "groups", "extra"),
    [(20000, 4096, 1, False), (20000, 4096, 32, True), (100003, 256, 16, False), (5001, 2048, 2, True),
     (3001, 16384, 4, False)],
)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_group_norm_walks_many_rows(gpu_device, m: int, c: int, groups: int, extra: bool, dtype: str) -> None:
    # More rows than the GPU holds workgroups at once: each workgroup of the
    # whole-row kernel normalizes many rows, loading the next row while it
    # reduces the current one, with w, b and extra held across rows (f32
    # vectors, as the benchmark passes them). Rows sampled from the start,
    # the end and between are checked against the oracle.
    gen = torch.Generator(device=gpu_device).manual_seed(m + c + groups)
    x = (torch.randn(m, c, device=gpu_device, generator=gen) * 3 + 1.5).to(torch.bfloat16 if dtype == "bf16" else torch.float32)
    w, b, e = (torch.randn(c, device=gpu_device, generator=gen) for _ in range(3))
    y = U.group_norm(x, groups, w, b, 1e-5, torch.add, e) if extra else U.group_norm(x, groups, w, b, 1e-5)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(8), m - 8 + np.arange(8), RNG.choice(m, 240, replace=False)]))
    idx = torch.from_numpy(rows).to(gpu_device)
    xs, ws, bs, es = to_np(x[idx]), to_np(w), to_np(b), to_np(e)
    if extra:
        ref = R.group_norm(xs, groups, ws, bs, 1e-5, es, "add", out=dtype)
    else:
        ref = R.group_norm(xs, groups, ws, bs, 1e-5, out=dtype)
    rtol, atol = _tol(dtype)
    assert_close(to_np(y[idx]), ref, rtol, atol * 10)


@pytest.mark.parametrize(("dtype", "c"), [("bf16", 4096), ("f32", 4096), ("bf16", 1000)])
def test_group_norm_bf16_vectors_through_the_abi(gpu_device, dtype: str, c: int) -> None:
    # bf16 weight, bias and extra operand (the C ABI takes either vector
    # dtype), loaded a row vector at a time where the rows allow it.
    m, groups = 33, 8
    x = tensor(RNG.normal(0, 2, (m, c)).astype(np.float32), dtype, gpu_device)
    w, b, e = (tensor(RNG.normal(0, 1, c).astype(np.float32), "bf16", gpu_device) for _ in range(3))
    y = torch.empty_like(x)
    native.call("hmx_group_norm_rows", native.dtype_code(x.dtype), x.data_ptr(), w.data_ptr(), b.data_ptr(),
                e.data_ptr(), native.DTYPE_BF16, y.data_ptr(), m, groups, c // groups, 1e-5, native.EXTRA_ADD,
                native.EPI_RELU, 0.0, None, torch.cuda.current_stream().cuda_stream)
    ref = R.group_norm(to_np(x), groups, to_np(w), to_np(b), 1e-5, to_np(e), "add", "relu", out=dtype)
    rtol, atol = _tol(dtype)
    assert_close(to_np(y), ref, rtol, atol * 10)


def test_group_norm_epilogues_and_layer_norm(gpu_device) -> None:
    x = tensor(RNG.normal(0, 2, (9, 130)).astype(np.float32), "f32", gpu_device)
    w, b, extra = (tensor(RNG.normal(0, 1, 130).astype(np.float32), "f32", gpu_device) for _ in range(3))
    xs, ws, bs, es = map(to_np, (x, w, b, extra))
    got = to_np(U.group_norm(x, 1, w, b, 1e-5, torch.add, extra))
    assert_close(got, R.group_norm(xs, 1, ws, bs, 1e-5, es, "add"), 1e-4, 1e-4)
    got = to_np(U.group_norm(x, 1, w, b, 1e-5, U.GroupNormEpilogue("mul", torch.relu), extra))
    assert_close(got, R.group_norm(xs, 1, ws, bs, 1e-5, es, "mul", "relu"), 1e-4, 1e-4)
    got = to_np(U.layer_norm(x, w, b, 1e-5))
    assert_close(got, R.group_norm(xs, 1, ws, bs, 1e-5), 1e-4, 1e-4)


# ---------------------------------------------------------------------------
# Reductions, gemv, elementwise


@pytest.mark.parametrize(("m", "n"), [(33, 517), (1, 4096), (300, 8), (16, 100000)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_reductions_match_oracle(gpu_device, m: int, n: int, dtype: str) -> None:
    x = tensor(RNG.normal(0, 1, (m, n)).astype(np.float32), dtype, gpu_device)
    v = torch.from_numpy(RNG.normal(0, 1, n).astype(np.float32)).to(gpu_device)
    xs, vs = to_np(x), to_np(v)
    rtol, atol = (1e-4, 1e-4 * np.sqrt(n)) if dtype == "f32" else (1e-2, 1e-2 * np.sqrt(n))
    assert_close(to_np(U.row_sum(x)), R.row_sum(xs, out=dtype), rtol, atol)
    assert_close(to_np(U.row_sum(x, torch.relu)), R.row_sum(xs, "relu", out=dtype), rtol, atol)
    assert_close(to_np(U.column_sum(x)), R.column_sum(xs), 1e-4, 1e-4 * np.sqrt(m))
    assert_close(to_np(U.row_dot(x, v)), R.row_dot(xs, vs, out=dtype), rtol, atol)
    xv = tensor(vs, dtype, gpu_device)
    got = to_np(U.matvec(x, xv.reshape(n, 1)))
    assert_close(got, R.matvec(xs, to_np(xv), out=dtype), rtol, atol)


@pytest.mark.parametrize(("m", "n"), [(5000, 300), (70000, 64), (4096, 4096), (1025, 517), (257, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_column_sum_row_chunks(gpu_device, m: int, n: int, dtype: str) -> None:
    # Several row chunks (partials in the workspace, added in chunk order),
    # ragged column blocks, and a row-offset view whose rows lose 16-byte
    # alignment when n is odd (the scalar loads).
    x = tensor(RNG.normal(0, 1, (m, n)).astype(np.float32), dtype, gpu_device)
    got = U.column_sum(x)
    assert torch.equal(got, U.column_sum(x))
    xs = to_np(x)
    assert_close(to_np(got), R.column_sum(xs), 1e-4, 1e-4 * np.sqrt(m))
    assert_close(to_np(U.column_sum(x[1:])), R.column_sum(xs[1:]), 1e-4, 1e-4 * np.sqrt(m))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_column_sum_benchmark_shape(gpu_device, dtype: str) -> None:
    # The benchmark's [32768, 4096]: 128 row chunks of 256 rows over column
    # blocks of 1 KiB row pieces, chunk sums added in order by 8 threads per
    # column. Against the oracle on the whole tensor, and stable run to run.
    gen = torch.Generator(device=gpu_device).manual_seed(7)
    x = torch.randn(32768, 4096, device=gpu_device, generator=gen).to(torch.bfloat16 if dtype == "bf16" else torch.float32)
    got = U.column_sum(x)
    assert torch.equal(got, U.column_sum(x))
    assert_close(to_np(got), R.column_sum(to_np(x)), 1e-4, 1e-4 * np.sqrt(32768))


@pytest.mark.parametrize("numel", [1, 7, 4096, 1000003])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_elementwise_matches_oracle(gpu_device, numel: int, dtype: str) -> None:
    x = tensor(np.concatenate([RNG.normal(0, 2, numel - 1), [np.nan]]).astype(np.float32), dtype, gpu_device)
    xs = to_np(x)
    for got, ref in (
        (U.relu(x), R.relu(xs, dtype)),
        (U.leaky_relu(x, 0.1), R.leaky_relu(xs, 0.1, dtype)),
        (U.scalar_mul(x, 2.5), R.scalar_mul(xs, 2.5, dtype)),
    ):
        np.testing.assert_array_equal(to_np(got), ref)
