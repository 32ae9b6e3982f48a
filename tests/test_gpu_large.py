"""Operands past 2^31 bytes, against the CPU oracle on sampled rows.

The direct-to-LDS GEMM kernels address their operands through buffer
resources with 32-bit offsets: a row-major A or a B [N, K] that spans 2^31
bytes or more is cut into blocks of whole tiles that each span less, one
product per block (bf16 and f32 A, B [N, K] with the skinny kernel and the
256 x 256 tiles, bias/scale/shift offset per block); the register-staged
kernels, whose loads and stores use 64-bit offsets, take what cannot be cut.
The row kernels index rows in 64 bits throughout. These tests run both past
the 32-bit range: the sampled rows include the last ones, whose byte offsets
are past 2^31 (GEMM operands) or 2^32 (row inputs), so an offset truncated to
32 bits would read another row's data. Tolerances as in the other parity tests: rtol 1e-2 plus a sqrt(K)-scaled
atol for bf16 GEMMs, rtol 1e-4 for f32; max-normalised error < 1e-2 for bf16
softmax (the reference's, tests/test_cpu_utils_softmax.py:18-34); one bf16
rounding for RMSNorm; column sums of integers are exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import helion_mlir_utils as U
from oracle import restate as R
from tests.helpers import assert_close, bf16_gemm_atol, max_rel_error, tile_rows, to_np

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(2031)

# 139264 x 8192 bf16 (or 69632 x 8192 f32): 2.28e9 bytes, past 2^31.
BIG_ROWS_BF16, BIG_ROWS_F32, K = 139264, 69632, 8192
# 2^19 + 5 rows of 4096 bf16: 4.29e9 bytes, past 2^32, ragged against every
# rows-per-workgroup count.
ROWS, COLS = (1 << 19) + 5, 4096


def _uniform(shape, dtype, device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.empty(shape, dtype=dtype, device=device).uniform_(-1.0, 1.0, generator=g)


def _with_last(rows: np.ndarray, m: int) -> np.ndarray:
    return np.unique(np.concatenate([rows, np.arange(m - 3, m)]))


def _check(got, ref, k, a, b, dtype):
    if dtype == "f32":
        assert_close(got, ref, 1e-4, 1e-5 * np.sqrt(k) * max(1.0, float(np.abs(ref).max()) * 1e-2))
    else:
        assert_close(got, ref, 1e-2, bf16_gemm_atol(k, a, b))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_matmul_a_past_2gib(gpu_device, dtype: str) -> None:
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    m, n = (BIG_ROWS_BF16, 256) if dtype == "bf16" else (BIG_ROWS_F32, 128)
    a = _uniform((m, K), tdt, gpu_device, 11)
    b = _uniform((K, n), tdt, gpu_device, 12)
    assert a.numel() * a.element_size() > 2**31
    c = U.matmul(a, b)
    torch.cuda.synchronize()
    rows = torch.from_numpy(_with_last(tile_rows(RNG, m, 1), m)).to(gpu_device)
    got, an, bn = to_np(c[rows]), to_np(a[rows]), to_np(b)
    ref = R.matmul(an, bn, out=dtype)
    _check(got, ref, K, an, bn, dtype)
    del a, b, c
    torch.cuda.empty_cache()


@pytest.mark.parametrize("m", [256, 32])
def test_linear_weight_past_2gib(gpu_device, m: int) -> None:
    # B [N, K] (a linear layer's weight) past 2^31 bytes, with bias, scale,
    # shift and SiLU: C's sampled columns (each block of columns reads its own
    # run of the vectors). 32 rows take the skinny kernel.
    n = BIG_ROWS_BF16
    x = _uniform((m, K), torch.bfloat16, gpu_device, 13)
    w = _uniform((n, K), torch.bfloat16, gpu_device, 14)
    bias, scale, shift = (_uniform((n,), torch.bfloat16, gpu_device, 20 + i) for i in range(3))
    assert w.numel() * 2 > 2**31
    c = U.matmul(x, w, trans_b=True, bias=bias, scale=scale, shift=shift, epilogue=F.silu)
    torch.cuda.synchronize()
    cols = torch.from_numpy(_with_last(tile_rows(RNG, n, 1), n)).to(gpu_device)
    got, xn, wn = to_np(c[:, cols]), to_np(x), to_np(w[cols])
    vb, vs, vh = (to_np(v[cols]) for v in (bias, scale, shift))
    ref = R.matmul(xn, wn, False, True, vb, vs, vh, "silu", 0.01, out="bf16")
    _check(got, ref, K, xn, wn, "bf16")
    del x, w, c
    torch.cuda.empty_cache()


@pytest.mark.parametrize("op", ["softmax", "rms_norm"])
def test_rows_past_4gib(gpu_device, op: str) -> None:
    x = _uniform((ROWS, COLS), torch.bfloat16, gpu_device, 15) * 3.0
    assert x.numel() * 2 > 2**32
    rows = torch.from_numpy(_with_last(tile_rows(RNG, ROWS, 1, 1024), ROWS)).to(gpu_device)
    xs = to_np(x[rows])
    if op == "softmax":
        got = to_np(U.softmax(x)[rows])
        assert max_rel_error(got, R.softmax(xs, "bf16")) < 1e-2
    else:
        w = _uniform((COLS,), torch.bfloat16, gpu_device, 16)
        got = to_np(U.rms_norm(x, w, 1e-6)[rows])
        assert_close(got, R.rms_norm(xs, to_np(w), 1e-6, "bf16"), 1e-2, 1e-3)
    del x
    torch.cuda.empty_cache()


def test_column_sum_past_4gib(gpu_device) -> None:
    # Ones, the last row 2 and column 0 of row 0 set to 3: every column sums to
    # ROWS + 1, column 0 to ROWS + 3, exactly (integers below 2^24 in f32).
    x = torch.ones((ROWS, COLS), dtype=torch.bfloat16, device=gpu_device)
    x[-1] = 2.0
    x[0, 0] = 3.0
    got = to_np(U.column_sum(x))
    want = np.full(COLS, ROWS + 1, dtype=np.float32)
    want[0] = ROWS + 3
    np.testing.assert_array_equal(got, want)
    del x
    torch.cuda.empty_cache()
