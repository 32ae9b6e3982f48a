"""Empty operands on every entry point: shapes and values as torch gives them
(an empty contraction is the epilogue of zeros, an empty row sum is zero), and
no kernel launch for an empty output."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import helion_mlir_utils as U

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_matmul_empty_operands(gpu_device, dtype) -> None:
    a = torch.randn(0, 5, device=gpu_device, dtype=dtype)
    b = torch.randn(5, 7, device=gpu_device, dtype=dtype)
    assert U.matmul(a, b).shape == (0, 7)
    assert U.matmul(torch.randn(3, 5, device=gpu_device, dtype=dtype), b[:, :0]).shape == (3, 0)
    # K = 0: every output is epilogue(bias).
    bias = torch.randn(4, device=gpu_device, dtype=dtype)
    got = U.matmul(torch.randn(3, 0, device=gpu_device, dtype=dtype),
                   torch.randn(0, 4, device=gpu_device, dtype=dtype), bias=bias, epilogue=F.silu)
    want = F.silu(bias.float()).to(dtype).expand(3, 4)
    assert got.shape == (3, 4)
    # SiLU in f32 on the kernel's accumulator, rounded once (a last-bit
    # difference to torch's exp).
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(got.cpu().float(), want.cpu().float(), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bmm_empty_operands(gpu_device, dtype) -> None:
    assert U.bmm(torch.randn(0, 3, 4, device=gpu_device, dtype=dtype),
                 torch.randn(0, 4, 5, device=gpu_device, dtype=dtype)).shape == (0, 3, 5)
    got = U.bmm(torch.randn(2, 3, 0, device=gpu_device, dtype=dtype),
                torch.randn(2, 0, 5, device=gpu_device, dtype=dtype))
    assert got.shape == (2, 3, 5) and bool((got == 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_row_ops_empty_operands(gpu_device, dtype) -> None:
    x = torch.randn(0, 16, device=gpu_device, dtype=dtype)
    w = torch.rand(16, device=gpu_device, dtype=dtype) + 0.5
    assert U.softmax(x).shape == (0, 16)
    assert U.rms_norm(x, w, 1e-6).shape == (0, 16)
    assert U.group_norm(x, 4, w, w, 1e-5).shape == (0, 16)
    assert U.layer_norm(x, w, w, 1e-5).shape == (0, 16)
    assert U.row_sum(x).shape == (0, 1)
    cols = U.column_sum(x)
    assert cols.shape == (16,) and bool((cols == 0).all())
    wide = torch.randn(4, 0, device=gpu_device, dtype=dtype)
    sums = U.row_sum(wide)
    assert sums.shape == (4, 1) and bool((sums == 0).all())
    dots = U.row_dot(wide, torch.randn(0, device=gpu_device))
    assert dots.shape == (4, 1) and bool((dots == 0).all())
    assert U.matvec(torch.randn(0, 8, device=gpu_device, dtype=dtype),
                    torch.randn(8, 1, device=gpu_device, dtype=dtype)).shape == (0, 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_elementwise_empty(gpu_device, dtype) -> None:
    x = torch.randn(0, 3, device=gpu_device, dtype=dtype)
    for y in (U.relu(x), U.leaky_relu(x, 0.1), U.scalar_mul(x, 2.0)):
        assert y.shape == (0, 3) and y.dtype == dtype
