"""The block-packed operands of the reference's benchmarks, on the gpu target.

The reference keeps these in two benchmark scripts: ``benchmarks/helion_block_pack.py``
(``pack_b_panels`` 40-51, ``pack_a_panels`` 54-62, ``pack_b`` 66-71, ``pack_a``
74-79) and ``benchmarks/helion_block_packed_f32_repro.py`` (``pack_b_panels_f32``
48-58, ``matmul_packed_b_f32`` 61-81, ``unpack_panel_major`` 84-87). Same
names, arguments and layouts here:

* ``[K, N]`` -> ``[N/BN, K, BN]``: panel ``j`` holds every K row of ``BN``
  columns (no K-pair interleave);
* ``[M, K]`` -> ``[K/BK, M, BK]``;
* ``matmul_packed_b_f32(a, packed_b)``: the panel-major product
  ``out[j] = a @ packed_b[j]``, ``[N/BN, M, BN]`` in f32.

The packs are the library's pack kernels (``hmx_pack``). The panel product is
one GEMM launch over the panels as a batch: A shared by every panel (batch
stride 0), panel ``j`` of B read in place as a ``[K, BN]`` row-major matrix,
output panel ``j`` written in place -- the layout is never converted.
"""

from __future__ import annotations

import torch
from torch import Tensor

from helion_mlir_backend import output_pool
from helion_mlir_backend._compiler import native

from ._gpu import SUPPORTED_DTYPES, is_gpu
from .matmul import _launch_gemm
from .matmul import pack_a_panels as _pack_a_panels
from .matmul import pack_b_panels as _pack_b_panels

__all__ = [
    "matmul_packed_b_f32",
    "pack_a",
    "pack_a_panels",
    "pack_b",
    "pack_b_panels",
    "pack_b_panels_f32",
    "unpack_panel_major",
]


def pack_b_panels(b3: Tensor) -> Tensor:
    """``[K, N/BN, BN]`` -> ``[N/BN, K, BN]``, one contiguous panel per column
    block (``helion_block_pack.py:40-51``)."""
    return _pack_b_panels(b3)


def pack_a_panels(a3: Tensor) -> Tensor:
    """``[M, K/BK, BK]`` -> ``[K/BK, M, BK]``, one contiguous panel per K block
    (``helion_block_pack.py:54-62``)."""
    return _pack_a_panels(a3)


def pack_b(b: Tensor, block_n: int) -> Tensor:
    """Pack ``[K, N]`` into ``[N/block_n, K, block_n]`` (``helion_block_pack.py:66-71``)."""
    return _pack_b_panels(b, block_n)


def pack_a(a: Tensor, block_k: int) -> Tensor:
    """Pack ``[M, K]`` into ``[K/block_k, M, block_k]`` (``helion_block_pack.py:74-79``)."""
    return _pack_a_panels(a, block_k)


def pack_b_panels_f32(b3: Tensor) -> Tensor:
    """Pack ``B`` from ``[K, N/BN, BN]`` to ``[N/BN, K, BN]``
    (``helion_block_packed_f32_repro.py:48-58``)."""
    return _pack_b_panels(b3)


def matmul_packed_b_f32(a: Tensor, packed_b: Tensor) -> Tensor:
    """Panel-major ``[N/BN, M, BN]`` f32 output from packed RHS panels:
    ``out[j] = a @ packed_b[j]`` with f32 accumulation
    (``helion_block_packed_f32_repro.py:61-81``)."""
    if a.dim() != 2 or packed_b.dim() != 3:
        raise ValueError(
            f"matmul_packed_b_f32() expects a [M, K] and packed_b [N/BN, K, BN], got "
            f"{tuple(a.shape)} and {tuple(packed_b.shape)}"
        )
    m, k = map(int, a.shape)
    panels, k2, block_n = map(int, packed_b.shape)
    if k != k2:
        raise ValueError(f"matmul dimension mismatch: a has K={k}, packed_b has K={k2}")
    if a.dtype != packed_b.dtype or a.dtype not in SUPPORTED_DTYPES or not is_gpu(a, packed_b) \
            or a.device != packed_b.device:
        raise ValueError(
            f"matmul_packed_b_f32() runs float32/bfloat16 operands on one ROCm device, got "
            f"a {a.dtype} on {a.device}, packed_b {packed_b.dtype} on {packed_b.device}"
        )
    out = output_pool.empty((panels, m, block_n), dtype=torch.float32, device=a.device)
    if panels == 0 or m == 0 or block_n == 0:
        return out
    if k == 0:
        return out.zero_()
    a = a.contiguous()
    packed_b = packed_b.contiguous()
    return _launch_gemm(
        a, k, False, packed_b, block_n, native.B_ROW, 0, 0, out, m, block_n, k,
        batch=panels, stride_a=0, stride_b=k * block_n, stride_c=m * block_n,
    )


def unpack_panel_major(panel_out: Tensor) -> Tensor:
    """``[N/BN, M, BN]`` back to row-major ``[M, N]``
    (``helion_block_packed_f32_repro.py:84-87``)."""
    n_panels, m, block_n = panel_out.shape
    return panel_out.permute(1, 0, 2).contiguous().view(m, n_panels * block_n)
