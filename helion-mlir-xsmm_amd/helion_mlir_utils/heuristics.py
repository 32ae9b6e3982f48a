"""Tile helpers of the reference's API, answered for the gpu target.

The reference's ``vnni_panel``, ``tall_output_tiles`` and ``whole_row_tiles``
(``helion_mlir_utils/matmul.py:1057-1136``) size CPU tiles from
``OMP_NUM_THREADS`` and cache capacities. On gfx950 the same questions -- how
wide a packed panel, which ``block_sizes`` for a GEMM -- are answered by the
GEMM's workgroup tile table (``gemm_plan``), so these return that table's
choices in the reference's return formats.
"""

from __future__ import annotations

import torch

from .matmul import BLOCK_N, gemm_plan

__all__ = ["tall_output_tiles", "vnni_panel", "whole_row_tiles"]


def vnni_panel(m: int, n: int, k: int | None = None) -> int:
    """Columns of :func:`~.matmul.pack_b_vnni_t` panels: the widest of 256,
    128 and 64 dividing ``n`` (the kernel's column tile reads whole panels),
    else 64."""
    del m, k
    for panel in (256, 128, 64):
        if n % panel == 0:
            return panel
    return 64


def tall_output_tiles(m: int, n: int, k: int) -> tuple[int, int, int] | None:
    """``block_sizes`` of :func:`~.matmul.matmul` for ``[m, k] @ [k, n]``: the
    workgroup tile the gpu GEMM picks; ``None`` for shapes the packed layouts
    cannot tile (N or K not whole 32-blocks), as in the reference."""
    if n <= 0 or n % BLOCK_N or k <= 0 or k % (2 * 32):
        return None
    plan = gemm_plan(torch.bfloat16, m, n, k)
    return plan["tile_m"], plan["tile_n"], plan["tile_k"]


def whole_row_tiles(m: int, n: int, panel: int | None = None) -> tuple[int, int] | None:
    """``(rows, columns)`` of output tiles: the gpu GEMM's workgroup tile, with
    ``panel`` columns when given; ``None`` unless the tile divides ``n``."""
    plan = gemm_plan(torch.bfloat16, m, n, 64)
    columns = panel or plan["tile_n"]
    if n % columns:
        return None
    return plan["tile_m"], columns
