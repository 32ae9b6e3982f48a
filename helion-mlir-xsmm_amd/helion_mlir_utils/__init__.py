"""Hot-path kernels of the Helion ``mlir`` backend, on the gfx950 ``gpu`` target.

The entry points and signatures are those of the reference's
``helion_mlir_utils`` (``helion_mlir_utils/__init__.py:5-69``); tensors on a
ROCm device run hand-written gfx950 kernels through ``libhmx.so``. New here:
``rms_norm``, ``layer_norm``, ``Activation`` epilogues, epilogue programs
(:func:`compile_epilogue`: any elementwise callable, fused), ``out_dtype`` of
``matmul``/``bmm``, and the benchmarks' panel packers and panel-major
product (:mod:`.block_pack`).
"""

from __future__ import annotations

from . import block_pack
from . import _gpu
from ._gpu import Activation, register_epilogue
from ._program import EpilogueProgram, compile_epilogue
from .block_pack import matmul_packed_b_f32, pack_b_panels_f32, unpack_panel_major
from .elementwise import leaky_relu, relu, scalar_mul
from .heuristics import tall_output_tiles, vnni_panel, whole_row_tiles
from .kernels import per_config
from .linear import (
    CACHE_PREPACKED_WEIGHTS_ENV,
    AffineLinearCache,
    LinearCache,
    cache_prepacked_weights,
    linear,
    linear_affine,
)
from .matmul import (
    bmm,
    gemm_plan,
    identity_epilogue,
    matmul,
    matmul_prepacked_b,
    matmul_prepacked_b_affine,
    pack_a_blocked,
    pack_a_blocked_t,
    pack_a_panels,
    pack_b_blocked,
    pack_b_blocked_t,
    pack_b_blocked_vnni,
    pack_b_blocked_vnni_t,
    pack_b_panels,
    pack_b_vnni_t,
    pad_2d,
    prepacked_b_call,
    supports,
)
from .normalization import GroupNormEpilogue, group_norm, layer_norm, rms_norm, softmax
from .reduction import column_sum, matvec, row_dot, row_sum, supports_matvec

__all__ = [
    "CACHE_PREPACKED_WEIGHTS_ENV",
    "Activation",
    "AffineLinearCache",
    "EpilogueProgram",
    "GroupNormEpilogue",
    "LinearCache",
    "bmm",
    "cache_prepacked_weights",
    "column_sum",
    "compile_epilogue",
    "gemm_plan",
    "group_norm",
    "identity_epilogue",
    "layer_norm",
    "leaky_relu",
    "linear",
    "linear_affine",
    "matmul",
    "matmul_prepacked_b",
    "matmul_prepacked_b_affine",
    "matmul_packed_b_f32",
    "matvec",
    "pack_a_blocked",
    "pack_a_blocked_t",
    "pack_a_panels",
    "pack_b_blocked",
    "pack_b_blocked_t",
    "pack_b_blocked_vnni",
    "pack_b_blocked_vnni_t",
    "pack_b_panels",
    "pack_b_panels_f32",
    "pack_b_vnni_t",
    "pad_2d",
    "per_config",
    "prepacked_b_call",
    "register_epilogue",
    "relu",
    "rms_norm",
    "row_dot",
    "row_sum",
    "scalar_mul",
    "softmax",
    "supports",
    "supports_matvec",
    "tall_output_tiles",
    "unpack_panel_major",
    "vnni_panel",
    "whole_row_tiles",
]
