"""``nn.Linear`` on the gpu target: the weight is prepared once and its launch
kept for reuse.

Interface of the reference's ``helion_mlir_utils/linear.py`` (``linear``
97-180, ``linear_affine`` 183-261): the same functions, arguments, cache
types and environment switch, so callers hold and pass caches unchanged.

How it works here. A call is one GEMM launch with the bias, the optional
per-column affine post-op and the activation fused. What can be prepared
ahead is:

* the weight in the layout the kernel reads -- ``[N, K]`` row-major, which is
  what ``nn.Linear.weight`` already is (the MFMA B fragment is 8 consecutive
  K values), kept contiguous in the input's dtype; or, when the caller names
  ``panel``, the reference's VNNI panels (``pack_b_vnni_t``), read in place;
* the biases, summed once into one vector;
* the launch itself (plan, workspace size, bound argument block): a
  :class:`~helion_mlir_backend.PreparedCall`, so a call is a shape check and
  one native launch.

A cache is valid while the parameters it was made from are unchanged as far
as their data pointers, ``_version`` counters, shapes, dtypes and devices
tell, and the input keeps its dtype, device and row count: in-place updates
and ``load_state_dict`` invalidate it, a write through ``.data`` does not
(pass ``cache=None`` after one).
"""

from __future__ import annotations

import functools
import os
from typing import TYPE_CHECKING, Callable, NamedTuple

import torch

from helion_mlir_backend import prepared_call
from helion_mlir_backend._compiler import native

from ._gpu import epilogue_code, identity_epilogue, is_gpu
from .matmul import GemmLaunch, _vectors, matmul, pack_b_vnni_t, prepacked_b_call

if TYPE_CHECKING:
    from torch import Tensor, nn

__all__ = [
    "CACHE_PREPACKED_WEIGHTS_ENV",
    "AffineLinearCache",
    "LinearCache",
    "cache_prepacked_weights",
    "linear",
    "linear_affine",
]

CACHE_PREPACKED_WEIGHTS_ENV = "HELION_MLIR_CACHE_PREPACKED_WEIGHTS"
_SWITCHED_OFF = frozenset({"0", "false", "no"})


def cache_prepacked_weights() -> bool:
    """False when ``HELION_MLIR_CACHE_PREPACKED_WEIGHTS`` is 0 / false / no:
    then every call prepares the weight again and returns no cache."""
    return os.environ.get(CACHE_PREPACKED_WEIGHTS_ENV, "").strip().lower() not in _SWITCHED_OFF


class LinearCache(NamedTuple):
    key: tuple
    packed_weight: Tensor
    bias: Tensor | None
    out_features: int
    call: tuple | None = None
    """``(epilogue, prepared call)`` made for the last epilogue used."""


class AffineLinearCache(NamedTuple):
    key: tuple
    packed_weight: Tensor
    bias: Tensor | None
    post_scale: Tensor
    post_bias: Tensor | None
    out_features: int
    call: tuple | None = None


def _fingerprint(t: Tensor | None) -> tuple | None:
    """What identifies a parameter's contents without reading them."""
    if t is None:
        return None
    return (t.data_ptr(), t._version, tuple(t.shape), t.dtype, t.device)


def _as_input(x: Tensor, t: Tensor | None) -> Tensor | None:
    """``t`` detached, in ``x``'s dtype, on ``x``'s device."""
    return None if t is None else t.detach().to(dtype=x.dtype, device=x.device)


def _one_bias(parts: tuple[Tensor, ...], x: Tensor) -> Tensor | None:
    """The given bias vectors added left to right in ``x``'s dtype (each sum
    rounded to it, as adding the tensors one by one would)."""
    if not parts:
        return None
    return functools.reduce(torch.add, (_as_input(x, p) for p in parts))


def _kernel_weight(weight: Tensor, panel: int | None) -> Tensor:
    """The weight as the kernel will read it: ``[N, K]`` contiguous, or VNNI
    panels of ``panel`` columns when asked for (bf16, even K)."""
    if panel is not None and weight.dtype == torch.bfloat16 and weight.shape[1] % 2 == 0:
        return pack_b_vnni_t(weight, panel)
    return weight.contiguous()


def _row_tiles(x: Tensor, n: int, k: int, whole_rows: bool, panel: int | None) -> tuple[int, int] | None:
    """The ``(rows, columns)`` whole-row tiles a ``whole_rows`` call asks for
    (bf16, even K: :func:`~.heuristics.whole_row_tiles`), else None."""
    if not whole_rows or x.dtype != torch.bfloat16 or k % 2 or x.dim() != 2:
        return None
    from .heuristics import whole_row_tiles

    return whole_row_tiles(int(x.shape[0]), n, panel)


def _launcher(
    x: Tensor,
    weight: Tensor,
    n: int,
    bias: Tensor | None,
    epilogue: Callable[[Tensor], Tensor],
    scale: Tensor | None = None,
    shift: Tensor | None = None,
    tile_m: int | None = None,
) -> Callable[[Tensor], Tensor]:
    """A prepared ``epilogue((x @ W^T + bias) * scale + shift)`` for inputs of
    ``x``'s shape, dtype and device (``tile_m``: the workgroup rows asked
    for); any other input goes through the general entry point, which checks
    it."""
    if weight.dim() != 2:  # VNNI panels
        return prepacked_b_call(x, weight, n, bias, epilogue, scale, shift, tile_m=tile_m)

    def general(a: Tensor) -> Tensor:
        return matmul(a, weight, trans_b=True, bias=bias, epilogue=epilogue, scale=scale, shift=shift)

    m, k = (int(d) for d in x.shape) if x.dim() == 2 else (0, 0)
    plain = (x.dim() == 2 and is_gpu(x, weight) and x.dtype == weight.dtype and m > 0 and n > 0 and k > 0
             and int(weight.shape[1]) == k)
    if not plain:
        return general
    vec_bias, vec_scale, vec_shift, vec_dtype = _vectors(bias, scale, shift, n, x)
    launch = GemmLaunch(
        native.dtype_code(x.dtype), x.dtype, x.device, (m, n), k, False, k, native.B_TRANS, 0, 0, m, n, k,
        bias=vec_bias, scale=vec_scale, shift=vec_shift, vec_dtype=vec_dtype, epilogue=epilogue_code(epilogue),
        tiles=(tile_m, 0, 0) if tile_m else None,
    )
    prepared = prepared_call(launch, (x, weight), [0], general)
    return general if prepared is None else prepared


def _with_call(cache, epilogue, make: Callable[[], Callable[[Tensor], Tensor]]):
    """``(call, cache)``: the cache's prepared call if it was made for this
    epilogue, else a new one, kept in the returned cache."""
    held = cache.call
    if held is not None and held[0] is epilogue:
        return held[1], cache
    call = make()
    return call, cache._replace(call=(epilogue, call))


def linear(
    x: Tensor,
    layer: nn.Linear,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    cache: LinearCache | None = None,
    biases: tuple[Tensor, ...] | None = None,
    panel: int | None = None,
    whole_rows: bool = False,
) -> tuple[Tensor, LinearCache | None]:
    """``(epilogue(x @ layer.weight.T + bias), cache)`` (``linear.py:97-180``).

    ``biases`` replaces ``layer.bias`` by the sum of the given vectors.
    ``panel`` keeps a bf16 weight as VNNI panels of that many columns.
    ``whole_rows`` (bf16, even ``in_features``, cached weights) takes the
    reference's whole-row tiles (``linear.py:88-94,156-171``): the weight is
    kept as VNNI panels of the tile's columns and the launch asks for the
    tile's rows (:func:`~.heuristics.whole_row_tiles`, the GPU tile table's
    answer); shapes it cannot tile keep the default launch. The results are
    those of the default launch. The flag is part of the cache key, as in the
    reference."""
    parts = tuple(biases) if biases is not None else (() if layer.bias is None else (layer.bias,))
    if not cache_prepacked_weights():
        y = matmul(x, _as_input(x, layer.weight), trans_b=True, bias=_one_bias(parts, x), epilogue=epilogue)
        return y, None
    key = (_fingerprint(layer.weight), tuple(_fingerprint(p) for p in parts), x.dtype, x.device,
           x.shape[0], panel, bool(whole_rows))
    tiles = _row_tiles(x, int(layer.out_features), int(layer.in_features), whole_rows, panel)
    if cache is None or cache.key != key:
        cache = LinearCache(key, _kernel_weight(_as_input(x, layer.weight), tiles[1] if tiles else panel),
                            _one_bias(parts, x), int(layer.out_features))
    fresh = cache
    call, cache = _with_call(
        cache, epilogue,
        lambda: _launcher(x, fresh.packed_weight, fresh.out_features, fresh.bias, epilogue,
                          tile_m=tiles[0] if tiles else None),
    )
    return call(x), cache


def linear_affine(
    x: Tensor,
    layer: nn.Linear,
    post_scale: Tensor,
    post_bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    cache: AffineLinearCache | None = None,
) -> tuple[Tensor, AffineLinearCache | None]:
    """``(epilogue(linear(x) * post_scale + post_bias), cache)``;
    ``post_scale`` and ``post_bias`` are ``[1]`` or ``[out_features]``
    (``linear.py:183-261``). Cached like :func:`linear`."""
    if not cache_prepacked_weights():
        y = matmul(x, _as_input(x, layer.weight), trans_b=True, bias=_as_input(x, layer.bias), epilogue=epilogue,
                   scale=_as_input(x, post_scale), shift=_as_input(x, post_bias))
        return y, None
    key = (_fingerprint(layer.weight), _fingerprint(layer.bias), _fingerprint(post_scale),
           _fingerprint(post_bias), x.dtype, x.device, x.shape[0])
    if cache is None or cache.key != key:
        cache = AffineLinearCache(key, _kernel_weight(_as_input(x, layer.weight), None), _as_input(x, layer.bias),
                                  _as_input(x, post_scale), _as_input(x, post_bias), int(layer.out_features))
    fresh = cache
    call, cache = _with_call(
        cache, epilogue,
        lambda: _launcher(x, fresh.packed_weight, fresh.out_features, fresh.bias, epilogue, fresh.post_scale,
                          fresh.post_bias),
    )
    return call(x), cache
