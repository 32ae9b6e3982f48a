"""``nn.Linear`` on the gpu target, with the weight prepared once and cached.

Reference: ``helion_mlir_utils/linear.py`` (``linear`` 97-180, ``linear_affine``
183-261). The cache is keyed, as there, by the parameters' data pointers,
``_version``, shapes, dtypes and devices plus the input's dtype, device and
rows: in-place updates and ``load_state_dict`` are seen, a change through
``.data`` is not.

On gfx950 the GEMM kernel's preferred B layout is ``[N, K]`` row-major (each
MFMA operand fragment is 8 consecutive K values), which is what
``nn.Linear.weight`` already is: "prepacking" keeps the weight contiguous in
the input's dtype. ``panel`` asks for the reference's VNNI panels
(:func:`~.matmul.pack_b_vnni_t`) instead, which the kernel reads in place too.
The cached call is a :class:`~helion_mlir_backend.PreparedCall`: per call, a
shape check and one launch.
"""

from __future__ import annotations

import os
from typing import TYPE_CHECKING, Callable, NamedTuple

import torch

from helion_mlir_backend import output_pool, prepared_call
from helion_mlir_backend._compiler import native

from ._gpu import epilogue_code, identity_epilogue, is_gpu
from .matmul import GemmLaunch, _vectors, matmul, matmul_prepacked_b, pack_b_vnni_t, prepacked_b_call

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


def cache_prepacked_weights() -> bool:
    """Whether constant weights are prepared once and reused (the default);
    ``HELION_MLIR_CACHE_PREPACKED_WEIGHTS=0`` prepares them on every call."""
    value = os.environ.get(CACHE_PREPACKED_WEIGHTS_ENV)
    return value is None or value.strip().lower() not in ("0", "false", "no")


class LinearCache(NamedTuple):
    key: tuple
    packed_weight: Tensor
    bias: Tensor | None
    out_features: int
    call: tuple | None = None
    """``(epilogue, prepared call)`` of the last call."""


class AffineLinearCache(NamedTuple):
    key: tuple
    packed_weight: Tensor
    bias: Tensor | None
    post_scale: Tensor
    post_bias: Tensor | None
    out_features: int
    call: tuple | None = None


def _parameter_key(parameter: Tensor | None) -> tuple | None:
    if parameter is None:
        return None
    return (
        parameter.data_ptr(),
        parameter._version,
        tuple(parameter.shape),
        parameter.dtype,
        parameter.device,
    )


def _combine_biases(biases: tuple[Tensor, ...], x: Tensor) -> Tensor | None:
    if not biases:
        return None
    bias = biases[0].to(dtype=x.dtype, device=x.device)
    for extra_bias in biases[1:]:
        bias = bias + extra_bias.to(dtype=x.dtype, device=x.device)
    return bias


def _pack_weight(weight: Tensor, panel: int | None) -> Tensor:
    """The weight as the kernel reads it: ``[N, K]`` row-major, or VNNI panels
    of ``panel`` columns when asked (bf16, even K)."""
    if panel is not None and weight.dtype == torch.bfloat16 and not weight.shape[1] % 2:
        return pack_b_vnni_t(weight, panel)
    return weight.contiguous()


def _weight_call(
    x: Tensor,
    packed: Tensor,
    n: int,
    bias: Tensor | None,
    epilogue: Callable[[Tensor], Tensor],
    scale: Tensor | None = None,
    shift: Tensor | None = None,
) -> Callable[[Tensor], Tensor]:
    """A prepared ``epilogue((x @ W^T + bias) * scale + shift)`` for inputs
    like ``x``."""
    if packed.dim() != 2:
        return prepacked_b_call(x, packed, n, bias, epilogue, scale, shift)

    def general(a: Tensor) -> Tensor:
        return matmul(a, packed, trans_b=True, bias=bias, epilogue=epilogue, scale=scale, shift=shift)

    if x.dim() != 2 or not is_gpu(x, packed) or x.dtype != packed.dtype:
        return general
    m, k = map(int, x.shape)
    if m == 0 or n == 0 or k == 0 or int(packed.shape[1]) != k:
        return general
    code = epilogue_code(epilogue)
    bias_, scale_, shift_, vec_dtype = _vectors(bias, scale, shift, n, x)
    dtype, device = x.dtype, x.device

    launch = GemmLaunch(
        native.dtype_code(dtype), dtype, device, (m, n), k, False, k, native.B_TRANS, 0, 0, m, n, k,
        bias=bias_, scale=scale_, shift=shift_, vec_dtype=vec_dtype, epilogue=code,
    )
    return prepared_call(lambda a: launch.run(a, packed), [x], general)


def linear(
    x: Tensor,
    layer: nn.Linear,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    cache: LinearCache | None = None,
    biases: tuple[Tensor, ...] | None = None,
    panel: int | None = None,
    whole_rows: bool = False,
) -> tuple[Tensor, LinearCache | None]:
    """``epilogue(x @ layer.weight.T + bias)`` and the cache to pass next time
    (``linear.py:97-180``). ``biases`` replaces ``layer.bias`` by the sum of
    the given vectors. ``panel`` packs a bf16 weight into VNNI panels of that
    width; ``whole_rows`` is accepted for the reference's API (on the GPU a
    row of output tiles always runs on one XCD)."""
    del whole_rows
    if biases is None:
        bias = layer.bias
        source_biases = () if bias is None else (bias,)
    else:
        source_biases = biases
    if not cache_prepacked_weights():
        weight = layer.weight.detach().to(dtype=x.dtype, device=x.device)
        return (
            matmul(x, weight, trans_b=True, bias=_combine_biases(source_biases, x), epilogue=epilogue),
            None,
        )
    key = (
        _parameter_key(layer.weight),
        tuple(map(_parameter_key, source_biases)),
        x.dtype,
        x.device,
        x.shape[0],
        panel,
    )
    if cache is None or cache.key != key:
        weight = layer.weight.detach().to(dtype=x.dtype, device=x.device)
        cache = LinearCache(
            key,
            _pack_weight(weight, panel),
            _combine_biases(tuple(b.detach() for b in source_biases), x),
            int(layer.out_features),
        )
    prepared = cache.call
    if prepared is None or prepared[0] is not epilogue:
        call = _weight_call(x, cache.packed_weight, cache.out_features, cache.bias, epilogue)
        cache = cache._replace(call=(epilogue, call))
    else:
        call = prepared[1]
    return call(x), cache


def linear_affine(
    x: Tensor,
    layer: nn.Linear,
    post_scale: Tensor,
    post_bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    cache: AffineLinearCache | None = None,
) -> tuple[Tensor, AffineLinearCache | None]:
    """``epilogue(linear(x) * post_scale + post_bias)``; ``post_scale`` and
    ``post_bias`` are ``[1]`` or ``[out_features]`` (``linear.py:183-261``).
    Cached like :func:`linear`."""
    use_cache = cache_prepacked_weights()
    key = (
        _parameter_key(layer.weight),
        _parameter_key(layer.bias),
        _parameter_key(post_scale),
        _parameter_key(post_bias),
        x.dtype,
        x.device,
        x.shape[0],
    )
    if not use_cache or cache is None or cache.key != key:
        weight = layer.weight.detach().to(dtype=x.dtype, device=x.device)
        bias = None if layer.bias is None else layer.bias.detach().to(dtype=x.dtype, device=x.device)
        cache = AffineLinearCache(
            key,
            _pack_weight(weight, None),
            bias,
            post_scale.detach().to(dtype=x.dtype, device=x.device),
            None if post_bias is None else post_bias.detach().to(dtype=x.dtype, device=x.device),
            int(layer.out_features),
        )
    if not use_cache:
        result = matmul(x, cache.packed_weight, trans_b=True, bias=cache.bias, epilogue=epilogue,
                        scale=cache.post_scale, shift=cache.post_bias)
        return result, None
    prepared = cache.call
    if prepared is None or prepared[0] is not epilogue:
        call = _weight_call(x, cache.packed_weight, cache.out_features, cache.bias, epilogue,
                            cache.post_scale, cache.post_bias)
        cache = cache._replace(call=(epilogue, call))
    else:
        call = prepared[1]
    return call(x), cache
