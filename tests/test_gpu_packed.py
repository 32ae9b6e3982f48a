"""Parity of the prepacked-B GEMMs on every packed layout: config 3b (the
4096^3 bf16 GEMM with B pre-packed) at full size against the oracle, the
per-column affine post-op (``matmul_prepacked_b_affine``, scale and shift)
on each layout and kernel path, f32 panels ``[N/P, K, P]`` read in place, and
the benchmarks' panel-major f32 product (``matmul_packed_b_f32`` with
``unpack_panel_major``, benchmarks/helion_block_packed_f32_repro.py:48-87).

Tolerances: bf16-in / f32-accumulate rtol 1e-2 plus an atol scaled by
sqrt(K); f32 rtol 1e-4 (the f32 repro's own check is rtol = atol = 1e-4,
helion_block_packed_f32_repro.py:117-118).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import helion_mlir_utils as U
import hmx_workloads as W
from oracle import restate as R
from tests.helpers import assert_close, bf16_gemm_atol, max_rel_error, tensor, tile_rows, to_np

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(11)


def _check(got: np.ndarray, ref: np.ndarray, k: int, a: np.ndarray, b: np.ndarray, dtype: str) -> None:
    if dtype == "f32":
        assert_close(got, ref, 1e-4, 1e-5 * np.sqrt(k) * max(1.0, float(np.abs(ref).max()) * 1e-2))
    else:
        assert_close(got, ref, 1e-2, bf16_gemm_atol(k, a, b))


def _packs(b: torch.Tensor, dtype: str) -> dict[str, torch.Tensor]:
    """B [K, N] in each packed layout the dtype takes."""
    bt = b.t().contiguous()
    out = {"blocked": U.pack_b_blocked(b)}
    for panel in (64, 256):
        if b.shape[1] % panel == 0:  # pack_b_panels takes whole panels
            out[f"panels{panel}"] = U.pack_b_panels(b, panel)
    if dtype == "bf16":
        out["blocked_vnni"] = U.pack_b_blocked_vnni(b)
        out["vnni64"] = U.pack_b_vnni_t(bt, 64)
        out["vnni256"] = U.pack_b_vnni_t(bt, 256)
    return out


# ---------------------------------------------------------------------------
# Config 3b at full size: each packed layout against the oracle on rows from
# every 128-row band (every tile), and bit-equal to the plain kernel over the
# whole product.


@pytest.mark.parametrize("layout", ["blocked_vnni", "vnni256", "panels256", "blocked"])
def test_config3b_full_size_each_layout(gpu_device, layout: str) -> None:
    cfg = W.config3()
    a, b = cfg["a"].to(gpu_device), cfg["b"].to(gpu_device)
    packed = _packs(b, "bf16")[layout]
    got = U.matmul_prepacked_b(a, packed, 4096)
    torch.cuda.synchronize()
    rows = tile_rows(RNG, 4096)
    idx = torch.from_numpy(rows)
    a_rows = to_np(cfg["a"][idx])
    ref = R.matmul(a_rows, to_np(cfg["b"]), out="bf16")
    _check(to_np(got[idx.to(gpu_device)]), ref, 4096, a_rows, to_np(cfg["b"]), "bf16")
    assert torch.equal(got, U.matmul(a, b))


# ---------------------------------------------------------------------------
# The affine post-op on each packed layout: (a @ B + bias) * scale + shift and
# an activation, through matmul_prepacked_b_affine and through
# matmul_prepacked_b's scale/shift. Shapes: whole 256 x 256 tiles with K in
# whole 64-element stages (direct-to-LDS kernel), ragged tiles and K
# (register-staged kernel), and a prepared call.

AFFINE_SHAPES = [(512, 320, 768), (70, 96, 130), (33, 64, 256)]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("mkn", AFFINE_SHAPES)
def test_prepacked_affine_every_layout(gpu_device, dtype: str, mkn) -> None:
    m, k, n = mkn
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.normal(0, 1, (k, n)).astype(np.float32), dtype, gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), dtype, gpu_device)
    scale = tensor(RNG.uniform(0.5, 2.0, n).astype(np.float32), dtype, gpu_device)
    shift = tensor(RNG.normal(0, 1, n).astype(np.float32), dtype, gpu_device)
    an, bn = to_np(a), to_np(b)
    ref = R.matmul(an, bn, bias=to_np(bias), scale=to_np(scale), shift=to_np(shift), act="silu", out=dtype)
    ref_scalar = R.matmul(an, bn, bias=to_np(bias), scale=np.float32(1.5), act="relu", out=dtype)
    for packed in _packs(b, dtype).values():
        got = U.matmul_prepacked_b_affine(a, packed, n, bias, scale, shift, F.silu)
        _check(to_np(got), ref, k, an, bn, dtype)
        got = U.matmul_prepacked_b(a, packed, n, bias, F.silu, scale=scale, shift=shift)
        _check(to_np(got), ref, k, an, bn, dtype)
        # a [1] scale broadcast over the columns, no shift
        got = U.matmul_prepacked_b_affine(a, packed, n, bias, torch.tensor([1.5], device=gpu_device), None,
                                          torch.relu)
        _check(to_np(got), ref_scalar, k, an, bn, dtype)
        call = U.prepacked_b_call(a, packed, n, bias, F.silu, scale, shift)
        _check(to_np(call(a)), ref, k, an, bn, dtype)


def test_linear_affine_matches_prepacked_affine(gpu_device) -> None:
    # linear_affine's cached call and the packed-layout affine GEMM agree.
    m, k, n = 64, 256, 384
    layer = torch.nn.Linear(k, n, device=gpu_device, dtype=torch.bfloat16)
    x = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    post_scale = tensor(RNG.uniform(0.5, 2.0, n).astype(np.float32), "bf16", gpu_device)
    post_bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    y, _ = U.linear_affine(x, layer, post_scale, post_bias, F.silu)
    packed = U.pack_b_vnni_t(layer.weight.detach(), 64)
    z = U.matmul_prepacked_b_affine(x, packed, n, layer.bias.detach(), post_scale, post_bias, F.silu)
    ref = R.matmul(to_np(x), to_np(layer.weight), False, True, to_np(layer.bias), to_np(post_scale),
                   to_np(post_bias), "silu", out="bf16")
    _check(to_np(y), ref, k, to_np(x), to_np(layer.weight), "bf16")
    _check(to_np(z), ref, k, to_np(x), to_np(layer.weight), "bf16")


# ---------------------------------------------------------------------------
# f32 panels [N/P, K, P] and the panel-major product of the f32 repro.


@pytest.mark.parametrize("mkn", [(96, 192, 256), (128, 128, 128), (70, 130, 192), (512, 256, 512)])
@pytest.mark.parametrize("panel", [32, 64])
def test_f32_bench_panels_read_in_place(gpu_device, mkn, panel: int) -> None:
    m, k, n = mkn
    a = tensor(RNG.uniform(-1, 1, (m, k)).astype(np.float32), "f32", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (k, n)).astype(np.float32), "f32", gpu_device)
    packed = U.pack_b_panels(b, panel)
    np.testing.assert_array_equal(to_np(packed), R.pack_b_panels(to_np(b), panel))
    got = to_np(U.matmul_prepacked_b(a, packed, n))
    ref = R.matmul(to_np(a), to_np(b), out="f32")
    _check(got, ref, k, to_np(a), to_np(b), "f32")


@pytest.mark.parametrize("size", [128, 512])
@pytest.mark.parametrize(("block_n", "dtype"), [(32, "f32"), (64, "f32"), (32, "bf16")])
def test_matmul_packed_b_f32_repro(gpu_device, size: int, block_n: int, dtype: str) -> None:
    # The repro's flow: b3 = b.view(K, N/BN, BN); pack; the panel-major
    # product; unpack; compare with a @ b at rtol = atol = 1e-4 (f32).
    a = tensor(RNG.standard_normal((size, size)).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.standard_normal((size, size)).astype(np.float32), dtype, gpu_device)
    b3 = b.view(size, size // block_n, block_n).contiguous()
    packed = U.pack_b_panels_f32(b3)
    assert torch.equal(packed, b3.permute(1, 0, 2).contiguous())
    panel_out = U.matmul_packed_b_f32(a, packed)
    assert panel_out.shape == (size // block_n, size, block_n) and panel_out.dtype == torch.float32
    result = to_np(U.unpack_panel_major(panel_out))
    exact = R.matmul(to_np(a), to_np(b), out="f32")
    if dtype == "f32":
        np.testing.assert_allclose(result, exact, rtol=1e-4, atol=1e-4)
    else:
        assert max_rel_error(result, exact) < 1e-5  # f32 output of bf16 inputs: f32 accumulation
    # the benchmark module's own names
    assert torch.equal(U.block_pack.pack_b(b, block_n), packed)
    assert torch.equal(U.block_pack.pack_a(a, 32), U.block_pack.pack_a_panels(a.view(size, size // 32, 32)))
