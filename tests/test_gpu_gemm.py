"""Parity of the gfx950 GEMMs with the CPU oracle: bf16 and f32 ``matmul``
(every transpose, ragged shapes, fused bias/scale/shift/activations), ``bmm``
with deterministic split-K, ``linear`` / ``linear_affine``, the prepacked-B
GEMMs over every packed layout, and the pack kernels (bit-exact).

Tolerances (BASELINE): bf16-in / f32-accumulate rtol 1e-2 plus an atol scaled
by sqrt(K) (``bf16_gemm_atol``); f32 rtol 1e-4, and the reference's own
max-normalised error < 1e-5 for bmm (tests/test_cpu_utils_split_k_bmm.py:15-16).
Full BASELINE sizes are checked against the oracle on rows drawn from every
128-row band (``tile_rows``), over all columns: every output tile is sampled.
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

RNG = np.random.default_rng(7)
ACTS = {"identity": U.identity_epilogue, "relu": torch.relu, "silu": F.silu, "sigmoid": torch.sigmoid,
        "gelu": F.gelu, "gelu_tanh": U.Activation("gelu_tanh"), "tanh": torch.tanh,
        "leaky_relu": U.Activation("leaky_relu", 0.2)}


def _operands(m, n, k, trans_a, trans_b, dtype, device, scale=1.0):
    a = tensor(RNG.normal(0, scale, (k, m) if trans_a else (m, k)).astype(np.float32), dtype, device)
    b = tensor(RNG.normal(0, scale, (n, k) if trans_b else (k, n)).astype(np.float32), dtype, device)
    return a, b


def _check(got, ref, k, a, b, dtype):
    if dtype == "f32":
        assert_close(got, ref, 1e-4, 1e-5 * np.sqrt(k) * max(1.0, float(np.abs(ref).max()) * 1e-2))
    else:
        assert_close(got, ref, 1e-2, bf16_gemm_atol(k, a, b))


@pytest.mark.parametrize("mnk", [(100, 100, 130), (33, 35, 66), (70, 40, 201), (20, 40, 50), (65, 372, 47),
                                 (256, 256, 256), (512, 256, 128), (1, 1, 1), (300, 64, 128), (37, 45, 19),
                                 # M >= 512 with row-major B: B transposed up front (ragged and whole)
                                 (600, 333, 129), (1024, 512, 256)])
@pytest.mark.parametrize(("trans_a", "trans_b"), [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_matmul_matches_oracle(gpu_device, mnk, trans_a, trans_b, dtype) -> None:
    m, n, k = mnk
    a, b = _operands(m, n, k, trans_a, trans_b, dtype, gpu_device)
    got = to_np(U.matmul(a, b, trans_a=trans_a, trans_b=trans_b))
    ref = R.matmul(to_np(a), to_np(b), trans_a, trans_b, out=dtype)
    _check(got, ref, k, to_np(a), to_np(b), dtype)


@pytest.mark.parametrize("act", list(ACTS))
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_matmul_fused_epilogues(gpu_device, act: str, dtype: str) -> None:
    m, n, k = 200, 300, 256
    a, b = _operands(m, n, k, False, True, dtype, gpu_device, 0.2)
    bias, scale, shift = (tensor(RNG.normal(0, 1, n).astype(np.float32), dtype, gpu_device) for _ in range(3))
    got = to_np(U.matmul(a, b, trans_b=True, bias=bias, scale=scale, shift=shift, epilogue=ACTS[act]))
    arg = 0.2 if act == "leaky_relu" else 0.01
    ref = R.matmul(to_np(a), to_np(b), False, True, to_np(bias), to_np(scale), to_np(shift), act, arg, out=dtype)
    _check(got, ref, k, to_np(a), to_np(b), dtype)


def test_matmul_scalar_affine_and_out_dtype(gpu_device) -> None:
    m, n, k = 64, 96, 128
    a, b = _operands(m, n, k, False, False, "bf16", gpu_device)
    scale = torch.tensor([0.5], device=gpu_device, dtype=torch.bfloat16)
    shift = torch.tensor([2.0], device=gpu_device, dtype=torch.bfloat16)
    got = U.matmul(a, b, scale=scale, shift=shift, out_dtype=torch.float32)
    assert got.dtype == torch.float32
    ref = R.matmul(to_np(a), to_np(b), scale=np.float32(0.5), shift=np.float32(2.0))
    assert_close(to_np(got), ref, 1e-5, 1e-4)


def test_matmul_transposed_views_are_read_in_place(gpu_device) -> None:
    a, b = _operands(96, 80, 64, False, False, "bf16", gpu_device)
    at = a.t().contiguous().t()  # a view with strides (1, 96)
    bt = b.t().contiguous().t()
    got = to_np(U.matmul(at, bt))
    ref = R.matmul(to_np(a), to_np(b), out="bf16")
    _check(got, ref, 64, to_np(a), to_np(b), "bf16")


@pytest.mark.parametrize("block_sizes", [(256, 256, 64), (128, 128, 64), (64, 64, 64)])
def test_matmul_block_sizes_pick_the_tile(gpu_device, block_sizes) -> None:
    a, b = _operands(300, 260, 200, False, False, "bf16", gpu_device)
    got = to_np(U.matmul(a, b, block_sizes=block_sizes))
    _check(got, R.matmul(to_np(a), to_np(b), out="bf16"), 200, to_np(a), to_np(b), "bf16")


# Whole 256 x 256 tiles of row-major A run the direct-to-LDS kernel, which
# reads B either K-contiguous or row-major (through transposing LDS reads);
# its register epilogue covers identity / ReLU / SiLU into bf16 or f32.
@pytest.mark.parametrize("act", ["identity", "relu", "silu"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("trans_b", [False, True])
def test_matmul_whole_tiles_direct_to_lds(gpu_device, act, out_dtype, trans_b) -> None:
    m, n, k = 512, 768, 320
    a, b = _operands(m, n, k, False, trans_b, "bf16", gpu_device, 0.3)
    bias, scale, shift = (tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device) for _ in range(3))
    got = U.matmul(a, b, trans_b=trans_b, bias=bias, scale=scale, shift=shift, epilogue=ACTS[act],
                   block_sizes=(256, 256, 64), out_dtype=out_dtype)
    out = "bf16" if out_dtype == torch.bfloat16 else "f32"
    ref = R.matmul(to_np(a), to_np(b), False, trans_b, to_np(bias), to_np(scale), to_np(shift), act, out=out)
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


# Ragged M and N with K in whole 32- or 64-element stages: the direct-to-LDS
# kernels with the guarded edge epilogue (tiles that cross M or N).
@pytest.mark.parametrize("mnk", [(300, 520, 256), (1000, 704, 320), (100, 1000, 512), (520, 260, 96), (257, 255, 64),
                                 (640, 392, 128)])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize(("act", "out_dtype"), [("identity", torch.bfloat16), ("silu", torch.float32),
                                                ("relu", torch.bfloat16)])
@pytest.mark.parametrize("tiles", [(256, 256, 64), (128, 128, 64)])
def test_matmul_ragged_direct_to_lds(gpu_device, mnk, trans_b, act, out_dtype, tiles) -> None:
    # 256 x 256 tiles: B [N, K] or [K, N] read in place; 128 x 128 tiles: B
    # [N, K] (row-major B of 512 rows or more is transposed up front).
    m, n, k = mnk
    a, b = _operands(m, n, k, False, trans_b, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    got = U.matmul(a, b, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype, block_sizes=tiles)
    out = "bf16" if out_dtype == torch.bfloat16 else "f32"
    ref = R.matmul(to_np(a), to_np(b), False, trans_b, to_np(bias), act=act, out=out)
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


@pytest.mark.parametrize(("m", "n", "k"), [(1900, 2000, 1024), (2000, 1960, 2048)])
@pytest.mark.parametrize(("act", "out_dtype"), [("identity", torch.bfloat16), ("silu", torch.bfloat16),
                                                ("relu", torch.float32)])
def test_matmul_ragged_128_tiles_one_round(gpu_device, m, n, k, act, out_dtype) -> None:
    # Ragged 128 x 128 tiles, one round (at most a tile per CU), 16 or more K
    # stages and no split: the 16x16x32 kernel with four LDS stages, bf16 C
    # leaving through each wave's own staging region (C rows of N = 2000 or
    # 1960 bf16 are 16-byte aligned, which that kernel needs for bf16 C).
    plan = U.gemm_plan(torch.bfloat16, m, n, k, trans_b=True, block_sizes=(128, 128, 64))
    assert plan["splits"] <= 1 and (plan["tile_m"], plan["tile_n"]) == (128, 128)
    assert -(-m // 128) * -(-n // 128) <= 256
    a, b = _operands(m, n, k, False, True, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    got = U.matmul(a, b, trans_b=True, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype, block_sizes=(128, 128, 64))
    out = "bf16" if out_dtype == torch.bfloat16 else "f32"
    ref = R.matmul(to_np(a), to_np(b), False, True, to_np(bias), act=act, out=out)
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


@pytest.mark.parametrize("trans_b", [False, True])
def test_matmul_ragged_large(gpu_device, trans_b) -> None:
    # 16 x 16 tiles of 256 x 256, the last row and column of tiles ragged
    # (4000 = 15 * 256 + 160), chosen by the planner itself.
    m, n, k = 4000, 4000, 256
    a, b = _operands(m, n, k, False, trans_b, "bf16", gpu_device, 0.3)
    c = U.matmul(a, b, trans_b=trans_b)
    rows = np.concatenate([np.arange(0, 8), np.arange(3830, 3850), np.arange(3990, 4000)])
    an, bn = to_np(a)[rows], to_np(b)
    _check(to_np(c)[rows], R.matmul(an, bn, False, trans_b, out="bf16"), k, an, bn, "bf16")


def test_matmul_ragged_row_major_b_view(gpu_device) -> None:
    # N = 203 of a [128, 208] buffer: row-major B whose last column chunk
    # straddles N (the clamped chunk reads inside the wider rows).
    a = tensor(RNG.normal(0, 0.3, (300, 128)).astype(np.float32), "bf16", gpu_device)
    wide = tensor(RNG.normal(0, 0.3, (128, 208)).astype(np.float32), "bf16", gpu_device)
    b = wide[:, :203]
    got = to_np(U.matmul(a, b))
    ref = R.matmul(to_np(a), to_np(b), out="bf16")
    _check(got, ref, 128, to_np(a), to_np(b), "bf16")


def test_bmm_ragged_split_k_direct_to_lds(gpu_device) -> None:
    a = tensor(RNG.uniform(-1, 1, (2, 300, 4096)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (2, 4096, 200)).astype(np.float32), "bf16", gpu_device)
    c = U.bmm(a, b, out_dtype=torch.float32, splits=4)
    assert torch.equal(c, U.bmm(a, b, out_dtype=torch.float32, splits=4))
    for s in range(2):
        an, bn = to_np(a)[s], to_np(b)[s]
        _check(to_np(c)[s], R.matmul(an, bn), 4096, an, bn, "bf16")


@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize(("act", "out_dtype"), [("identity", torch.bfloat16), ("silu", torch.float32)])
def test_matmul_trans_a_direct_to_lds(gpu_device, trans_b, act, out_dtype) -> None:
    # A stored [K, M]: its stage tiles are loaded and read as row-major B's.
    m, n, k = 512, 768, 320
    a, b = _operands(m, n, k, True, trans_b, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    got = U.matmul(a, b, trans_a=True, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype,
                   block_sizes=(256, 256, 64))
    out = "bf16" if out_dtype == torch.bfloat16 else "f32"
    ref = R.matmul(to_np(a), to_np(b), True, trans_b, to_np(bias), act=act, out=out)
    _check(to_np(got), ref, k, to_np(a).T, to_np(b), "bf16")


def test_matmul_trans_a_4096(gpu_device) -> None:
    cfg = W.config3()
    at = cfg["a"].t().contiguous().to(gpu_device)  # A stored [K, M]
    c = U.matmul(at, cfg["b"].to(gpu_device), trans_a=True)
    rows = tile_rows(RNG, 4096)
    an, bn = to_np(cfg["a"][torch.from_numpy(rows)]), to_np(cfg["b"])
    _check(to_np(c)[rows], R.matmul(an, bn, out="bf16"), 4096, an, bn, "bf16")


@pytest.mark.parametrize(("m", "n", "k"), [(4096, 8192, 1024), (1000, 1500, 777), (512, 512, 512),
                                         (2048, 520, 1024)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_matmul_trans_a_transposed_up_front(gpu_device, m, n, k, out_dtype) -> None:
    # From 512 rows, columns and K (but for whole 256 x 256 tiles filling the
    # CUs with N up to 4096), bf16 A stored [K, M] is transposed once into the
    # workspace and the product runs as one of row-major A: bit-equal to the
    # product of the explicitly transposed A, and checked on every tile.
    at = torch.from_numpy(RNG.uniform(-1, 1, (k, m)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    b = torch.from_numpy(RNG.uniform(-1, 1, (k, n)).astype(np.float32)).to(torch.bfloat16).to(gpu_device)
    bias = torch.from_numpy(RNG.normal(0, 1, n).astype(np.float32)).to(gpu_device)
    c = U.matmul(at, b, trans_a=True, bias=bias, epilogue=F.silu, out_dtype=out_dtype)
    c_nn = U.matmul(at.t().contiguous(), b, bias=bias, epilogue=F.silu, out_dtype=out_dtype)
    assert torch.equal(c, c_nn)
    rows = tile_rows(RNG, m)
    an, bn = to_np(at.t()[torch.from_numpy(rows).to(gpu_device)]), to_np(b)
    ref = R.matmul(an, bn, False, False, to_np(bias), act="silu",
                   out="bf16" if out_dtype == torch.bfloat16 else "f32")
    _check(to_np(c)[rows], ref, k, an, bn, "bf16" if out_dtype == torch.bfloat16 else "f32")


def _random_cases(count: int, seed: int) -> list[tuple]:
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        m = int(rng.choice([int(rng.integers(1, 700)), 256 * int(rng.integers(1, 4))]))
        n = int(rng.choice([int(rng.integers(1, 700)), 256 * int(rng.integers(1, 4))]))
        k = 64 * int(rng.integers(1, 9)) if rng.random() < 0.8 else int(rng.integers(1, 300))
        cases.append((m, n, k, bool(rng.random() < 0.3), bool(rng.random() < 0.5),
                      [None, (256, 256, 64), (128, 128, 64)][int(rng.integers(0, 3))],
                      ["identity", "relu", "silu"][int(rng.integers(0, 3))], bool(rng.random() < 0.5)))
    return cases


@pytest.mark.parametrize(("m", "n", "k", "trans_a", "trans_b", "tiles", "act", "f32_out"), _random_cases(40, 11))
def test_matmul_random_shapes(gpu_device, m, n, k, trans_a, trans_b, tiles, act, f32_out) -> None:
    # Seeded shapes over every bf16 path: whole, ragged and 128 x 128 tiles,
    # transposed A and B, K in whole stages or not, fused bias + activation.
    a, b = _operands(m, n, k, trans_a, trans_b, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    out_dtype = torch.float32 if f32_out else torch.bfloat16
    got = U.matmul(a, b, trans_a=trans_a, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype,
                   block_sizes=tiles)
    ref = R.matmul(to_np(a), to_np(b), trans_a, trans_b, to_np(bias), act=act, out="f32" if f32_out else "bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


def _long_k_cases(count: int, seed: int) -> list[tuple]:
    # K chunks of 16 or more 64-element stages: the 16x16x32 kernel's 128 x 128
    # tiles (whole and ragged) next to its 256 x 256 ones.
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(count):
        # At least 16 x 16 tiles of 128 x 128 (and too few of 256 x 256 to fill
        # the CUs): 128 x 128 tiles with whole K chunks.
        m = int(rng.choice([int(rng.integers(1921, 2400)), 128 * int(rng.integers(16, 19))]))
        n = int(rng.choice([8 * int(rng.integers(241, 300)), 128 * int(rng.integers(16, 19))]))
        k = 64 * int(rng.integers(16, 40))
        cases.append((m, n, k, bool(rng.random() < 0.5), [None, (128, 128, 64)][int(rng.integers(0, 2))],
                      ["identity", "relu", "silu"][int(rng.integers(0, 3))], bool(rng.random() < 0.5)))
    return cases


@pytest.mark.parametrize(("m", "n", "k", "trans_b", "tiles", "act", "f32_out"), _long_k_cases(16, 23))
def test_matmul_long_k_tiles(gpu_device, m, n, k, trans_b, tiles, act, f32_out) -> None:
    if torch.cuda.get_device_properties(gpu_device).multi_processor_count == 256:
        plan = U.gemm_plan(torch.bfloat16, m, n, k, trans_b=trans_b, block_sizes=tiles)
        assert (plan["splits"], plan["tile_m"]) == (1, 128)
    a, b = _operands(m, n, k, False, trans_b, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    out_dtype = torch.float32 if f32_out else torch.bfloat16
    got = U.matmul(a, b, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype, block_sizes=tiles)
    ref = R.matmul(to_np(a), to_np(b), False, trans_b, to_np(bias), act=act, out="f32" if f32_out else "bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


@pytest.mark.parametrize(("m", "n", "k", "trans_b", "splits"), [
    (1024, 1024, 4096, False, 4), (256, 4000, 4096, True, 4), (768, 768, 3072, False, 2),
    (128, 4096, 4096, True, 4), (512, 2048, 8192, False, 4),
])
@pytest.mark.parametrize(("act", "f32_out"), [("identity", False), ("gelu", True), ("silu", False)])
def test_matmul_fill_splits(gpu_device, m, n, k, trans_b, splits, act, f32_out) -> None:
    # Few 128 x 128 tiles with K in whole stages: split K until the grid holds
    # one workgroup per CU; the partials are summed in split order.
    if torch.cuda.get_device_properties(gpu_device).multi_processor_count == 256:
        plan = U.gemm_plan(torch.bfloat16, m, n, k, trans_b=trans_b)
        assert (plan["splits"], plan["tile_m"]) == (splits, 128)
    a, b = _operands(m, n, k, False, trans_b, "bf16", gpu_device, 0.3)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    out_dtype = torch.float32 if f32_out else torch.bfloat16
    got = U.matmul(a, b, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype)
    ref = R.matmul(to_np(a), to_np(b), False, trans_b, to_np(bias), act=act, out="f32" if f32_out else "bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")
    assert torch.equal(got, U.matmul(a, b, trans_b=trans_b, bias=bias, epilogue=ACTS[act], out_dtype=out_dtype))


@pytest.mark.parametrize(("m", "n", "k", "lda"), [
    (1, 11008, 4096, 0), (32, 11008, 4096, 0), (12, 9000, 512, 0), (31, 17000, 256, 0),  # 2 waves
    (8, 4096, 4096, 0), (16, 203, 192, 0), (17, 1000, 64, 0), (32, 300, 128, 0), (5, 33, 640, 0),  # 4 waves
    (64, 11008, 4096, 0), (64, 9000, 64, 0), (33, 4096, 1024, 0), (48, 203, 192, 0),  # two 32-row blocks of A
    (32, 4096, 1024, 1088),  # A a strided view
    (20, 500, 256, 257),  # A rows misaligned: the register-staged kernel
])
@pytest.mark.parametrize(("act", "f32_out"), [("identity", False), ("silu", True), ("gelu", False)])
def test_matmul_skinny(gpu_device, m, n, k, lda, act, f32_out) -> None:
    # Decode-shaped products (M <= 64, B [N, K]): one workgroup per 32 columns
    # of C, K split over its waves (ranges empty when K has fewer 64-element
    # stages than waves), ragged N, 8 / 16 / 32 / 64 rows of A loaded, fused bias,
    # scale, shift and activation; two calls give equal bits.
    a_full = tensor(RNG.normal(0, 0.3, (m, lda or k)).astype(np.float32), "bf16", gpu_device)
    a = a_full[:, :k]
    b = tensor(RNG.normal(0, 0.3, (n, k)).astype(np.float32), "bf16", gpu_device)
    bias, scale, shift = (tensor(RNG.normal(1, 0.5, n).astype(np.float32), "bf16", gpu_device) for _ in range(3))
    out_dtype = torch.float32 if f32_out else torch.bfloat16

    def run() -> torch.Tensor:
        return U.matmul(a, b, trans_b=True, bias=bias, scale=scale, shift=shift, epilogue=ACTS[act],
                        out_dtype=out_dtype)

    assert U.gemm_plan(torch.bfloat16, m, n, k, trans_b=True)["tile_m"] == 32
    got = run()
    assert torch.equal(run(), got)
    ref = R.matmul(to_np(a), to_np(b), False, True, to_np(bias), to_np(scale), to_np(shift), act,
                   out="f32" if f32_out else "bf16")
    _check(to_np(got), ref, k, to_np(a), to_np(b), "bf16")


def test_bmm_whole_tiles_split_k_direct_to_lds(gpu_device) -> None:
    a = tensor(RNG.uniform(-1, 1, (1, 4096, 1024)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (1, 1024, 4096)).astype(np.float32), "bf16", gpu_device)
    c = U.bmm(a, b, splits=2)
    assert torch.equal(U.bmm(a, b, splits=2), c)
    torch.cuda.synchronize()
    rows = tile_rows(RNG, 4096)
    an, bn = to_np(a)[0][rows], to_np(b)[0]
    _check(to_np(c)[0][rows], R.matmul(an, bn, out="bf16"), 1024, an, bn, "bf16")


def test_matmul_config1_f32_512(gpu_device) -> None:
    cfg = W.config1()
    got = to_np(U.matmul(cfg["a"].to(gpu_device), cfg["b"].to(gpu_device), block_sizes=[64, 64, 64]))
    ref = R.matmul(cfg["a"].numpy(), cfg["b"].numpy())
    assert max_rel_error(got, ref) < 1e-5
    f64 = cfg["a"].double().numpy() @ cfg["b"].double().numpy()
    assert max_rel_error(got, f64) < 1e-5


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_matmul_config3_bf16_4096(gpu_device, out_dtype) -> None:
    cfg = W.config3()
    a, b = cfg["a"].to(gpu_device), cfg["b"].to(gpu_device)
    c = U.matmul(a, b, out_dtype=out_dtype)
    torch.cuda.synchronize()
    rows = torch.from_numpy(tile_rows(RNG, 4096))
    got = to_np(c[rows.to(gpu_device)])
    an, bn = to_np(cfg["a"][rows]), to_np(cfg["b"])
    ref = R.matmul(an, bn, out="bf16" if out_dtype == torch.bfloat16 else "f32")
    _check(got, ref, 4096, an, bn, "bf16")


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("trans_b", [True, False])
def test_matmul_whole_rounds_split(gpu_device, out, trans_b) -> None:
    # 16 x 17 = 272 tiles of 256 x 256 on 256 CUs: the first 16 tile columns (one
    # whole round) run as 256 x 256 tiles, the last 256 columns as 256 x 128
    # tiles (B rows or columns, C columns and bias from column 4096 on).
    # Checked in full.
    m, n, k = 4096, 4352, 320
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    w = tensor(RNG.normal(0, 1, (n, k) if trans_b else (k, n)).astype(np.float32), "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    odt = torch.float32 if out == "f32" else None
    got = to_np(U.matmul(a, w, trans_b=trans_b, bias=bias, epilogue=F.silu, out_dtype=odt))
    ref = R.matmul(to_np(a), to_np(w), False, trans_b, to_np(bias), act="silu", out=out)
    _check(got, ref, k, to_np(a), to_np(w), "bf16")


@pytest.mark.parametrize(("trans_b", "epilogue", "out"),
                         [(False, "identity", "f32"), (True, "relu", "f32"), (False, "silu", "bf16"),
                          (True, "identity", "bf16")])
def test_f32_big_tile_unsplit(gpu_device, trans_b: bool, epilogue: str, out: str) -> None:
    # 4096 x 4096 x 1024 f32: 256 whole 256 x 256 tiles fill the CUs, so the
    # direct-to-LDS f32 kernel runs unsplit and finishes C itself (bias, the
    # activation, f32 or bf16 C). A with a row pitch that loses 16-byte
    # alignment takes the 128 x 128 register-staged tile instead. Sampled rows
    # of both against the oracle.
    m, n, k = 4096, 4096, 1024
    if torch.cuda.get_device_properties(gpu_device).multi_processor_count == 256:
        plan = U.gemm_plan(torch.float32, m, n, k, trans_b=trans_b)
        assert (plan["splits"], plan["tile_m"], plan["tile_n"], plan["tile_k"]) == (1, 256, 256, 32)
    gen = torch.Generator(device=gpu_device).manual_seed(17)
    a = torch.randn(m, k, device=gpu_device, generator=gen)
    w = torch.randn((n, k) if trans_b else (k, n), device=gpu_device, generator=gen)
    bias = torch.randn(n, device=gpu_device, generator=gen)
    fn = {"silu": F.silu, "relu": torch.relu, "identity": None}[epilogue]
    kw = dict(trans_b=trans_b, out_dtype=torch.bfloat16 if out == "bf16" else None)
    if fn is not None:
        kw.update(bias=bias, epilogue=fn)
    a_pitch = torch.empty(m, k + 1, device=gpu_device)[:, :k]
    a_pitch.copy_(a)
    rows = torch.from_numpy(tile_rows(RNG, m, 1)).to(gpu_device)
    an, wn = to_np(a[rows]), to_np(w)
    ref = R.matmul(an, wn, False, trans_b, to_np(bias) if fn is not None else None, act=epilogue, out=out)
    for x in (a, a_pitch):
        got = to_np(U.matmul(x, w, **kw)[rows])
        if out == "f32":
            _check(got, ref, k, an, wn, "f32")
        else:
            assert_close(got, ref, 1e-2, 1e-2)


def test_linear_config4_silu(gpu_device) -> None:
    cfg = W.config4()
    x, w, b = (cfg[k].to(gpu_device) for k in ("x", "w", "b"))
    layer = torch.nn.Linear(4096, 11008, device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.weight.copy_(w)
        layer.bias.copy_(b)
        y, cache = U.linear(x, layer, F.silu)
        y2, cache2 = U.linear(x, layer, F.silu, cache=cache)
    assert cache2.call is cache.call and torch.equal(y, y2)
    torch.cuda.synchronize()
    rows = torch.from_numpy(tile_rows(RNG, 8192, 1))
    got = to_np(y[rows.to(gpu_device)])
    xn, wn, bn = to_np(cfg["x"][rows]), to_np(cfg["w"]), to_np(cfg["b"])
    ref = R.matmul(xn, wn, False, True, bn, act="silu", out="bf16")
    _check(got, ref, 4096, xn, wn, "bf16")


@pytest.mark.parametrize(("trans_b", "act"), [(True, "relu"), (False, "identity")])
def test_rounds_and_tail_f32_out(gpu_device, trans_b, act) -> None:
    # Whole rounds of 256 x 256 tiles and a 256 x 128 tail in one launch, f32
    # C: equal bit for bit to single rounds of 1024-row blocks, and to the
    # oracle on rows of every tile.
    m, n, k = 4096, 4608, 256
    a = tensor(RNG.uniform(-1, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32), "bf16", gpu_device)
    bias = torch.randn(n, device=gpu_device, dtype=torch.float32)
    kw = {"bias": bias, "epilogue": ACTS[act], "out_dtype": torch.float32}
    full = U.matmul(a, b, trans_b=trans_b, **kw)
    blocks = torch.cat([U.matmul(a[r:r + 1024], b, trans_b=trans_b, **kw) for r in range(0, m, 1024)])
    assert full.dtype == torch.float32 and torch.equal(full, blocks)
    rows = torch.from_numpy(tile_rows(RNG, m, 1))
    an, bn = to_np(a[rows.to(gpu_device)]), to_np(b)
    ref = R.matmul(an, bn, False, trans_b, to_np(bias), act=act, out="f32")
    _check(to_np(full[rows.to(gpu_device)]), ref, k, an, bn, "bf16")


@pytest.mark.parametrize(
    ("m", "n", "k", "trans_b", "vectors"),
    [(8192, 11008, 4096, True, "bias"), (4096, 8192, 256, False, "none"), (3072, 6144, 128, True, "all_f32"),
     (4096, 4608, 512, False, "all_f32"), (4096, 4352, 128, True, "bias"), (8192, 8448, 64, False, "none")],
)
def test_multi_round_tiles_match_single_rounds(gpu_device, m, n, k, trans_b, vectors) -> None:
    # More 256 x 256 tiles than CUs (several rounds; config 4 first, and
    # 4096 x 4608 with row-major B, both whole rounds of 256 x 256 tiles and a
    # tail of 256 x 128 tiles in one launch) against blocks of 1024 rows,
    # each a single round of one workgroup per tile. Each output is the same
    # K walk in either, so the results are equal bit for bit; bias, scale and
    # shift in bf16 and f32 take the epilogue's 8- and 16-byte loads.
    a = tensor(RNG.uniform(-1, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32), "bf16", gpu_device)
    vdt = torch.float32 if vectors == "all_f32" else torch.bfloat16
    kw = {}
    if vectors != "none":
        kw["bias"] = torch.randn(n, device=gpu_device, dtype=vdt)
    if vectors == "all_f32":
        kw["scale"] = torch.rand(n, device=gpu_device, dtype=vdt) + 0.5
        kw["shift"] = torch.randn(n, device=gpu_device, dtype=vdt)
    fn = F.silu if vectors != "none" else None
    if fn is not None:
        kw["epilogue"] = fn
    full = U.matmul(a, b, trans_b=trans_b, **kw)
    blocks = torch.cat([U.matmul(a[r:r + 1024], b, trans_b=trans_b, **kw) for r in range(0, m, 1024)])
    assert torch.equal(full, blocks)
    rows = torch.from_numpy(tile_rows(RNG, m, 1))
    an, bn = to_np(a[rows.to(gpu_device)]), to_np(b)
    vec = {key: to_np(kw[key]) for key in ("bias", "scale", "shift") if key in kw}
    ref = R.matmul(an, bn, False, trans_b, vec.get("bias"), vec.get("scale"), vec.get("shift"),
                   act="silu" if fn is not None else "identity", out="bf16")
    _check(to_np(full[rows.to(gpu_device)]), ref, k, an, bn, "bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_linear_follows_weight_updates(gpu_device, dtype) -> None:
    tdtype = torch.float32 if dtype == "f32" else torch.bfloat16
    layer = torch.nn.Linear(128, 64).to(device=gpu_device, dtype=tdtype)
    x = tensor(RNG.normal(0, 1, (32, 128)).astype(np.float32), dtype, gpu_device)
    with torch.no_grad():
        y, cache = U.linear(x, layer, torch.relu)
        layer.weight.mul_(-1.0)
        y3, cache3 = U.linear(x, layer, torch.relu, cache=cache)
    assert cache3.packed_weight is not cache.packed_weight
    ref = R.matmul(to_np(x), to_np(layer.weight), False, True, to_np(layer.bias), act="relu", out=dtype)
    _check(to_np(y3), ref, 128, to_np(x), to_np(layer.weight), dtype)


def test_linear_affine_and_panel(gpu_device) -> None:
    layer = torch.nn.Linear(96, 70).to(device=gpu_device, dtype=torch.bfloat16)
    x = tensor(RNG.normal(0, 1, (40, 96)).astype(np.float32), "bf16", gpu_device)
    post_scale = tensor(RNG.uniform(0, 1, 70).astype(np.float32), "bf16", gpu_device)
    post_bias = tensor(RNG.normal(0, 1, 1).astype(np.float32), "bf16", gpu_device)
    with torch.no_grad():
        y, _ = U.linear_affine(x, layer, post_scale, post_bias, torch.relu)
        yp, cache = U.linear(x, layer, torch.relu, panel=64)
    assert cache.packed_weight.dim() == 4
    xs, ws, bs = to_np(x), to_np(layer.weight), to_np(layer.bias)
    ref = R.matmul(xs, ws, False, True, bs, to_np(post_scale), to_np(post_bias), "relu", out="bf16")
    _check(to_np(y), ref, 96, xs, ws, "bf16")
    _check(to_np(yp), R.matmul(xs, ws, False, True, bs, act="relu", out="bf16"), 96, xs, ws, "bf16")


@pytest.mark.parametrize(("m", "n", "k"), [(1024, 1536, 512), (512, 11008, 256), (300, 768, 128)])
def test_linear_whole_rows(gpu_device, m: int, n: int, k: int) -> None:
    # whole_rows takes the whole-row tiles (the weight as VNNI panels of the
    # tile's columns, the tile's rows asked for): the same products as the
    # default launch, bit for bit, and its own cache entry.
    layer = torch.nn.Linear(k, n).to(device=gpu_device, dtype=torch.bfloat16)
    x = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    with torch.no_grad():
        y, cache = U.linear(x, layer, F.silu)
        yw, cache_w = U.linear(x, layer, F.silu, whole_rows=True)
        yw2, cache_w2 = U.linear(x, layer, F.silu, cache=cache_w, whole_rows=True)
    assert cache_w.key != cache.key and cache_w2.call is cache_w.call
    tiles = U.whole_row_tiles(m, n)
    if tiles is not None:
        assert cache_w.packed_weight.dim() == 4 and cache_w.packed_weight.shape[2] == tiles[1]
    assert torch.equal(y, yw) and torch.equal(yw, yw2)
    xs, ws, bs = to_np(x), to_np(layer.weight), to_np(layer.bias)
    _check(to_np(yw), R.matmul(xs, ws, False, True, bs, act="silu", out="bf16"), k, xs, ws, "bf16")


# ---------------------------------------------------------------------------
# bmm / split-K


@pytest.mark.parametrize("shape", [(2, 160, 96, 224), (2, 65, 129, 129), (3, 100, 70, 130), (4, 64, 64, 8192),
                                   (1, 33, 17, 40000), (4, 2048, 2048, 128)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_bmm_matches_oracle(gpu_device, shape, dtype) -> None:
    batch, m, n, k = shape
    a = tensor(RNG.uniform(-1, 1, (batch, m, k)).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.uniform(-1, 1, (batch, k, n)).astype(np.float32), dtype, gpu_device)
    got = to_np(U.bmm(a, b))
    ref = R.bmm(to_np(a), to_np(b), out=dtype)
    if dtype == "f32":
        assert max_rel_error(got, ref) < 1e-5
    else:
        assert max_rel_error(got, ref) < 2e-2
        assert_close(got, ref, 1e-2, bf16_gemm_atol(k, to_np(a), to_np(b)))


@pytest.mark.parametrize("splits", [1, 2, 5, 16])
def test_bmm_split_k_is_deterministic(gpu_device, splits) -> None:
    a = tensor(RNG.uniform(-1, 1, (3, 64, 4096)).astype(np.float32), "f32", gpu_device)
    b = tensor(RNG.uniform(-1, 1, (3, 4096, 96)).astype(np.float32), "f32", gpu_device)
    first = U.bmm(a, b, splits=splits)
    for _ in range(3):
        assert torch.equal(U.bmm(a, b, splits=splits), first)
    assert max_rel_error(to_np(first), R.bmm(to_np(a), to_np(b))) < 1e-5


def test_bmm_rejects_mismatched_operands(gpu_device) -> None:
    a = torch.randn(3, 64, 64, device=gpu_device)
    with pytest.raises(RuntimeError, match="batch2"):
        U.bmm(a, torch.randn(1, 64, 64, device=gpu_device))
    with pytest.raises(RuntimeError, match="batch2"):
        U.bmm(a, torch.randn(3, 32, 64, device=gpu_device))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_bmm_config5_full_size(gpu_device, dtype) -> None:
    cfg = W.config5(torch.float32 if dtype == "f32" else torch.bfloat16)
    a, b = cfg["a"].to(gpu_device), cfg["b"].to(gpu_device)
    plan = U.gemm_plan(a.dtype, 256, 256, 65536, batch=16)
    assert plan["splits"] >= 16
    c = U.bmm(a, b, out_dtype=torch.float32)
    c2 = U.bmm(a, b, out_dtype=torch.float32)
    assert torch.equal(c, c2)
    torch.cuda.synchronize()
    for s in (0, 11):
        got = to_np(c[s])
        ref = R.bmm(to_np(cfg["a"][s]), to_np(cfg["b"][s]))
        assert max_rel_error(got, ref) < (1e-5 if dtype == "f32" else 1e-5)


# ---------------------------------------------------------------------------
# Packing and prepacked GEMMs


@pytest.mark.parametrize(("rows", "cols"), [(128, 96), (70, 45), (1, 1), (33, 64), (600, 1040), (1040, 600),
                                          (259, 77)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_pack_kernels_match_oracle(gpu_device, rows, cols, dtype) -> None:
    x = tensor(RNG.normal(0, 1, (rows, cols)).astype(np.float32), dtype, gpu_device)
    xs = to_np(x)
    xt = x.t().contiguous()
    np.testing.assert_array_equal(to_np(U.pack_a_blocked(x)), R.pack_a_blocked(xs))
    np.testing.assert_array_equal(to_np(U.pack_a_blocked_t(xt)), R.pack_a_blocked(xs))
    np.testing.assert_array_equal(to_np(U.pack_b_blocked(x)), R.pack_b_blocked(xs))
    np.testing.assert_array_equal(to_np(U.pack_b_blocked_t(xt)), R.pack_b_blocked(xs))
    np.testing.assert_array_equal(to_np(U.pack_b_blocked_vnni(x)), R.pack_b_blocked_vnni(xs))
    np.testing.assert_array_equal(to_np(U.pack_b_blocked_vnni_t(xt)), R.pack_b_blocked_vnni(xs))
    np.testing.assert_array_equal(to_np(U.pad_2d(x, rows + 3, cols + 5)), R.pad_2d(xs, rows + 3, cols + 5))
    if cols % 2 == 0:  # x as a transposed weight [N, K], K even
        np.testing.assert_array_equal(to_np(U.pack_b_vnni_t(x)), R.pack_b_vnni_t(xs))
        np.testing.assert_array_equal(to_np(U.pack_b_vnni_t(x, 32)), R.pack_b_vnni_t(xs, 32))
    if cols % 16 == 0:
        np.testing.assert_array_equal(to_np(U.pack_b_panels(x, 16)), R.pack_b_panels(xs, 16))
        np.testing.assert_array_equal(to_np(U.pack_a_panels(x, 16)), R.pack_a_panels(xs, 16))


@pytest.mark.parametrize(("n", "k"), [(1000, 4096), (130, 70), (64, 2), (257, 520)])
@pytest.mark.parametrize("panel", [64, 128, 256])
def test_pack_vnni_t_tiled_transpose(gpu_device, n, k, panel) -> None:
    # pack_b_vnni_t with panels of a multiple of 64 columns runs the tiled
    # word transpose: 16-byte row loads when K % 8 == 0, 4-byte loads
    # otherwise (K = 70), zero padding past N and K, bit-exact.
    w = tensor(RNG.normal(0, 1, (n + 1, k)).astype(np.float32), "bf16", gpu_device)
    np.testing.assert_array_equal(to_np(U.pack_b_vnni_t(w[:n], panel)), R.pack_b_vnni_t(to_np(w[:n]), panel))
    # A row-offset view (its base moves by one row of K values).
    np.testing.assert_array_equal(to_np(U.pack_b_vnni_t(w[1:], panel)), R.pack_b_vnni_t(to_np(w[1:]), panel))


@pytest.mark.parametrize("mkn", [(64, 256, 128), (40, 66, 100), (64, 4096, 64), (300, 128, 64), (33, 64, 70)])
@pytest.mark.parametrize("panel", [64, 128])
def test_matmul_prepacked_vnni(gpu_device, mkn, panel) -> None:
    m, k, n = mkn
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    w = tensor(RNG.normal(0, 1, (n, k)).astype(np.float32), "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    got = to_np(U.matmul_prepacked_b(a, U.pack_b_vnni_t(w, panel), n, bias, torch.relu))
    ref = R.matmul(to_np(a), to_np(w), False, True, to_np(bias), act="relu", out="bf16")
    _check(got, ref, k, to_np(a), to_np(w), "bf16")


@pytest.mark.parametrize("mkn", [(64, 256, 96), (33, 256, 64), (130, 96, 70), (17, 64, 32), (40, 100, 64)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_matmul_prepacked_blocked(gpu_device, mkn, dtype) -> None:
    m, k, n = mkn
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), dtype, gpu_device)
    w = tensor(RNG.normal(0, 1, (n, k)).astype(np.float32), dtype, gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), dtype, gpu_device)
    ref = R.matmul(to_np(a), to_np(w), False, True, to_np(bias), act="relu", out=dtype)
    got = to_np(U.matmul_prepacked_b(a, U.pack_b_blocked_t(w), n, bias, torch.relu))
    _check(got, ref, k, to_np(a), to_np(w), dtype)
    call = U.prepacked_b_call(a, U.pack_b_blocked_t(w), n, bias, torch.relu)
    _check(to_np(call(a)), ref, k, to_np(a), to_np(w), dtype)
    if dtype == "bf16":
        got = to_np(U.matmul_prepacked_b(a, U.pack_b_blocked_vnni_t(w), n, bias, torch.relu))
        _check(got, ref, k, to_np(a), to_np(w), dtype)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_matmul_bench_panels(gpu_device, dtype) -> None:
    m, k, n = 96, 192, 256
    a = tensor(RNG.uniform(-1, 1, (m, k)).astype(np.float32), dtype, gpu_device)
    b = tensor(RNG.uniform(-1, 1, (k, n)).astype(np.float32), dtype, gpu_device)
    got = to_np(U.matmul_prepacked_b(a, U.pack_b_panels(b, 64), n))
    _check(got, R.matmul(to_np(a), to_np(b), out=dtype), k, to_np(a), to_np(b), dtype)


@pytest.mark.parametrize("panel", [32, 64, 128, 256, 512, 768])
@pytest.mark.parametrize(("n", "k"), [(4096, 64), (4608, 320), (4096, 4096)])
def test_vnni_relayout_sweep(gpu_device, panel: int, n: int, k: int) -> None:
    # The 16x16x32 kernel re-lays VNNI panels as they land (4 KiB slabs per K
    # pair index): panels narrower than, equal to and wider than a tile, tiles
    # at every offset in a panel, one K stage to 64. At least 256 tiles, so
    # the product is not split (split-K runs the 32x32 kernel): bit-equal to
    # the plain B product (the same K walk), and to the oracle on rows of
    # every tile.
    m = 4096
    a = tensor(RNG.uniform(-1, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    w = tensor(RNG.uniform(-1, 1, (n, k)).astype(np.float32), "bf16", gpu_device)
    got = U.matmul_prepacked_b(a, U.pack_b_vnni_t(w, panel), n)
    assert torch.equal(got, U.matmul(a, w, trans_b=True))
    rows = tile_rows(RNG, m, 1)
    an, wn = to_np(a)[rows], to_np(w)
    _check(to_np(got)[rows], R.matmul(an, wn, False, True, out="bf16"), k, an, wn, "bf16")


@pytest.mark.parametrize("panel", [32, 64, 128, 256, 512])
def test_matmul_prepacked_vnni_whole_tiles(gpu_device, panel) -> None:
    # Whole 256 x 256 tiles with K a multiple of 64: the direct-to-LDS kernel
    # reads the VNNI panels in place (panels narrower and wider than a tile),
    # with the fused bias + SiLU epilogue.
    m, k, n = 512, 320, 768
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    w = tensor(RNG.normal(0, 1, (n, k)).astype(np.float32), "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    got = to_np(U.matmul_prepacked_b(a, U.pack_b_vnni_t(w, panel), n, bias, torch.nn.functional.silu))
    ref = R.matmul(to_np(a), to_np(w), False, True, to_np(bias), act="silu", out="bf16")
    _check(got, ref, k, to_np(a), to_np(w), "bf16")
    plain = U.matmul(a, w, trans_b=True, bias=bias, epilogue=torch.nn.functional.silu)
    assert torch.equal(torch.from_numpy(got), plain.cpu().float())


@pytest.mark.parametrize("layout", ["panels16", "panels64", "panels256", "panels384", "panels768", "blocked"])
def test_matmul_prepacked_rowmajor_whole_tiles(gpu_device, layout) -> None:
    # Whole 256 x 256 tiles with K a multiple of 64: the direct-to-LDS kernel
    # reads K-major panels [N/P, K, P] (narrower than a tile, one tile, tiles
    # straddling two panels, wider than a tile) and 32 x 32 blocks in place,
    # with the fused bias + SiLU epilogue.
    m, k, n = 512, 320, 768
    a = tensor(RNG.normal(0, 1, (m, k)).astype(np.float32), "bf16", gpu_device)
    b = tensor(RNG.normal(0, 1, (k, n)).astype(np.float32), "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, n).astype(np.float32), "bf16", gpu_device)
    packed = U.pack_b_blocked(b) if layout == "blocked" else U.pack_b_panels(b, int(layout[6:]))
    got = to_np(U.matmul_prepacked_b(a, packed, n, bias, torch.nn.functional.silu))
    ref = R.matmul(to_np(a), to_np(b), bias=to_np(bias), act="silu", out="bf16")
    _check(got, ref, k, to_np(a), to_np(b), "bf16")
    plain = U.matmul(a, b, bias=bias, epilogue=torch.nn.functional.silu)
    assert torch.equal(torch.from_numpy(got), plain.cpu().float())


def test_matmul_config3_prepacked_layouts(gpu_device) -> None:
    cfg = W.config3(scale=4)  # 1024^3, the config-3 distribution
    a, b = cfg["a"].to(gpu_device), cfg["b"].to(gpu_device)
    plain = U.matmul(a, b)
    bt = b.t().contiguous()
    for packed in (U.pack_b_blocked_vnni(b), U.pack_b_vnni_t(bt, 256), U.pack_b_panels(b, 256), U.pack_b_blocked(b)):
        got = U.matmul_prepacked_b(a, packed, 1024)
        # The same products summed in the same K order: bit-equal to the plain kernel.
        assert torch.equal(got, plain)
