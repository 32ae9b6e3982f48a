"""Pins of the CPU oracle (``oracle/restate.py``) before it judges the GPU.

The reference's JIT'd CPU kernels cannot run here and its tests hold no
numeric fixtures, so each oracle function is pinned to something it does not
share code with: torch's float64 library routines (softmax, group_norm,
layer_norm, rms_norm, matmul, activations), brute-force element loops of the
layout definitions in the reference's docstrings, torch's own bf16 rounding,
the reference's special cases (one-column softmax) and its tolerances
(tests/test_cpu_utils_softmax.py:18-34, test_cpu_utils_split_k_bmm.py:15-16).
Inputs are chosen so that plausible mistakes fail: non-square shapes for
transposes, shifted rows for a missing max subtraction, tiny rows for a
misplaced eps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import restate as R
from tests.helpers import max_rel_error

RNG = np.random.default_rng(1234)


def _f64(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.asarray(x, np.float64))


# ---------------------------------------------------------------------------
# bf16 rounding


def test_bf16_rounding_matches_torch() -> None:
    x = np.concatenate(
        [
            RNG.normal(0, 3, 20000).astype(np.float32),
            RNG.normal(0, 1e-38, 200).astype(np.float32),  # subnormals
            np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 1.0078125 * 1.0000001,
                      3.3895314e38, -3.4e38, np.inf, -np.inf], np.float32),
            # exact ties between two bf16 values: round to even
            (np.arange(1, 300, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        ]
    )
    ours = R.bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    nan = R.from_bf16_bits(R.bf16_bits(np.array([np.nan, -np.nan], np.float32)))
    assert np.isnan(nan).all()


# ---------------------------------------------------------------------------
# Activations


@pytest.mark.parametrize("name", R.ACTIVATIONS)
def test_activations_match_torch(name: str) -> None:
    x = np.concatenate([RNG.normal(0, 4, 4096), [0.0, -0.0, 30.0, -30.0, 1e-8]]).astype(np.float32)
    t = _f64(x)
    ref = {
        "identity": t,
        "relu": torch.relu(t),
        "silu": F.silu(t),
        "sigmoid": torch.sigmoid(t),
        "gelu": F.gelu(t),
        "gelu_tanh": F.gelu(t, approximate="tanh"),
        "tanh": torch.tanh(t),
        "leaky_relu": F.leaky_relu(t, 0.2),
    }[name].numpy()
    got = R.activation(name, x, 0.2)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# Softmax


@pytest.mark.parametrize(
    ("m", "n", "shift"),
    # The reference's partial-last-chunk cases (test_cpu_utils_softmax.py:18-26)
    # and a large positive shift (exp overflows without the max subtraction).
    [(130, 515, 0.0), (4, 129, -50.0), (2, 200, -50.0), (4, 256, -50.0), (3, 47, 0.0), (5, 300, 100.0)],
)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_matches_torch(m: int, n: int, shift: float, dtype: str) -> None:
    x = R.round_to(RNG.normal(0, 1, (m, n)).astype(np.float32) + np.float32(shift), dtype)
    got = R.softmax(x, dtype)
    ref = torch.softmax(_f64(x), -1).numpy()
    assert max_rel_error(got, ref) < (1e-6 if dtype == "f32" else 1e-2)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_one_column_and_nonfinite_rows(dtype: str) -> None:
    # test_cpu_utils_softmax.py:37-47: 1, NaN for NaN and infinite inputs.
    x = np.array([[0.5], [-3e4], [np.nan], [np.inf], [-np.inf]], np.float32)
    got = R.softmax(x, dtype)
    ref = torch.softmax(torch.from_numpy(x), -1).numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    rows = np.array([[1.0, np.nan, 2.0], [1.0, np.inf, 2.0], [-np.inf] * 3, [1.0, -np.inf, 1.0]], np.float32)
    got = R.softmax(rows, dtype)
    ref = torch.softmax(torch.from_numpy(rows), -1).numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_allclose(got[3], [0.5, 0.0, 0.5])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_large_finite_rows_match_torch(dtype: str) -> None:
    # exp(x - row_max) (normalization.py:61-72) stays finite however large the
    # row's values: a formulation that folds the maximum into the exponent's
    # scaling (exp2(x * log2e - max * log2e)) carries max * log2e's rounding
    # error into every exponent and fails these rows.
    x = R.round_to(np.array([[1e10, 0.0], [-1e10, -1e10 + 2048.0], [3e38, -3e38], [5e9, 5e9],
                             [-5e9, 1e-30]], np.float32), dtype)
    got = R.softmax(x, dtype)
    np.testing.assert_array_equal(got, torch.softmax(_f64(x), -1).numpy().astype(np.float32))
    col = R.round_to(np.array([[5e9], [3e38], [-3e38], [1e-30]], np.float32), dtype)
    np.testing.assert_array_equal(R.softmax(col, dtype), np.ones_like(col))
    # The folded formulation with one FMA, exp2(fma(x, log2e, -RN(max *
    # log2e))), modelled in float64 (exact product, one rounding), is wrong on
    # the first row: the oracle would catch a kernel that used it.
    log2e = np.float32(1.4426950408889634)
    ml = np.float32(x[0].max() * log2e)
    t = (x[0].astype(np.float64) * np.float64(log2e) - np.float64(ml)).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp2(t)
        folded = e / e.sum(dtype=np.float32)
    assert not np.array_equal(folded, [1.0, 0.0])


# ---------------------------------------------------------------------------
# RMSNorm / GroupNorm / LayerNorm


@pytest.mark.parametrize("scale", [2.0, 1e-4])  # 1e-4: eps dominates mean(x^2)
def test_rms_norm_matches_torch(scale: float) -> None:
    x = (RNG.normal(0, scale, (17, 333))).astype(np.float32)
    w = RNG.uniform(0.5, 1.5, 333).astype(np.float32)
    got = R.rms_norm(x, w, 1e-6)
    ref = F.rms_norm(_f64(x), (333,), _f64(w), eps=1e-6).numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=1e-6)
    ref_no_w = F.rms_norm(_f64(x), (333,), eps=1e-6).numpy()
    np.testing.assert_allclose(R.rms_norm(x, None, 1e-6), ref_no_w, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize(
    ("m", "c", "groups"),
    # test_cpu_utils_softmax.py:82-85's GroupNorm shapes.
    [(32, 256, 16), (33, 256, 4), (64, 512, 512), (5, 96, 3), (2, 65, 5)],
)
def test_group_norm_matches_torch(m: int, c: int, groups: int) -> None:
    x = (RNG.normal(0, 3, (m, c)) + 1.5).astype(np.float32)
    w = RNG.normal(0, 1, c).astype(np.float32)
    b = RNG.normal(0, 1, c).astype(np.float32)
    got = R.group_norm(x, groups, w, b, 1e-5)
    ref = F.group_norm(_f64(x), groups, _f64(w), _f64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=2e-4)


def test_layer_norm_and_group_norm_epilogues() -> None:
    x = (RNG.normal(0, 2, (9, 130)) - 3.0).astype(np.float32)
    w, b, extra = (RNG.normal(0, 1, 130).astype(np.float32) for _ in range(3))
    ln = F.layer_norm(_f64(x), (130,), _f64(w), _f64(b), eps=1e-5).numpy()
    np.testing.assert_allclose(R.group_norm(x, 1, w, b, 1e-5), ln, rtol=1e-4, atol=2e-4)
    added = R.group_norm(x, 1, w, b, 1e-5, extra, "add", "relu")
    np.testing.assert_allclose(added, np.maximum(ln + extra, 0), rtol=1e-4, atol=2e-4)
    multiplied = R.group_norm(x, 1, w, b, 1e-5, extra, "mul")
    np.testing.assert_allclose(multiplied, ln * extra, rtol=1e-4, atol=2e-4)
    # A callable epilogue(y, extra) gets the normalized values and the extra
    # operand broadcast over rows (normalization.py:121); without an extra
    # operand, the weight (normalization.py:190-192).
    called = R.group_norm(x, 1, w, b, 1e-5, extra, "callable", lambda y, e: torch.tanh(y) * e - y)
    np.testing.assert_allclose(called, np.tanh(ln) * extra - ln, rtol=1e-4, atol=2e-4)
    defaulted = R.group_norm(x, 1, w, b, 1e-5, None, "callable", lambda y, e: y + e)
    np.testing.assert_allclose(defaulted, ln + w, rtol=1e-4, atol=2e-4)


def test_callable_epilogues_are_applied_in_f32() -> None:
    x = RNG.normal(0, 4, (64, 33)).astype(np.float32)
    # A callable naming a known activation gives that activation.
    for name, fn in (("silu", F.silu), ("gelu", F.gelu), ("tanh", torch.tanh), ("relu", torch.relu)):
        np.testing.assert_allclose(R.apply_epilogue(fn, x), R.activation(name, x), rtol=2e-6, atol=1e-6)
    # Any other callable: its f32 value (the reference applies it to the f32
    # accumulator), checked against float64 evaluation.
    got = R.apply_epilogue(lambda t: F.hardswish(t) * 3 - t / 7, x)
    ref = (F.hardswish(_f64(x)) * 3 - _f64(x) / 7).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    assert got.dtype == np.float32
    # In the GEMM: after bias, scale and shift, before the one rounding.
    a = RNG.normal(0, 1, (20, 30)).astype(np.float32)
    b = RNG.normal(0, 1, (30, 40)).astype(np.float32)
    bias = RNG.normal(0, 1, 40).astype(np.float32)
    got = R.matmul(a, b, bias=bias, act=lambda t: F.mish(t) + 1, out="bf16")
    ref = (F.mish(_f64(a) @ _f64(b) + _f64(bias)) + 1).float().to(torch.bfloat16).float().numpy()
    np.testing.assert_allclose(got, ref, rtol=2**-7, atol=1e-6)


# ---------------------------------------------------------------------------
# GEMMs


@pytest.mark.parametrize(("trans_a", "trans_b"), [(False, False), (True, False), (False, True), (True, True)])
def test_matmul_matches_float64(trans_a: bool, trans_b: bool) -> None:
    m, n, k = 37, 45, 19  # the reference's irregular shape (test_mlir_execution.py:1839)
    a = RNG.normal(0, 1, (k, m) if trans_a else (m, k)).astype(np.float32)
    b = RNG.normal(0, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
    bias, scale, shift = (RNG.normal(0, 1, n).astype(np.float32) for _ in range(3))
    got = R.matmul(a, b, trans_a, trans_b, bias, scale, shift, "silu")
    ta, tb = _f64(a), _f64(b)
    acc = (ta.T if trans_a else ta) @ (tb.T if trans_b else tb)
    ref = F.silu((acc + _f64(bias)) * _f64(scale) + _f64(shift)).numpy()
    assert max_rel_error(got, ref) < 1e-5


def test_matmul_bf16_rounds_once() -> None:
    a = R.round_bf16(RNG.uniform(-1, 1, (64, 96)).astype(np.float32))
    b = R.round_bf16(RNG.uniform(-1, 1, (96, 40)).astype(np.float32))
    got = R.matmul(a, b, out="bf16")
    ref = (torch.from_numpy(a).double() @ torch.from_numpy(b).double()).float().to(torch.bfloat16).float().numpy()
    # One rounding of the f32 accumulator: at most one bf16 ulp from rounding
    # the exact sum, never two.
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-7 + 1e-30)
    assert np.array_equal(got, R.round_bf16(got))


def test_split_k_bmm_matches_float64_and_is_ordered() -> None:
    a = RNG.uniform(-1, 1, (3, 16, 1000)).astype(np.float32)
    b = RNG.uniform(-1, 1, (3, 1000, 24)).astype(np.float32)
    ref = (_f64(a) @ _f64(b)).numpy()
    for splits in (1, 2, 7, 16):
        got = R.split_k_bmm(a, b, splits)
        assert max_rel_error(got, ref) < 1e-5
        assert np.array_equal(got, R.split_k_bmm(a, b, splits))
    assert np.array_equal(R.split_k_bmm(a, b, 1), R.bmm(a, b))
    # The fixed order: partial sums added as s = 0, 1, ..., S-1.
    chunks = [np.matmul(a[..., i * 250:(i + 1) * 250], b[..., i * 250:(i + 1) * 250, :]) for i in range(4)]
    ordered = ((chunks[0] + chunks[1]) + chunks[2]) + chunks[3]
    assert np.array_equal(R.split_k_bmm(a, b, 4), ordered)


# ---------------------------------------------------------------------------
# Packed layouts, against element loops of the reference's definitions.


def test_pack_layouts_match_element_definitions() -> None:
    a = RNG.normal(0, 1, (70, 45)).astype(np.float32)  # ragged: padding
    m, k = a.shape
    pa = R.pack_a_blocked(a)
    assert pa.shape == (3, 2, 32, 32)
    for i in range(3):
        for j in range(2):
            for r in range(32):
                for c in range(32):
                    row, col = 32 * i + r, 32 * j + c
                    want = a[row, col] if row < m and col < k else 0.0
                    assert pa[i, j, r, c] == want
    b = a  # as B [K=70, N=45]
    pb = R.pack_b_blocked(b)
    vn = R.pack_b_blocked_vnni(b)
    assert pb.shape == (2, 3, 32, 32) and vn.shape == (2, 3, 16, 32, 2)
    for j in range(2):
        for i in range(3):
            for r in range(32):
                for c in range(32):
                    kk, nn = 32 * i + r, 32 * j + c
                    want = b[kk, nn] if kk < 70 and nn < 45 else 0.0
                    assert pb[j, i, r, c] == want
                    # out[j, i, r, n, p] = B[32i + 2r + p, 32j + n] (matmul.py:952-953)
                    assert vn[j, i, r // 2, c, r % 2] == want
    bt = RNG.normal(0, 1, (45, 70)).astype(np.float32)  # [N, K]
    pv = R.pack_b_vnni_t(bt, 32)
    assert pv.shape == (2, 48, 32, 2)
    for jp in range(2):
        for c in range(48):
            for nn in range(32):
                for p in range(2):
                    row, col = 32 * jp + nn, 2 * c + p
                    want = bt[row, col] if row < 45 and col < 70 else 0.0
                    assert pv[jp, c, nn, p] == want
    bp = R.pack_b_panels(RNG.normal(0, 1, (12, 64)).astype(np.float32), 16)
    src = bp  # [N/16, K, 16]
    assert src.shape == (4, 12, 16)


def test_pack_layouts_match_reference_closed_forms() -> None:
    # The reference's own closed forms (tests/test_mlir_execution.py:1963-1981),
    # written with torch reshape/permute.
    for rows, cols in [(128, 96), (70, 45)]:
        x = RNG.normal(0, 1, (rows, cols)).astype(np.float32)
        r, c = -(-rows // 32) * 32, -(-cols // 32) * 32
        padded = F.pad(torch.from_numpy(x), (0, c - cols, 0, r - rows))
        a4 = padded.reshape(r // 32, 32, c // 32, 32).permute(0, 2, 1, 3)
        b4 = padded.reshape(r // 32, 32, c // 32, 32).permute(2, 0, 1, 3)
        vnni = b4.reshape(c // 32, r // 32, 16, 2, 32).transpose(3, 4)
        assert np.array_equal(R.pack_a_blocked(x), a4.numpy())
        assert np.array_equal(R.pack_b_blocked(x), b4.numpy())
        assert np.array_equal(R.pack_b_blocked_vnni(x), vnni.numpy())


def test_panel_packs_match_element_definitions() -> None:
    b = RNG.normal(0, 1, (10, 48)).astype(np.float32)
    p = R.pack_b_panels(b, 16)
    for j in range(3):
        for kk in range(10):
            for nn in range(16):
                assert p[j, kk, nn] == b[kk, 16 * j + nn]
    a = RNG.normal(0, 1, (7, 24)).astype(np.float32)
    q = R.pack_a_panels(a, 8)
    for kb in range(3):
        for mm in range(7):
            for t in range(8):
                assert q[kb, mm, t] == a[mm, 8 * kb + t]


# ---------------------------------------------------------------------------
# Reductions and elementwise


def test_reductions_match_float64() -> None:
    x = RNG.normal(0, 1, (33, 517)).astype(np.float32)
    v = RNG.normal(0, 1, 517).astype(np.float32)
    t = _f64(x)
    np.testing.assert_allclose(R.row_sum(x), t.sum(1, keepdim=True).numpy(), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(R.column_sum(x), t.sum(0).numpy(), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(R.row_dot(x, v), (t @ _f64(v)).reshape(-1, 1).numpy(), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(R.matvec(x, v), (t @ _f64(v)).reshape(-1, 1).numpy(), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(R.row_sum(x, "relu"), torch.relu(t.sum(1, keepdim=True)).numpy(), rtol=1e-5, atol=1e-4)
    neg_zero = np.array([[-0.0, 1.0]], np.float32)
    assert np.signbit(R.column_sum(neg_zero)[0]) == False  # noqa: E712  (+0.0, reduction.py:151-153)


def test_elementwise_match_torch() -> None:
    x = np.concatenate([RNG.normal(0, 2, 1000), [0.0, -0.0, np.nan]]).astype(np.float32)
    t = torch.from_numpy(x)
    np.testing.assert_array_equal(R.relu(x), torch.relu(t).numpy())
    np.testing.assert_array_equal(R.leaky_relu(x, 0.1), F.leaky_relu(t, 0.1).numpy())
    np.testing.assert_array_equal(R.scalar_mul(x, 2.5), (t * 2.5).numpy())
