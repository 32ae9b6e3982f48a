"""Shared helpers of the tests: seeded inputs, tolerance checks, dtype maps."""

from __future__ import annotations

import numpy as np
import torch

from oracle import restate as R

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16}


def to_np(t: torch.Tensor) -> np.ndarray:
    """A tensor's values as float32 numpy (bf16 widened exactly)."""
    return t.detach().float().cpu().numpy()


def tensor(x: np.ndarray, dtype: str, device: torch.device | str = "cpu") -> torch.Tensor:
    """numpy float32 values as a tensor of ``dtype`` ('f32' or 'bf16'); bf16
    values are rounded to nearest even, as the oracle rounds them."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to(DTYPES[dtype]).to(device)


def rounded(x: np.ndarray, dtype: str) -> np.ndarray:
    """The values a tensor of ``dtype`` holds for ``x``."""
    return R.round_to(np.asarray(x, np.float32), dtype)


def max_rel_error(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the reference's error measure,
    tests/test_cpu_utils_split_k_bmm.py:15-16)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (scale if scale > 0 else 1.0))


def assert_close(got: np.ndarray, ref: np.ndarray, rtol: float, atol: float) -> None:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    same_nan = np.isnan(got) == np.isnan(ref)
    assert same_nan.all(), f"NaN mismatch at {np.argwhere(~same_nan)[:5]}"
    ok = np.isnan(ref) | (np.abs(got - ref) <= atol + rtol * np.abs(ref))
    if not ok.all():
        bad = np.argwhere(~ok)[:5]
        detail = [(tuple(i), got[tuple(i)], ref[tuple(i)]) for i in bad]
        raise AssertionError(f"{(~ok).sum()} of {ok.size} elements off (rtol={rtol}, atol={atol}): {detail}")


def bf16_gemm_atol(k: int, a: np.ndarray, b: np.ndarray) -> float:
    """atol of bf16-in / f32-accumulate results: sqrt(K) * 2^-8 * rms(A) *
    rms(B) * 0.01 (with rtol 1e-2: rtol 1e-2 plus an atol scaled by sqrt(K))."""
    ra = float(np.sqrt(np.mean(np.square(a, dtype=np.float64)))) if a.size else 1.0
    rb = float(np.sqrt(np.mean(np.square(b, dtype=np.float64)))) if b.size else 1.0
    return float(np.sqrt(max(k, 1)) * 2.0**-8 * ra * rb * 0.01) + 1e-6
