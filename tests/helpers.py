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


# ---------------------------------------------------------------------------
# Adversarial inputs: the values where an op's answer changes (signed zeros,
# infinities, NaN, the smallest normal and the largest finite value of the
# dtype, and the dtype's neighbours of given constants), laid out so that
# neighbouring rows, neighbouring columns and columns 16 or 64 apart hold
# different values: a kernel that reads the wrong row or lane cannot pass.
# The reference's tests use values of this kind (tests/inputs.py:22-76).


def special_values(dtype: str, constants: tuple[float, ...] = (), finite: bool = False,
                   largest: bool = True) -> list[float]:
    """±0, ±inf, NaN, ±tiny, ±max of ``dtype`` ('f32'/'bf16') and, for each
    constant, its value in ``dtype`` and the two neighbouring values, both
    signs; ``finite`` drops inf and NaN, ``largest=False`` drops ±max (for
    sums, whose overflow would depend on the order of the terms)."""
    tdt = DTYPES[dtype]
    info = torch.finfo(tdt)
    values = [0.0, -0.0, float(info.tiny), -float(info.tiny)]
    if largest:
        values += [float(info.max), -float(info.max)]
    if not finite:
        values += [float("inf"), float("-inf"), float("nan")]
    for c in constants:
        at = torch.tensor(c, dtype=torch.float64).to(tdt)
        for v in (at, torch.nextafter(at, torch.tensor(float("-inf"), dtype=tdt)),
                  torch.nextafter(at, torch.tensor(float("inf"), dtype=tdt))):
            values += [float(v), -float(v)]
    out, seen = [], set()
    for v in values:
        key = np.float64(v).tobytes()
        if key not in seen:
            seen.add(key)
            out.append(v)
    return out


def spread(values: list[float], rows: int, cols: int, extra: float = 3.0) -> np.ndarray:
    """``values`` over [rows, cols] as float32: element (r, c) is value
    (r + c) mod count. The count is made odd (one more value, ``extra``), so
    it divides neither 16 nor 64: columns 16 or 64 apart, and neighbouring
    rows and columns, differ."""
    vals = list(values)
    if len(vals) % 2 == 0:
        vals.append(extra)
    idx = (np.arange(rows)[:, None] + np.arange(cols)[None, :]) % len(vals)
    return np.asarray(vals, dtype=np.float64)[idx].astype(np.float32)


def assert_specials_close(got: np.ndarray, ref: np.ndarray, rtol: float, atol: "float | np.ndarray") -> None:
    """The same NaNs and the same infinities (by sign) as ``ref``; every
    finite element within ``atol + rtol * |ref|`` (``atol`` a scalar or an
    array broadcast to ``ref``'s shape)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    atol = np.broadcast_to(np.asarray(atol, np.float64), ref.shape)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    for what, fn in (("NaN", np.isnan), ("+inf", np.isposinf), ("-inf", np.isneginf)):
        bad = fn(got) != fn(ref)
        if bad.any():
            at = np.argwhere(bad)[:5]
            detail = [(tuple(i), got[tuple(i)], ref[tuple(i)]) for i in at]
            raise AssertionError(f"{int(bad.sum())} {what} elements differ: {detail}")
    fin = np.isfinite(ref)
    assert_close(got[fin], ref[fin], rtol, atol[fin])


def tile_rows(rng: np.random.Generator, m: int, per_band: int = 2, band: int = 128) -> np.ndarray:
    """Sorted row indices, ``per_band`` drawn from every ``band``-row slice of
    ``m`` rows (the last, ragged slice included). Checked over all columns,
    such a sample meets every 128- or 256-row tile of a GEMM's output, which a
    plain random sample of rows does not promise."""
    picks = []
    for start in range(0, m, band):
        stop = min(m, start + band)
        picks.append(rng.choice(np.arange(start, stop), min(per_band, stop - start), replace=False))
    return np.sort(np.concatenate(picks))
