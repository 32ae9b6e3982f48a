"""CPU oracle: a numpy restatement of the reference's hot-path arithmetic.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or the timed CPU baseline); the product path (``libhmx.so`` behind
``helion_mlir_utils``) never calls it.

Each function restates a kernel body of adam-smnk/helion-mlir-xsmm (paths
relative to the reference root) in numpy, in the reference's arithmetic
types: bf16 operands widened exactly to f32, f32 accumulation, epilogue on
the f32 accumulator, one rounding to the output dtype (round-to-nearest-even
for bf16, as torch's ``.to(torch.bfloat16)``). The reference's CPU pipeline
itself (Helion + MLIR + lighthouse, JIT-compiled AMX code) cannot run here,
so bit-level parity with its JIT'd kernels (K order after the AMX rewrite,
the polynomial ``exp``) is not pinned; every function is pinned instead to
closed forms, library routines and brute force in ``tests/test_oracle.py``.

bf16 data is carried as float32 arrays holding bf16-representable values
(``round_bf16``), or as uint16 bit patterns at the boundaries.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# ---------------------------------------------------------------------------
# bf16 <-> f32


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even; NaN stays
    a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=F32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def from_bf16_bits(h: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16, kept as float32."""
    return from_bf16_bits(bf16_bits(x))


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """The single rounding of a result to its output dtype ('f32' or 'bf16')."""
    x = np.asarray(x, dtype=F32)
    return round_bf16(x) if dtype == "bf16" else x


# ---------------------------------------------------------------------------
# Epilogue activations, in f32 (torch's definitions of the functions the
# reference's callers pass as ``epilogue``: matmul.py:321-327 applies them to
# the f32 accumulator).

ACTIVATIONS = ("identity", "relu", "silu", "sigmoid", "gelu", "gelu_tanh", "tanh", "leaky_relu")


def activation(name: str, x: np.ndarray, arg: float = 0.01) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        if name == "identity":
            return x
        if name == "relu":
            return np.where(x > 0, x, np.where(np.isnan(x), x, F32(0))).astype(F32)
        if name == "silu":
            return (x / (F32(1) + np.exp(-x))).astype(F32)
        if name == "sigmoid":
            return (F32(1) / (F32(1) + np.exp(-x))).astype(F32)
        if name == "gelu":
            from scipy.special import erf

            return (F32(0.5) * x * (F32(1) + erf(x / np.sqrt(F32(2))).astype(F32))).astype(F32)
        if name == "gelu_tanh":
            u = F32(np.sqrt(2.0 / np.pi)) * (x + F32(0.044715) * x * x * x)
            return (F32(0.5) * x * (F32(1) + np.tanh(u))).astype(F32)
        if name == "tanh":
            return np.tanh(x).astype(F32)
        if name == "leaky_relu":
            return np.where(x >= 0, x, x * F32(arg)).astype(F32)
    raise ValueError(f"unknown activation {name!r}")


# ---------------------------------------------------------------------------
# GEMM family


def apply_epilogue(act, x: np.ndarray, arg: float = 0.01, extra: np.ndarray | None = None) -> np.ndarray:
    """The epilogue on f32 values: a named activation (``activation``), or the
    caller's own callable applied to f32 tensors, as the reference applies
    ``epilogue(acc)`` to its f32 accumulator (helion_mlir_utils/matmul.py:321-327)
    and ``epilogue(y, extra)`` to f32 group-norm values (normalization.py:121)."""
    if not callable(act):
        return activation(act, x, arg)
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, dtype=F32))
    operands = (t,) if extra is None else (t, torch.from_numpy(np.ascontiguousarray(extra, dtype=F32)))
    with torch.no_grad():
        return act(*operands).numpy().astype(F32)


def _op(x: np.ndarray, trans: bool) -> np.ndarray:
    return np.asarray(x, dtype=F32).T if trans else np.asarray(x, dtype=F32)


def matmul(
    a: np.ndarray,
    b: np.ndarray,
    trans_a: bool = False,
    trans_b: bool = False,
    bias: np.ndarray | None = None,
    scale: np.ndarray | None = None,
    shift: np.ndarray | None = None,
    act="identity",
    act_arg: float = 0.01,
    out: str = "f32",
) -> np.ndarray:
    """``act((op(A) @ op(B) + bias) * scale + shift)`` with f32 accumulation
    and one rounding: helion_mlir_utils/matmul.py:294-327 (bf16 fused-pack,
    ``acc`` f32, ``+bias``, ``*scale``, ``+shift``, ``epilogue(acc).to(dtype)``),
    1332-1368 (f32 fused) and 156-228, 862-904 (blocked, bias, affine)."""
    acc = _op(a, trans_a) @ _op(b, trans_b)  # f32 x f32 -> f32 accumulation
    acc = acc.astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):  # IEEE overflow / NaN are results here
        if bias is not None:
            acc = acc + np.asarray(bias, dtype=F32)
        if scale is not None:
            acc = acc * np.asarray(scale, dtype=F32)
        if shift is not None:
            acc = acc + np.asarray(shift, dtype=F32)
    return round_to(apply_epilogue(act, acc, act_arg), out)


def bmm(a: np.ndarray, b: np.ndarray, out: str = "f32") -> np.ndarray:
    """Batched ``A @ B``, f32 accumulation, one rounding: matmul.py:1842-1855
    (f32 ``_bmm_direct``) and 1864-1882 (bf16 ``_bmm_batched``, bf16 result)."""
    acc = np.matmul(np.asarray(a, dtype=F32), np.asarray(b, dtype=F32)).astype(F32)
    return round_to(acc, out)


def split_k_bmm(a: np.ndarray, b: np.ndarray, splits: int, out: str = "f32") -> np.ndarray:
    """Batched ``A @ B`` as ``splits`` K chunks whose f32 partials are summed
    over the split index in increasing order: the reference's split-K
    (matmul.py:1195-1221: ``_split_k_partials`` writes ``[S, M, N]`` f32,
    ``_sum_partials`` reduces ``partials[:, tm, tn].sum(0)``), applied per
    batch slice. Chunks are ``ceil(K / splits)`` wide, the last one shorter."""
    a = np.asarray(a, dtype=F32)
    b = np.asarray(b, dtype=F32)
    k = a.shape[-1]
    chunk = -(-k // splits)
    total = None
    for s in range(splits):
        lo, hi = s * chunk, min(k, (s + 1) * chunk)
        if lo >= hi:
            continue
        part = np.matmul(a[..., lo:hi], b[..., lo:hi, :]).astype(F32)
        total = part if total is None else (total + part).astype(F32)
    if total is None:
        total = np.zeros(a.shape[:-1] + b.shape[-1:], dtype=F32)
    return round_to(total, out)


# ---------------------------------------------------------------------------
# Packed layouts (closed forms; the reference's kernels write them one 32x32
# block per iteration: matmul.py:92-153, 972-983; panels:
# benchmarks/helion_block_pack.py:40-62).


def _pad(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Zero padding to [rows, cols] (``pad_2d``, matmul.py:78-89)."""
    out = np.zeros((rows, cols), dtype=x.dtype)
    out[: x.shape[0], : x.shape[1]] = x
    return out


def pad_2d(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    return _pad(np.asarray(x), rows, cols)


def _up(v: int, b: int) -> int:
    return -(-v // b) * b


def pack_a_blocked(a: np.ndarray) -> np.ndarray:
    """``[M, K]`` -> ``[M/32, K/32, 32, 32]``: block (i, j) is A[32i:, 32j:]
    (matmul.py:92-99)."""
    m, k = a.shape
    p = _pad(a, _up(m, 32), _up(k, 32))
    return p.reshape(p.shape[0] // 32, 32, p.shape[1] // 32, 32).transpose(0, 2, 1, 3).copy()


def pack_b_blocked(b: np.ndarray) -> np.ndarray:
    """``[K, N]`` -> ``[N/32, K/32, 32, 32]``: block (j, i) is B[32i:, 32j:]
    (matmul.py:112-119)."""
    k, n = b.shape
    p = _pad(b, _up(k, 32), _up(n, 32))
    return p.reshape(p.shape[0] // 32, 32, p.shape[1] // 32, 32).transpose(2, 0, 1, 3).copy()


def pack_b_blocked_vnni(b: np.ndarray) -> np.ndarray:
    """``[K, N]`` -> ``[N/32, K/32, 16, 32, 2]`` with
    ``out[j, i, r, n, p] = B[32i + 2r + p, 32j + n]`` (matmul.py:132-140, 952-953)."""
    blocks = pack_b_blocked(b)  # [NB, KB, 32(k), 32(n)]
    nb, kb = blocks.shape[:2]
    return blocks.reshape(nb, kb, 16, 2, 32).transpose(0, 1, 2, 4, 3).copy()


def pack_b_vnni_t(b_t: np.ndarray, panel: int = 64) -> np.ndarray:
    """``[N, K]`` -> ``[N_pad/P, K_pad/2, P, 2]`` with N padded to panels and K
    to a multiple of 32: ``out[j, c, n, p] = B_t[jP + n, 2c + p]``
    (matmul.py:972-983, 1138-1157)."""
    n, k = b_t.shape
    p = _pad(b_t, _up(n, panel), _up(k, 32))
    np_, kp = p.shape
    return p.reshape(np_ // panel, panel, kp // 2, 2).transpose(0, 2, 1, 3).copy()


def pack_b_panels(b: np.ndarray, block_n: int) -> np.ndarray:
    """``[K, N]`` -> ``[N/BN, K, BN]`` (benchmarks/helion_block_pack.py:40-51)."""
    k, n = b.shape
    return b.reshape(k, n // block_n, block_n).transpose(1, 0, 2).copy()


def pack_a_panels(a: np.ndarray, block_k: int) -> np.ndarray:
    """``[M, K]`` -> ``[K/BK, M, BK]`` (benchmarks/helion_block_pack.py:54-62)."""
    m, k = a.shape
    return a.reshape(m, k // block_k, block_k).transpose(1, 0, 2).copy()


# ---------------------------------------------------------------------------
# Row kernels


def softmax(x: np.ndarray, out: str = "f32") -> np.ndarray:
    """Row softmax of helion_mlir_utils/normalization.py:47-72: f32 row max
    (NaN-propagating, as ``torch.maximum``), ``sum(exp(x - max))`` in f32,
    ``inv = 1 / sum``, ``(exp(x - max) * inv)`` rounded once. One column
    (normalization.py:76-87): ``x - x + 1``."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        if x.shape[1] == 1:
            return round_to(x - x + F32(1), out)
        mx = np.max(x, axis=1, keepdims=True)  # NaN-propagating
        e = np.exp(x - mx).astype(F32)
        inv = (F32(1) / e.sum(axis=1, keepdims=True, dtype=F32)).astype(F32)
        return round_to(e * inv, out)


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float, out: str = "f32") -> np.ndarray:
    """RMSNorm ``x * rsqrt(mean(x^2) + eps) * w`` in f32, rounded once. The
    reference has no RMSNorm; this is the standard definition, written in the
    reference's convention for row statistics (normalization.py:113-122: f32
    statistics, one rounding)."""
    x = np.asarray(x, dtype=F32)
    ms = (np.sum(x * x, axis=1, keepdims=True, dtype=F32) / F32(x.shape[1])).astype(F32)
    r = (F32(1) / np.sqrt(ms + F32(eps))).astype(F32)
    y = x * r
    if w is not None:
        y = y * np.asarray(w, dtype=F32)
    return round_to(y, out)


def group_norm(
    x: np.ndarray,
    groups: int,
    w: np.ndarray | None,
    b: np.ndarray | None,
    eps: float,
    extra: np.ndarray | None = None,
    extra_op: str | None = None,
    act="identity",
    act_arg: float = 0.01,
    out: str = "f32",
) -> np.ndarray:
    """GroupNorm of helion_mlir_utils/normalization.py:113-122 on ``[M, C]``
    viewed ``[M, G, C/G]``: f32 ``mean``, centered ``var``, ``centered *
    rsqrt(var + eps) * w + b``, ``epilogue(y, extra)``, one rounding."""
    x = np.asarray(x, dtype=F32)
    m, c = x.shape
    x3 = x.reshape(m, groups, c // groups)
    mean = (x3.sum(axis=2, keepdims=True, dtype=F32) / F32(c // groups)).astype(F32)
    centered = x3 - mean
    var = ((centered * centered).sum(axis=2, keepdims=True, dtype=F32) / F32(c // groups)).astype(F32)
    y = centered * (F32(1) / np.sqrt(var + F32(eps))).astype(F32)
    y = y.reshape(m, c)
    if w is not None:
        y = y * np.asarray(w, dtype=F32)
    if b is not None:
        y = y + np.asarray(b, dtype=F32)
    if extra_op == "add":
        y = y + np.asarray(extra, dtype=F32)
    elif extra_op == "mul":
        y = y * np.asarray(extra, dtype=F32)
    elif extra_op == "callable":  # act is the caller's epilogue(y, extra)
        extra_v = np.asarray(extra if extra is not None else w, dtype=F32)
        return round_to(apply_epilogue(act, y, act_arg, np.broadcast_to(extra_v, y.shape)), out)
    return round_to(apply_epilogue(act, y, act_arg), out)


def row_sum(x: np.ndarray, act="identity", out: str = "f32") -> np.ndarray:
    """``epilogue(x.sum(1, keepdim=True))`` in f32 (reduction.py:79-91)."""
    s = np.asarray(x, dtype=F32).sum(axis=1, keepdims=True, dtype=F32)
    return round_to(apply_epilogue(act, s), out)


def column_sum(x: np.ndarray) -> np.ndarray:
    """``x.sum(0)`` in f32, ``+0.0`` (reduction.py:124-163)."""
    return (np.asarray(x, dtype=F32).sum(axis=0, dtype=F32) + F32(0)).astype(F32)


def row_dot(x: np.ndarray, v: np.ndarray, act="identity", out: str = "f32") -> np.ndarray:
    """``epilogue(x @ v)`` in f32, ``[M, 1]`` (reduction.py:166-182)."""
    s = (np.asarray(x, dtype=F32) * np.asarray(v, dtype=F32)[None, :]).sum(axis=1, keepdims=True, dtype=F32)
    return round_to(apply_epilogue(act, s), out)


def matvec(a: np.ndarray, x: np.ndarray, out: str = "f32") -> np.ndarray:
    """``A @ x`` in f32, ``[M, 1]`` (reduction.py:24-37)."""
    s = (np.asarray(a, dtype=F32) * np.asarray(x, dtype=F32).reshape(1, -1)).sum(axis=1, keepdims=True, dtype=F32)
    return round_to(s, out)


def relu(x: np.ndarray, out: str = "f32") -> np.ndarray:
    """elementwise.py:14-18."""
    return round_to(activation("relu", x), out)


def leaky_relu(x: np.ndarray, slope: float = 0.01, out: str = "f32") -> np.ndarray:
    """elementwise.py:23-31 (``F.leaky_relu``: x if x > 0 else x * slope)."""
    x = np.asarray(x, dtype=F32)
    return round_to(np.where(x > 0, x, x * F32(slope)), out)


def scalar_mul(x: np.ndarray, s: float, out: str = "f32") -> np.ndarray:
    """elementwise.py:34-39."""
    with np.errstate(over="ignore", invalid="ignore"):
        return round_to(np.asarray(x, dtype=F32) * F32(s), out)
