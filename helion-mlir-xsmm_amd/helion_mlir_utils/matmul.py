"""GEMMs of the gpu target: one gfx950 kernel per call, epilogue fused.

Entry points and signatures are the reference's
(``helion_mlir_utils/matmul.py`` of adam-smnk/helion-mlir-xsmm):

- :func:`matmul` (``matmul.py:1446-1570``): ``epilogue((op(A) @ op(B) + bias) *
  scale + shift)``. bf16 inputs run ``v_mfma_f32_32x32x16_bf16`` with f32
  accumulation and one rounding to the output (bf16 by default, as the
  reference; ``out_dtype=torch.float32`` keeps f32). f32 inputs run
  ``v_mfma_f32_32x32x2_f32``. Any shape: partial edge tiles are masked in the
  kernel, not padded on the host. ``block_sizes`` (rows, columns, K chunk)
  requests the workgroup tile: the largest instantiated tile within it.
- :func:`bmm` (``matmul.py:1965-2006``): batch on the grid; K split into a
  fixed number of chunks when the grid would underfill the 256 CUs, partials
  summed in a fixed order (deterministic).
- :func:`matmul_prepacked_b` / :func:`matmul_prepacked_b_affine` /
  :func:`prepacked_b_call` (``matmul.py:1593-1839``): B already packed, read in
  place by the kernel's layout-aware loader (VNNI panels, 32 x 32 blocks,
  VNNI blocks, bench panels).
- ``pack_*`` (``matmul.py:907-970, 1138-1157``): the packings, as GPU kernels.

Unsupported operands raise ``ValueError`` (never a silent eager fallback);
mismatched ``bmm`` operands raise ``RuntimeError`` mentioning ``batch2``, as
the reference and ``torch.bmm`` do.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence
import ctypes

import torch
from torch import Tensor

from helion_mlir_backend import output_pool
from helion_mlir_backend._compiler import native
from helion_mlir_backend._compiler.prepared import GpuLaunch

from ._gpu import IDENTITY, SUPPORTED_DTYPES, Epilogue, epilogue_code, identity_epilogue, is_gpu, on_device

__all__ = [
    "BLOCK_K",
    "BLOCK_M",
    "BLOCK_N",
    "bmm",
    "identity_epilogue",
    "matmul",
    "matmul_prepacked_b",
    "matmul_prepacked_b_affine",
    "pack_a_blocked",
    "pack_a_blocked_t",
    "pack_b_blocked",
    "pack_b_blocked_t",
    "pack_b_blocked_vnni",
    "pack_b_blocked_vnni_t",
    "pack_b_vnni_t",
    "pack_a_panels",
    "pack_b_panels",
    "pad_2d",
    "prepacked_b_call",
    "supports",
]

# Block of the packed layouts (the reference's AMX tile, matmul.py:60-64).
BLOCK_M = 32
BLOCK_N = 32
BLOCK_K = 32
_SUPPORTED_DTYPES = SUPPORTED_DTYPES
# Columns of a VNNI panel and K pairs per pack tile of pack_b_vnni_t
# (matmul.py:345-347): K is padded to a multiple of 2 * _PANEL_PAIRS.
_VNNI_PANEL = 64
_PANEL_PAIRS = 16


def _round_up(value: int, block: int) -> int:
    return (value + block - 1) // block * block


def supports(a: Tensor, b: Tensor, trans_a: bool = False, trans_b: bool = False) -> bool:
    """Whether :func:`matmul` can run these operands on the gpu target: 2-D,
    same dtype (bf16 or f32), both on a ROCm device, matching K."""
    if a.dtype != b.dtype or a.dtype not in _SUPPORTED_DTYPES:
        return False
    if not is_gpu(a, b) or a.device != b.device:
        return False
    if a.dim() != 2 or b.dim() != 2:
        return False
    k_a = a.shape[0] if trans_a else a.shape[1]
    k_b = b.shape[1] if trans_b else b.shape[0]
    return k_a == k_b


def _storage(t: Tensor) -> tuple[Tensor, int, bool]:
    """``t`` (2-D) as a row-major buffer: ``(tensor, ld, flipped)`` where
    ``flipped`` says the buffer holds ``t``'s transpose (``t`` is a transposed
    view). Other layouts are made contiguous."""
    rows, cols = t.shape
    if rows > 1 and cols > 1:
        if t.stride(1) == 1 and t.stride(0) >= cols:
            return t, t.stride(0), False
        if t.stride(0) == 1 and t.stride(1) >= rows:
            return t, t.stride(1), True
    t = t.contiguous()
    return t, max(cols, 1), False


def _vector(v: Tensor | None, n: int, name: str, dtype: torch.dtype, device: torch.device) -> Tensor | None:
    """A per-column operand as a contiguous ``[n]`` of ``dtype`` (a ``[1]`` or
    0-d one broadcast, as ``_affine_vector`` does, matmul.py:1573-1590)."""
    if v is None:
        return None
    if not isinstance(v, Tensor):
        v = torch.tensor(float(v))
    if v.dim() > 1 or v.numel() not in (1, n):
        raise ValueError(
            f"{name} must be scalar or have shape (1,) or ({n},), got {tuple(v.shape)}"
        )
    v = v.to(device=device, dtype=dtype).reshape(-1)
    if v.numel() == 1 and n != 1:
        v = v.expand(n)
    return v.contiguous()


def _vectors(
    bias: Tensor | None, scale: Tensor | None, shift: Tensor | None, n: int, like: Tensor
) -> tuple[Tensor | None, Tensor | None, Tensor | None, int]:
    """bias/scale/shift in one dtype: f32 if any is f32 (or the GEMM is f32),
    else bf16, so no operand loses precision before the f32 epilogue."""
    given = [v for v in (bias, scale, shift) if isinstance(v, Tensor)]
    dtype = torch.float32
    if like.dtype == torch.bfloat16 and given and all(v.dtype == torch.bfloat16 for v in given):
        dtype = torch.bfloat16
    out = tuple(
        _vector(v, n, name, dtype, like.device)
        for v, name in ((bias, "bias"), (scale, "scale"), (shift, "shift"))
    )
    return out[0], out[1], out[2], native.dtype_code(dtype)


# hmx_gemm_plan results by problem: the plan is a pure function of these
# arguments, so a repeated shape skips the native call (bounded, cleared when
# full, like the reference's LRU of bound kernels, matmul.py:487-489).
_PLANS: dict[tuple, tuple[int, int, int, int, int]] = {}
_PLANS_MAX = 1024


def _plan(ab: int, m: int, n: int, k: int, batch: int, trans_a: bool, layout: int,
          splits: int, tiles: Sequence[int] | None, units: int = 0,
          epilogue: int = native.EPI_IDENTITY) -> tuple[int, int, int, int, int]:
    """hmx_gemm_plan for a device of ``units`` compute units (0: the
    library's default) and the epilogue code: (splits, tile_m, tile_n,
    tile_k, workspace bytes)."""
    tm, tn, tk = (list(tiles) + [0, 0, 0])[:3] if tiles else (0, 0, 0)
    key = (ab, m, n, k, batch, bool(trans_a), layout, splits, int(tm), int(tn), int(tk), units, epilogue)
    hit = _PLANS.get(key)
    if hit is not None:
        return hit
    out = [ctypes.c_int() for _ in range(4)]
    ws = ctypes.c_int64()
    native.check(
        native.lib().hmx_gemm_plan(ab, m, n, k, batch, int(trans_a), layout, splits, -1,
                                   int(tm), int(tn), int(tk), units, epilogue, *[ctypes.byref(o) for o in out],
                                   ctypes.byref(ws)),
        "hmx_gemm_plan",
    )
    plan = (out[0].value, out[1].value, out[2].value, out[3].value, ws.value)
    if len(_PLANS) >= _PLANS_MAX:
        _PLANS.clear()
    _PLANS[key] = plan
    return plan


def gemm_plan(a_dtype: torch.dtype, m: int, n: int, k: int, batch: int = 1,
              splits: int = 0, block_sizes: Sequence[int] | None = None,
              trans_b: bool = False, compute_units: int | None = None) -> dict[str, int]:
    """The launch the gpu GEMM makes for this problem: K splits, workgroup tile
    and workspace bytes (host-only; the GPU tile table that replaces the
    reference's CPU heuristics, matmul.py:368-446, 1257-1287). ``trans_b``
    plans for B stored [N, K] (``nn.Linear`` weights); tile (32, 32, 64) is
    the skinny kernel (at most 64 rows of A against such a B). The plan is
    for a device of ``compute_units`` CUs: by default the current ROCm
    device's, or MI355X's 256 where none is visible."""
    if compute_units is None:
        compute_units = native.device_units(torch.device("cuda") if torch.cuda.is_available() else None)
    s, tm, tn, tk, ws = _plan(native.dtype_code(a_dtype), m, n, k, batch, False,
                              native.B_TRANS if trans_b else native.B_ROW, splits, block_sizes,
                              int(compute_units))
    return {"splits": s, "tile_m": tm, "tile_n": tn, "tile_k": tk, "workspace_bytes": ws}


class GemmLaunch(GpuLaunch):
    """One ``hmx_gemm`` problem with everything but the operand and output
    data pointers bound: the plan (splits, workspace bytes), shapes, strides,
    layout, epilogue and per-column vectors. A call allocates C (and the
    workspace, from torch's caching allocator), reads the current stream and
    makes the one native call -- the prepared launch that stands in for the
    reference's ``PreparedRun`` (``native/call.cpp:703-830``). The bound
    vectors are kept alive by the launch."""

    __slots__ = ("_fn", "_args", "_vectors", "_ws_bytes", "_staged_ws", "_rows_ok", "_device", "_shape",
                 "_dtype", "splits", "calls")

    def __init__(
        self, ab: int, c_dtype: torch.dtype, device: torch.device, c_shape: tuple[int, ...],
        lda: int, trans_a: bool, ldb: int, layout: int, panel: int, kpad: int,
        m: int, n: int, k: int, batch: int = 1, stride_a: int = 0, stride_b: int = 0,
        stride_c: int = 0, bias: Tensor | None = None, scale: Tensor | None = None,
        shift: Tensor | None = None, vec_dtype: int = native.DTYPE_F32,
        epilogue: Epilogue = IDENTITY, splits: int = 0,
        tiles: Sequence[int] | None = None,
    ) -> None:
        # The launch passes the plan's own splits and tile back with a
        # workspace of the planned size, which reproduces the plan exactly.
        s, tm, tn, tk, ws_bytes = _plan(ab, m, n, k, batch, trans_a, layout, splits, tiles,
                                        native.device_units(device), epilogue[0])
        self._fn = native.lib().hmx_gemm
        # The bound vectors and the epilogue program stay alive with the launch.
        self._vectors = (bias, scale, shift, epilogue[2])
        # The arguments of hmx_gemm in order (include/hmx.h); slots 2 (A),
        # 5 (B), 10 (C), 27 (workspace) and 32 (stream) are filled per call.
        self._args = [
            ab, native.dtype_code(c_dtype),
            None, lda, int(trans_a),
            None, ldb, layout, panel, kpad,
            None, n,
            m, n, k,
            batch, stride_a, stride_b, stride_c,
            native.ptr(bias), native.ptr(scale), native.ptr(shift), vec_dtype,
            epilogue[0], epilogue[1], native.program_arg(epilogue[2]),
            s, None, ws_bytes,
            int(tm), int(tn), int(tk),
            None,
        ]
        self._ws_bytes = ws_bytes
        # The plan assumes operands in 16-byte aligned rows. An epilogue
        # program on operands that are not runs staged (f32 partials, then
        # the reduction) and needs the partials too: such calls pass a larger
        # workspace.
        partials = batch * m * n * 4
        program = epilogue[0] == native.EPI_PROGRAM and layout in (native.B_ROW, native.B_TRANS)
        self._staged_ws = ws_bytes + partials if program and ws_bytes < partials else None
        vec = 8 if ab == native.DTYPE_BF16 else 4
        self._rows_ok = all(v % vec == 0 for v in (lda, ldb, stride_a, stride_b))
        self._device = device
        self._shape = c_shape
        self._dtype = c_dtype
        self.splits = s
        self.calls = 0  # launches made

    def plan(self) -> dict[str, int]:
        """The bound plan: K splits, workgroup tile and workspace bytes."""
        return {"splits": self.splits, "tile_m": int(self._args[29]), "tile_n": int(self._args[30]),
                "tile_k": int(self._args[31]), "workspace_bytes": self._ws_bytes}

    def unbind_vectors(self) -> None:
        """Drop the references to the bound bias, scale and shift: every later
        call passes its own (``run(..., vectors=...)``)."""
        self._vectors = (None, None, None, self._vectors[3])

    def __call__(self, a: Tensor, b: Tensor) -> Tensor:
        """C = the bound GEMM of ``a`` and ``b`` in a fresh output (the
        :class:`~helion_mlir_backend.PreparedCall` protocol)."""
        return self.run(a, b)

    def run(self, a: Tensor, b: Tensor, c: Tensor | None = None,
            vectors: tuple[Tensor | None, Tensor | None, Tensor | None] | None = None) -> Tensor:
        """C = the bound GEMM of ``a`` and ``b`` (buffers as planned);
        ``vectors`` replaces the bound bias, scale and shift by tensors of the
        same presence and dtype."""
        if c is None:
            c = output_pool.empty(self._shape, dtype=self._dtype, device=self._device)
        args = list(self._args)
        args[2] = a.data_ptr()
        args[5] = b.data_ptr()
        args[10] = c.data_ptr()
        if vectors is not None:
            args[19], args[20], args[21] = (None if v is None else v.data_ptr() for v in vectors)
        ws = None
        ws_bytes = self._ws_bytes
        if self._staged_ws is not None and (not self._rows_ok or a.data_ptr() % 16 or b.data_ptr() % 16):
            ws_bytes = self._staged_ws
            args[28] = ws_bytes
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=self._device)
            args[27] = ws.data_ptr()
        device = self._device
        if device.index is None or device.index == torch.cuda.current_device():
            native.ensure_device(device)
            args[32] = native.stream_of(device)
            status = self._fn(*args)
        else:
            with on_device(device) as stream:
                args[32] = stream
                status = self._fn(*args)
        native.count_call()
        if status:
            native.check(status, "hmx_gemm")
        self.calls += 1
        return c


# Bound GEMM launches of eager calls, by everything a launch binds except the
# data pointers: a repeated problem is a pointer patch and one native call
# (the reference likewise keeps bound kernels in an LRU, matmul.py:470-523).
# Bounded, cleared when full. A launch holds its epilogue program, so the
# program's id in the key cannot be reused while the entry lives.
_LAUNCHES: dict[tuple, GemmLaunch] = {}
_LAUNCHES_MAX = 256


def _launch_gemm(
    a: Tensor, lda: int, trans_a: bool,
    b: Tensor, ldb: int, layout: int, panel: int, kpad: int,
    c: Tensor, m: int, n: int, k: int,
    batch: int = 1, stride_a: int = 0, stride_b: int = 0, stride_c: int = 0,
    bias: Tensor | None = None, scale: Tensor | None = None, shift: Tensor | None = None,
    vec_dtype: int = native.DTYPE_F32, epilogue: Epilogue = IDENTITY,
    splits: int = 0, tiles: Sequence[int] | None = None,
) -> Tensor:
    key = (a.dtype, c.dtype, a.device, tuple(c.shape), lda, trans_a, ldb, layout, panel, kpad, m, n, k, batch,
           stride_a, stride_b, stride_c, bias is None, scale is None, shift is None, vec_dtype, epilogue[0],
           epilogue[1], id(epilogue[2]), splits, None if tiles is None else tuple(tiles))
    launch = _LAUNCHES.get(key)
    if launch is None:
        launch = GemmLaunch(
            native.dtype_code(a.dtype), c.dtype, a.device, tuple(c.shape), lda, trans_a, ldb, layout,
            panel, kpad, m, n, k, batch, stride_a, stride_b, stride_c, bias, scale, shift, vec_dtype,
            epilogue, splits, tiles,
        )
        launch.unbind_vectors()
        if len(_LAUNCHES) >= _LAUNCHES_MAX:
            _LAUNCHES.clear()
        _LAUNCHES[key] = launch
    return launch.run(a, b, c, (bias, scale, shift))


def matmul(
    a: Tensor,
    b: Tensor,
    trans_a: bool = False,
    trans_b: bool = False,
    bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    block_sizes: Sequence[int] | None = None,
    scale: Tensor | None = None,
    shift: Tensor | None = None,
    *,
    out_dtype: torch.dtype | None = None,
) -> Tensor:
    """``epilogue((op(A) @ op(B) + bias) * scale + shift)``, ``op`` transposing
    with ``trans_a``/``trans_b`` (reference ``matmul.py:1446-1570``).

    One kernel: A and B are read in place (a transposed view is read as its
    transpose, not copied), bias/scale/shift (``[N]``, or ``[1]`` for
    scale/shift) and the epilogue are applied to the f32 accumulator, and C
    is rounded once. The result dtype is ``a.dtype`` unless ``out_dtype``
    says otherwise.

    Raises ``ValueError`` for operands :func:`supports` rejects and for
    epilogues the kernel cannot fuse.
    """
    if not supports(a, b, trans_a=trans_a, trans_b=trans_b):
        raise ValueError(
            f"matmul() does not support these operands (trans_a={trans_a}, "
            f"trans_b={trans_b}): a.shape={tuple(a.shape)} a.dtype={a.dtype} "
            f"a.device={a.device}, b.shape={tuple(b.shape)} b.dtype={b.dtype} "
            f"b.device={b.device}. dtype must be one of {_SUPPORTED_DTYPES}, "
            "both tensors must be 2-D on the same ROCm (gfx950) device with a "
            "matching contracted dim. Check supports() before calling, or use "
            "torch.matmul directly for unsupported cases."
        )
    code = epilogue_code(epilogue)
    m = int(a.shape[1]) if trans_a else int(a.shape[0])
    n = int(b.shape[0]) if trans_b else int(b.shape[1])
    k = int(a.shape[0]) if trans_a else int(a.shape[1])
    out_dtype = a.dtype if out_dtype is None else out_dtype
    native.dtype_code(out_dtype)
    c = output_pool.empty((m, n), dtype=out_dtype, device=a.device)
    if m == 0 or n == 0:
        return c
    if k == 0:
        # An empty contraction: the epilogue of zeros, through the same kernel.
        a = torch.zeros((m, 1), dtype=a.dtype, device=a.device)
        b = torch.zeros((1, n), dtype=b.dtype, device=b.device)
        trans_a = trans_b = False
        k = 1
    bias, scale, shift, vec_dtype = _vectors(bias, scale, shift, n, a)
    a_buf, lda, a_flip = _storage(a)
    b_buf, ldb, b_flip = _storage(b)
    kernel_trans_a = trans_a != a_flip
    b_is_nk = trans_b != b_flip
    layout = native.B_TRANS if b_is_nk else native.B_ROW
    return _launch_gemm(
        a_buf, lda, kernel_trans_a, b_buf, ldb, layout, 0, 0, c, m, n, k,
        bias=bias, scale=scale, shift=shift, vec_dtype=vec_dtype, epilogue=code,
        tiles=block_sizes,
    )


def bmm(a: Tensor, b: Tensor, *, out_dtype: torch.dtype | None = None, splits: int | None = None) -> Tensor:
    """Batched ``A @ B`` (reference ``matmul.py:1965-2006``): one kernel, the
    batch on the grid. f32 runs the f32 MFMA, bf16 the bf16 MFMA with f32
    accumulation and a bf16 result (``out_dtype`` may ask for f32). When the
    output tiles underfill the GPU, K is split into ``splits`` chunks (default:
    chosen by the tile table) whose f32 partials are summed in a fixed order.
    """
    if a.dim() != 3:
        raise RuntimeError(f"batch1 must be a 3D tensor, got {a.dim()}D")
    batch, m, k = a.shape
    if b.dim() != 3 or b.shape[0] != batch or b.shape[1] != k:
        raise RuntimeError(
            "Expected size for first two dimensions of batch2 tensor to be: "
            f"[{batch}, {k}] but got: {list(b.shape[:2])}."
        )
    n = int(b.shape[2])
    if a.dtype != b.dtype or a.dtype not in _SUPPORTED_DTYPES or not is_gpu(a, b) or a.device != b.device:
        raise ValueError(
            f"bmm() does not support these operands: a {a.dtype} on {a.device}, "
            f"b {b.dtype} on {b.device}; both must be float32 or bfloat16 on one ROCm device"
        )
    out_dtype = a.dtype if out_dtype is None else out_dtype
    c = output_pool.empty((batch, m, n), dtype=out_dtype, device=a.device)
    if batch == 0 or m == 0 or n == 0:
        return c
    if k == 0:
        return c.zero_()
    if a.stride(2) != 1 or a.stride(1) < k:
        a = a.contiguous()
    if b.stride(2) != 1 or b.stride(1) < n:
        b = b.contiguous()
    return _launch_gemm(
        a, a.stride(1), False, b, b.stride(1), native.B_ROW, 0, 0, c, m, n, k,
        batch=batch, stride_a=a.stride(0), stride_b=b.stride(0), stride_c=m * n,
        splits=0 if splits is None else int(splits),
    )


# ---------------------------------------------------------------------------
# Packing (reference matmul.py:78-153, 907-983, 1138-1157; bench panels of
# benchmarks/helion_block_pack.py:40-81).


def _pack(kind: int, src: Tensor, rows_pad: int, cols_pad: int, out_shape: tuple[int, ...],
          panel: int = 0) -> Tensor:
    if not is_gpu(src) or src.dtype not in _SUPPORTED_DTYPES or src.dim() != 2:
        raise ValueError(
            f"pack expects a 2-D float32/bfloat16 tensor on a ROCm device, got "
            f"{tuple(src.shape)} {src.dtype} on {src.device}"
        )
    src = src.contiguous()
    out = output_pool.empty(out_shape, dtype=src.dtype, device=src.device)
    rows, cols = map(int, src.shape)
    with on_device(src.device) as stream:
        native.call("hmx_pack", kind, native.dtype_code(src.dtype), src.data_ptr(), rows, cols,
                    max(cols, 1), out.data_ptr(), rows_pad, cols_pad, panel, stream)
    return out


def pad_2d(x: Tensor, rows: int, cols: int) -> Tensor:
    """Contiguous ``x`` zero-padded to ``[rows, cols]`` (``matmul.py:87-89``)."""
    return _pack(native.PACK_PAD, x, rows, cols, (rows, cols))


def pack_a_blocked(a: Tensor, m_pad: int | None = None, k_pad: int | None = None) -> Tensor:
    """Row-major ``[M, K]`` into ``[M/BM, K/BK, BM, BK]`` (``matmul.py:907-915``)."""
    m, k = map(int, a.shape)
    mp = _round_up(m, BLOCK_M) if m_pad is None else m_pad
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    return _pack(native.PACK_A_BLOCKED, a, mp, kp, (mp // 32, kp // 32, 32, 32))


def pack_a_blocked_t(a_t: Tensor, m_pad: int | None = None, k_pad: int | None = None) -> Tensor:
    """Transposed ``[K, M]`` into ``[M/BM, K/BK, BM, BK]`` (``matmul.py:917-925``)."""
    k, m = map(int, a_t.shape)
    mp = _round_up(m, BLOCK_M) if m_pad is None else m_pad
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    return _pack(native.PACK_A_BLOCKED_T, a_t, mp, kp, (mp // 32, kp // 32, 32, 32))


def pack_b_blocked(b: Tensor, k_pad: int | None = None, n_pad: int | None = None) -> Tensor:
    """Row-major ``[K, N]`` into ``[N/BN, K/BK, BK, BN]`` (``matmul.py:927-935``)."""
    k, n = map(int, b.shape)
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    np_ = _round_up(n, BLOCK_N) if n_pad is None else n_pad
    return _pack(native.PACK_B_BLOCKED, b, kp, np_, (np_ // 32, kp // 32, 32, 32))


def pack_b_blocked_t(b_t: Tensor, k_pad: int | None = None, n_pad: int | None = None) -> Tensor:
    """Transposed ``[N, K]`` into ``[N/BN, K/BK, BK, BN]`` (``matmul.py:937-945``)."""
    n, k = map(int, b_t.shape)
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    np_ = _round_up(n, BLOCK_N) if n_pad is None else n_pad
    return _pack(native.PACK_B_BLOCKED_T, b_t, kp, np_, (np_ // 32, kp // 32, 32, 32))


def pack_b_blocked_vnni(b: Tensor, k_pad: int | None = None, n_pad: int | None = None) -> Tensor:
    """Row-major ``[K, N]`` into VNNI blocks ``[N/BN, K/BK, BK/2, BN, 2]``:
    ``out[j, i, r, n, p] = B[32i + 2r + p, 32j + n]`` (``matmul.py:947-959``)."""
    k, n = map(int, b.shape)
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    np_ = _round_up(n, BLOCK_N) if n_pad is None else n_pad
    return _pack(native.PACK_B_BLOCKED_VNNI, b, kp, np_, (np_ // 32, kp // 32, 16, 32, 2))


def pack_b_blocked_vnni_t(b_t: Tensor, k_pad: int | None = None, n_pad: int | None = None) -> Tensor:
    """Transposed ``[N, K]`` into the layout of :func:`pack_b_blocked_vnni` of
    ``b_t.T`` (``matmul.py:962-970``)."""
    n, k = map(int, b_t.shape)
    kp = _round_up(k, BLOCK_K) if k_pad is None else k_pad
    np_ = _round_up(n, BLOCK_N) if n_pad is None else n_pad
    return _pack(native.PACK_B_BLOCKED_VNNI_T, b_t, kp, np_, (np_ // 32, kp // 32, 16, 32, 2))


def pack_b_vnni_t(b_t: Tensor, panel: int = _VNNI_PANEL) -> Tensor:
    """Transposed ``[N, K]`` (K even) into column panels of the VNNI layout of
    ``b_t.T``, ``[N_pad/P, K_pad/2, P, 2]`` with ``P = panel`` (a multiple of
    32), N padded to whole panels and K to a multiple of 32
    (``matmul.py:1138-1157``)."""
    n, k = map(int, b_t.shape)
    if k % 2 or panel % BLOCK_N or panel <= 0:
        raise ValueError(
            f"pack_b_vnni_t() needs an even K and a panel of a multiple of "
            f"{BLOCK_N} columns, got b_t.shape={(n, k)}, panel={panel}"
        )
    n_pad, k_pad = _round_up(n, panel), _round_up(k, 2 * _PANEL_PAIRS)
    return _pack(native.PACK_B_VNNI_PANELS_T, b_t, k_pad, n_pad,
                 (n_pad // panel, k_pad // 2, panel, 2), panel)


def pack_b_panels(b: Tensor, block_n: int | None = None) -> Tensor:
    """``[K, N]`` into panel-major ``[N/block_n, K, block_n]``
    (``benchmarks/helion_block_pack.py:66-71``). Also takes the benchmark's
    own form, a ``[K, N/BN, BN]`` view with no ``block_n``
    (``helion_block_pack.py:40-51``)."""
    if b.dim() == 3 and block_n is None:
        k, panels, block_n = map(int, b.shape)
        b = b.reshape(k, panels * block_n)
    if block_n is None:
        raise ValueError("pack_b_panels() of a 2-D [K, N] tensor needs block_n")
    k, n = map(int, b.shape)
    if block_n <= 0 or n % block_n:
        raise ValueError(f"N={n} is not a multiple of block_n={block_n}")
    return _pack(native.PACK_B_PANELS, b, k, n, (n // block_n, k, block_n), block_n)


def pack_a_panels(a: Tensor, block_k: int | None = None) -> Tensor:
    """``[M, K]`` into ``[K/block_k, M, block_k]``
    (``benchmarks/helion_block_pack.py:74-79``). Also takes the benchmark's
    own form, a ``[M, K/BK, BK]`` view with no ``block_k``
    (``helion_block_pack.py:54-62``)."""
    if a.dim() == 3 and block_k is None:
        m, panels, block_k = map(int, a.shape)
        a = a.reshape(m, panels * block_k)
    if block_k is None:
        raise ValueError("pack_a_panels() of a 2-D [M, K] tensor needs block_k")
    m, k = map(int, a.shape)
    if block_k <= 0 or k % block_k:
        raise ValueError(f"K={k} is not a multiple of block_k={block_k}")
    return _pack(native.PACK_A_PANELS, a, m, k, (k // block_k, m, block_k), block_k)


# ---------------------------------------------------------------------------
# GEMMs with a packed B.


def _packed_layout(a: Tensor, b4: Tensor, n: int) -> tuple[int, int, int, int]:
    """(layout, panel, K extent of the packing, N extent of the packing) of a
    packed RHS, or ``ValueError`` if it does not fit ``a`` and ``n``."""
    m, k = map(int, a.shape)
    shape = tuple(map(int, b4.shape))
    if b4.dim() == 4 and shape[-1] == 2:  # pack_b_vnni_t: [N/P, K/2, P, 2]
        panels, pairs, panel, _ = shape
        if (
            a.dtype != torch.bfloat16
            or panel % BLOCK_N
            or k % 2
            or 2 * pairs != _round_up(k, 2 * _PANEL_PAIRS)
            or _round_up(n, panel) != panels * panel
        ):
            raise ValueError(
                f"VNNI-packed RHS {shape} {b4.dtype} is incompatible with "
                f"a.shape={(m, k)} {a.dtype} and n={n}"
            )
        return native.B_VNNI_PANELS, panel, 2 * pairs, panels * panel
    if b4.dim() == 4:  # pack_b_blocked[_t]: [N/32, K/32, 32, 32]
        blocks_n, blocks_k, block_k, block_n = shape
        if block_k != BLOCK_K or block_n != BLOCK_N:
            raise ValueError(
                f"invalid packed RHS block shape {shape}; expected trailing dimensions "
                f"({BLOCK_K}, {BLOCK_N})"
            )
        if (
            blocks_k * BLOCK_K != _round_up(k, BLOCK_K)
            or not 0 < n <= blocks_n * BLOCK_N
            or _round_up(n, BLOCK_N) != blocks_n * BLOCK_N
        ):
            raise ValueError(
                f"packed RHS shape {shape} is incompatible with a.shape={(m, k)} and n={n}"
            )
        return native.B_BLOCKED, 32, blocks_k * BLOCK_K, blocks_n * BLOCK_N
    if b4.dim() == 5:  # pack_b_blocked_vnni[_t]: [N/32, K/32, 16, 32, 2]
        blocks_n, blocks_k, half, block_n, two = shape
        if (
            (half, block_n, two) != (16, 32, 2)
            or a.dtype != torch.bfloat16
            or blocks_k * BLOCK_K != _round_up(k, BLOCK_K)
            or _round_up(n, BLOCK_N) != blocks_n * BLOCK_N
        ):
            raise ValueError(
                f"VNNI-blocked RHS {shape} {b4.dtype} is incompatible with "
                f"a.shape={(m, k)} {a.dtype} and n={n}"
            )
        return native.B_BLOCKED_VNNI, 32, blocks_k * BLOCK_K, blocks_n * BLOCK_N
    if b4.dim() == 3:  # bench panels: [N/P, K, P] (bf16 or f32)
        panels, kk, panel = shape
        if (
            kk != k
            or panel % 8
            or _round_up(n, panel) != panels * panel
        ):
            raise ValueError(
                f"panel-packed RHS {shape} {b4.dtype} is incompatible with "
                f"a.shape={(m, k)} {a.dtype} and n={n}"
            )
        return native.B_PANELS, panel, kk, panels * panel
    raise ValueError(
        f"matmul_prepacked_b() expects rank-2 a and a packed b4 (rank 3-5), got "
        f"a.shape={(m, k)} and b4.shape={shape}"
    )


def _check_prepacked(a: Tensor, b4: Tensor, bias: Tensor | None, n: int) -> None:
    if a.dim() != 2:
        raise ValueError(
            f"matmul_prepacked_b() expects rank-2 a and rank-4 b4, got "
            f"a.shape={tuple(a.shape)} and b4.shape={tuple(b4.shape)}"
        )
    if a.dtype != b4.dtype or a.device != b4.device:
        raise ValueError(
            "matmul_prepacked_b() requires matching dtype and device: "
            f"a=({a.dtype}, {a.device}), b4=({b4.dtype}, {b4.device})"
        )
    if not is_gpu(a) or a.dtype not in _SUPPORTED_DTYPES:
        raise ValueError(
            f"matmul_prepacked_b() runs float32/bfloat16 operands on a ROCm device, got "
            f"{a.dtype} on {a.device}"
        )
    if bias is not None and (bias.dim() != 1 or int(bias.shape[0]) != n):
        raise ValueError(f"bias must have shape ({n},), got {tuple(bias.shape)}")


def matmul_prepacked_b(
    a: Tensor,
    b4: Tensor,
    n: int,
    bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    scale: Tensor | None = None,
    shift: Tensor | None = None,
) -> Tensor:
    """``epilogue((a @ B + bias) * scale + shift)`` with B packed by
    :func:`pack_b_vnni_t`, :func:`pack_b_blocked_t` / :func:`pack_b_blocked`,
    :func:`pack_b_blocked_vnni[_t] <pack_b_blocked_vnni>` or
    :func:`pack_b_panels`; ``n`` is B's width before padding
    (``matmul.py:1593-1671``). The kernel reads B in its packed layout: nothing
    is repacked per call."""
    _check_prepacked(a, b4, bias, n)
    layout, panel, kpad, _ = _packed_layout(a, b4, n)
    code = epilogue_code(epilogue)
    m, k = map(int, a.shape)
    c = output_pool.empty((m, n), dtype=a.dtype, device=a.device)
    if m == 0 or n == 0:
        return c
    bias_, scale_, shift_, vec_dtype = _vectors(bias, scale, shift, n, a)
    a_buf = a.contiguous()
    return _launch_gemm(
        a_buf, max(k, 1), False, b4.contiguous(), 0, layout, panel, kpad, c, m, n, k,
        bias=bias_, scale=scale_, shift=shift_, vec_dtype=vec_dtype, epilogue=code,
    )


def matmul_prepacked_b_affine(
    a: Tensor,
    b4: Tensor,
    n: int,
    bias: Tensor | None,
    post_scale: Tensor,
    post_bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
) -> Tensor:
    """Prepacked-RHS GEMM with a per-output affine post-op,
    ``epilogue((a @ B + bias) * post_scale + post_bias)`` (``matmul.py:1788-1839``)."""
    return matmul_prepacked_b(a, b4, n, bias, epilogue, post_scale, post_bias)


def prepacked_b_call(
    a: Tensor,
    b4: Tensor,
    n: int,
    bias: Tensor | None = None,
    epilogue: Callable[[Tensor], Tensor] = identity_epilogue,
    scale: Tensor | None = None,
    shift: Tensor | None = None,
    tile_m: int | None = None,
) -> Callable[[Tensor], Tensor]:
    """``lambda x: matmul_prepacked_b(x, b4, n, bias, epilogue, scale, shift)``
    with the host work done once for activations like ``a`` (same shape,
    dtype, device, contiguous): checks, vector conversion, the launch plan and
    workspace. Other activations take :func:`matmul_prepacked_b`
    (``matmul.py:1674-1785``). ``tile_m`` requests the workgroup's rows."""
    from helion_mlir_backend import prepared_call

    def general(x: Tensor) -> Tensor:
        return matmul_prepacked_b(x, b4, n, bias, epilogue, scale, shift)

    if a.dim() != 2 or not is_gpu(a, b4):
        return general
    _check_prepacked(a, b4, bias, n)
    layout, panel, kpad, _ = _packed_layout(a, b4, n)
    code = epilogue_code(epilogue)
    m, k = map(int, a.shape)
    if m == 0 or n == 0:
        return general
    bias_, scale_, shift_, vec_dtype = _vectors(bias, scale, shift, n, a)
    b_buf = b4.contiguous()
    tiles = (tile_m, 0, 0) if tile_m else None
    launch = GemmLaunch(
        native.dtype_code(a.dtype), a.dtype, a.device, (m, n), k, False, 0, layout, panel, kpad,
        m, n, k, bias=bias_, scale=scale_, shift=shift_, vec_dtype=vec_dtype, epilogue=code,
        tiles=tiles,
    )
    prepared = prepared_call(launch, (a, b_buf), [0], general)
    return general if prepared is None else prepared
