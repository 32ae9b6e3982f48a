"""The native call path of the ``gpu`` target: ``libhmx.so``, a C-ABI library of
hand-written gfx950 HIP kernels, bound with ctypes.

Stands in for the reference's native call path
(``helion_mlir_backend/_compiler/native/__init__.py:107-236`` and ``call.cpp``):
there, a C++ CPython extension checks arguments and calls a JIT-compiled CPU
entry without the GIL. Here every hot-path kernel family has one typed C entry
point (``include/hmx.h``); this module loads the library, declares the
signatures, and turns a non-zero status into a Python exception. ctypes
releases the GIL around each call, as ``call.cpp:194-196`` does.

There is no fallback: if the library is missing or the device is not a
gfx950, calls raise. ``HMX_LIBRARY`` may name another build of the library.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
import threading

import torch

from ..support.errors import UnsupportedTargetError

LIBRARY_ENV = "HMX_LIBRARY"
ABI_VERSION = 5  # HMX_ABI_VERSION of include/hmx.h
NATIVE_CALL_ENV = "HELION_MLIR_NATIVE_CALL"
_DEFAULT = Path(__file__).resolve().parents[3] / "csrc" / "libhmx.so"

# Status codes, dtypes and enumerations of include/hmx.h.
OK, ERR_INVALID, ERR_HIP, ERR_UNSUPPORTED = 0, 1, 2, 3
DTYPE_F32, DTYPE_BF16 = 0, 1
EPI_IDENTITY, EPI_RELU, EPI_SILU, EPI_SIGMOID = 0, 1, 2, 3
EPI_GELU, EPI_GELU_TANH, EPI_TANH, EPI_LEAKY_RELU = 4, 5, 6, 7
EPI_PROGRAM = 8
PROGRAM_MAX, PROGRAM_REGS = 16, 8  # HMX_PROGRAM_MAX, HMX_PROGRAM_REGS
# Epilogue program opcodes (HMX_OP_*), in order.
OPCODES = (
    "copy", "neg", "abs", "relu", "sigmoid", "tanh", "silu", "gelu", "gelu_tanh", "exp", "log",
    "sqrt", "rsqrt", "recip", "erf", "sin", "cos", "log1p", "expm1", "floor", "ceil", "trunc",
    "round", "softplus", "mish", "hardswish", "hardsigmoid", "elu", "leaky_relu", "clamp",
    "add_c", "mul_c", "div_c", "rsub_c", "rdiv_c", "pow_c", "add", "sub", "mul", "div", "max",
    "min", "pow",
)
OP = {name: code for code, name in enumerate(OPCODES)}


class Instr(ctypes.Structure):
    """``hmx_instr``: ``dst = op(a[, b][, c0, c1])``."""

    _fields_ = [("op", ctypes.c_uint8), ("dst", ctypes.c_uint8), ("a", ctypes.c_uint8),
                ("b", ctypes.c_uint8), ("c0", ctypes.c_float), ("c1", ctypes.c_float)]


class Program(ctypes.Structure):
    """``hmx_program``: an epilogue of at most PROGRAM_MAX instructions."""

    _fields_ = [("count", ctypes.c_int32), ("result", ctypes.c_int32), ("code", Instr * PROGRAM_MAX)]


def program_arg(program: "Program | None") -> "int | None":
    """The address to pass for an ``hmx_program*`` argument (None: NULL)."""
    return None if program is None else ctypes.addressof(program)
B_ROW, B_TRANS, B_VNNI_PANELS, B_BLOCKED_VNNI, B_PANELS, B_BLOCKED = range(6)
GEMM_SCRATCH_BYTES = 64 << 20  # HMX_GEMM_SCRATCH_BYTES
EXTRA_NONE, EXTRA_ADD, EXTRA_MUL = 0, 1, 2
ELT_RELU, ELT_LEAKY_RELU, ELT_SCALE = 0, 1, 2
(
    PACK_PAD,
    PACK_A_BLOCKED,
    PACK_A_BLOCKED_T,
    PACK_B_BLOCKED,
    PACK_B_BLOCKED_T,
    PACK_B_BLOCKED_VNNI,
    PACK_B_BLOCKED_VNNI_T,
    PACK_B_VNNI_PANELS_T,
    PACK_B_PANELS,
    PACK_A_PANELS,
) = range(10)

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_IP = ctypes.POINTER(ctypes.c_int)
_LP = ctypes.POINTER(ctypes.c_int64)

# name -> argument types (restype is int unless listed in _RESTYPES).
SIGNATURES: dict[str, list[object]] = {
    "hmx_last_error": [],
    "hmx_abi_version": [],
    "hmx_device_check": [_IP],
    "hmx_time_launches": [_P, _P],
    "hmx_jit_info": [_LP, _LP, _LP],
    "hmx_jit_last_log": [],
    "hmx_gemm": [
        _I, _I,  # ab_dtype, c_dtype
        _P, _L, _I,  # a, lda, trans_a
        _P, _L, _I, _L, _L,  # b, ldb, b_layout, b_panel, b_kpad
        _P, _L,  # c, ldc
        _L, _L, _L,  # m, n, k
        _L, _L, _L, _L,  # batch, stride_a, stride_b, stride_c
        _P, _P, _P, _I,  # bias, scale, shift, vec_dtype
        _I, _F, _P,  # epilogue, epilogue_arg, program
        _I, _P, _L,  # splits, workspace, workspace_bytes
        _I, _I, _I,  # tile_m, tile_n, tile_k
        _P,  # stream
    ],
    "hmx_gemm_noalloc": [
        _I, _I,  # ab_dtype, c_dtype
        _P, _L, _I,  # a, lda, trans_a
        _P, _L, _I, _L, _L,  # b, ldb, b_layout, b_panel, b_kpad
        _P, _L,  # c, ldc
        _L, _L, _L,  # m, n, k
        _L, _L, _L, _L,  # batch, stride_a, stride_b, stride_c
        _P, _P, _P, _I,  # bias, scale, shift, vec_dtype
        _I, _F, _P,  # epilogue, epilogue_arg, program
        _I,  # splits
        _I, _I, _I,  # tile_m, tile_n, tile_k
        _P,  # stream
    ],
    "hmx_gemm_plan": [
        _I, _L, _L, _L, _L, _I, _I, _I, _L, _I, _I, _I, _I, _I,
        _IP, _IP, _IP, _IP, _LP,
    ],
    "hmx_softmax_rows": [_I, _P, _P, _L, _L, _P],
    "hmx_rmsnorm_rows": [_I, _P, _P, _I, _P, _L, _L, _F, _P],
    "hmx_group_norm_rows": [_I, _P, _P, _P, _P, _I, _P, _L, _L, _L, _F, _I, _I, _F, _P, _P],
    "hmx_row_sum": [_I, _P, _P, _L, _L, _I, _F, _P, _P],
    "hmx_column_sum": [_I, _P, _P, _L, _L, _P, _L, _P],
    "hmx_column_sum_plan": [_L, _L, _P],
    "hmx_row_dot": [_I, _P, _P, _P, _L, _L, _I, _F, _P, _P],
    "hmx_matvec": [_I, _P, _P, _P, _L, _L, _P],
    "hmx_elementwise": [_I, _I, _P, _P, _L, _F, _P],
    "hmx_pack": [_I, _I, _P, _L, _L, _L, _P, _L, _L, _L, _P],
}
_RESTYPES = {"hmx_last_error": ctypes.c_char_p, "hmx_jit_last_log": ctypes.c_char_p}

_lock = threading.Lock()
_lib: list[ctypes.CDLL] = []
_device_units: dict[int, int] = {}  # compute units of each checked device
_calls = [0]


def library_path() -> Path:
    """Where the library is loaded from: ``HMX_LIBRARY`` or the in-tree build."""
    value = os.environ.get(LIBRARY_ENV, "").strip()
    return Path(value) if value else _DEFAULT


def lib() -> ctypes.CDLL:
    """The loaded library; raises ``RuntimeError`` if it is not built."""
    if _lib:
        return _lib[0]
    with _lock:
        if _lib:
            return _lib[0]
        path = library_path()
        if not path.is_file():
            raise RuntimeError(
                f"libhmx is not built ({path} is missing): build it with "
                "`make -C helion-mlir-xsmm_amd/csrc` or __graft_entry__.build()"
            )
        handle = ctypes.CDLL(str(path))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        if handle.hmx_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {handle.hmx_abi_version()}, expected {ABI_VERSION}")
        _lib.append(handle)
        return handle


def available() -> bool:
    """Whether the library is built (it may still refuse a non-gfx950 device)."""
    return library_path().is_file()


_load_error: list[str] = []


def module() -> ctypes.CDLL | None:
    """The loaded library, the counterpart of the reference's native extension
    module (``native/__init__.py:107-127``): ``None`` while native calls are
    off, or when it cannot be loaded (:func:`load_error` says why). The
    ``helion_mlir_utils`` entry points do not consult it: they always launch
    the library's kernels and raise when it is missing."""
    if not enabled():
        return None
    try:
        return lib()
    except (OSError, RuntimeError, AttributeError) as exc:
        if not _load_error:
            _load_error.append(str(exc))
        return None


def load_error() -> str | None:
    """Why :func:`module` found no library, if loading it failed."""
    return _load_error[0] if _load_error else None


def last_error() -> str:
    return lib().hmx_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    """Raise for a non-zero status: ``ValueError`` for arguments the kernels
    refused, ``UnsupportedTargetError`` for a non-gfx950 device, else
    ``RuntimeError``."""
    if status == OK:
        return
    message = f"{what}: {last_error()}"
    if status == ERR_INVALID:
        raise ValueError(message)
    if status == ERR_UNSUPPORTED:
        raise UnsupportedTargetError(what, reason=message)
    raise RuntimeError(message)


def call(name: str, *args: object) -> None:
    """``name(*args)`` of the library, its status checked."""
    fn = getattr(lib(), name)
    _calls[0] += 1
    check(fn(*args), name)


def time_launches(start: "torch.cuda.Event | None", stop: "torch.cuda.Event | None") -> None:
    """Arms timing events for the kernels this thread enqueues next
    (``hmx_time_launches``): ``start`` is recorded as the first kernel begins,
    ``stop`` as each kernel ends. ``None, None`` disarms. The events must have
    been created (recorded once) with ``enable_timing=True``."""
    handles = [None if e is None else e.cuda_event for e in (start, stop)]
    if any(h == 0 for h in handles):
        raise ValueError("time_launches: record each event once before arming it")
    check(lib().hmx_time_launches(*handles), "hmx_time_launches")


def jit_info() -> dict[str, object]:
    """Run-time compiled GEMM epilogues so far (``hmx_jit_info``): kernels
    compiled, compilations that failed (their GEMMs ran the interpreter),
    launches of compiled kernels, and the last failure's compiler log."""
    vals = [ctypes.c_int64() for _ in range(3)]
    check(lib().hmx_jit_info(*[ctypes.byref(v) for v in vals]), "hmx_jit_info")
    log = lib().hmx_jit_last_log() or b""
    return {"compiled": vals[0].value, "failed": vals[1].value, "launches": vals[2].value,
            "last_failure_log": log.decode(errors="replace")}


def count_call() -> None:
    """Count a library call made through a bound function."""
    _calls[0] += 1


def native_calls() -> int:
    """Kernel-library calls made by this process."""
    return _calls[0]


def ensure_device(device: torch.device) -> None:
    """Check once per device that it is a gfx950 the library was built for."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index in _device_units:
        return
    with torch.cuda.device(index):
        units = ctypes.c_int(0)
        check(lib().hmx_device_check(ctypes.byref(units)), "hmx_device_check")
    _device_units[index] = int(units.value)


def device_units(device: torch.device | None) -> int:
    """Compute units of ``device`` (checked as ``ensure_device`` does); 0 --
    the library's default, MI355X's 256 -- for ``None`` or a non-ROCm device,
    where plans are made without a GPU."""
    if device is None or device.type != "cuda":
        return 0
    if device.index is not None:
        units = _device_units.get(device.index)
        if units is not None:
            return units
    if not torch.cuda.is_available():
        return 0
    ensure_device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _device_units[index]


# torch's raw current-stream query skips building a Stream object (~0.1 us
# instead of ~2 us per call); the public API is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The current torch HIP stream of ``device``, as a ``hipStream_t`` value."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _raw_stream is not None:
        return int(_raw_stream(index))
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"the gpu target computes in float32 or bfloat16, got {dtype}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# The native call switch (HELION_MLIR_NATIVE_CALL, set_native_call), as in the
# reference (native/__init__.py:73-95): it governs the prepared-call paths.
_enabled = os.environ.get(NATIVE_CALL_ENV, "").strip().lower() not in ("0", "false", "no", "off")


def enabled() -> bool:
    """Whether prepared calls launch natively (:func:`set_native_call`)."""
    return _enabled


def set_native_call(enabled: bool) -> None:
    """Turn the native call paths on or off for the whole process
    (``helion_mlir_backend.set_native_call``; ``HELION_MLIR_NATIVE_CALL``
    gives the initial state, read once at import). Off takes effect at once
    for every prepared call (each checks it per call): it takes its fallback,
    the general entry point; and ``prepared_call`` made while off returns
    ``None``, as the reference's kernels compiled while off have no native
    run. The ``helion_mlir_utils`` entry points themselves launch their
    ``libhmx`` kernels either way: on this target there is no other path to
    take."""
    global _enabled
    _enabled = bool(enabled)


def refresh_allocator() -> None:
    """No-op: device outputs come from torch's caching allocator."""
