"""hmx_gemm_noalloc: the GEMM entry point that allocates nothing (its split-K
partials and transposed A and B live in the library's static per-device
scratch),
checked through the C ABI against hmx_gemm, the entry point it mirrors, on
two calls in a row -- the second smaller, so it reads a scratch that still
holds the first call's data -- and against the CPU oracle.

The entry point has no counterpart in the reference; the GEMMs it runs are
``matmul`` / ``bmm`` (helion_mlir_utils/matmul.py:1446-1570, 1965-2006).
Equality with hmx_gemm is bit for bit: with a plan that fits the scratch
both entry points launch the same kernels with the same splits.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helion_mlir_backend._compiler import native
from oracle import restate as R
from tests.helpers import max_rel_error, tensor, to_np

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(31)


def _plan(a: torch.Tensor, m: int, n: int, k: int, batch: int,
          act: int = native.EPI_IDENTITY) -> tuple[int, int, int, int, int]:
    out = [ctypes.c_int() for _ in range(4)]
    ws = ctypes.c_int64()
    native.check(native.lib().hmx_gemm_plan(native.dtype_code(a.dtype), m, n, k, batch, 0, native.B_ROW, 0, -1,
                                            0, 0, 0, native.device_units(a.device), act,
                                            *[ctypes.byref(o) for o in out], ctypes.byref(ws)), "hmx_gemm_plan")
    return (*[o.value for o in out], ws.value)


def _gemm(a: torch.Tensor, b: torch.Tensor, noalloc: bool, bias: torch.Tensor | None = None,
          act: int = native.EPI_IDENTITY, splits: int = 0,
          program: "native.Program | None" = None) -> tuple[int, torch.Tensor]:
    """C[i] = act(A[i] @ B[i] + bias) of A [batch, M, K], B [batch, K, N]
    (row-major), through one of the two entry points; (status, C)."""
    batch, m, k = a.shape
    n = b.shape[2]
    c = torch.full((batch, m, n), float("nan"), dtype=a.dtype, device=a.device)
    stream = torch.cuda.current_stream(a.device).cuda_stream
    head = (native.dtype_code(a.dtype), native.dtype_code(c.dtype), a.data_ptr(), k, 0,
            b.data_ptr(), n, native.B_ROW, 0, 0, c.data_ptr(), n, m, n, k, batch, m * k, k * n, m * n,
            native.ptr(bias), None, None, native.dtype_code(a.dtype) if bias is not None else native.DTYPE_F32,
            act, 0.0, native.program_arg(program), splits)
    if noalloc:
        status = native.lib().hmx_gemm_noalloc(*head, 0, 0, 0, stream)
    else:
        ws_bytes = _plan(a, m, n, k, batch, act)[4] if splits == 0 else 0
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=a.device)
        status = native.lib().hmx_gemm(*head, ws.data_ptr(), ws_bytes, 0, 0, 0, stream)
    torch.cuda.synchronize()
    return status, c


def _operands(batch: int, m: int, n: int, k: int, dtype: str, device) -> tuple[torch.Tensor, torch.Tensor]:
    a = tensor(RNG.uniform(-1, 1, (batch, m, k)).astype(np.float32), dtype, device)
    b = tensor(RNG.uniform(-1, 1, (batch, k, n)).astype(np.float32), dtype, device)
    return a, b


def _check_pair(a: torch.Tensor, b: torch.Tensor, dtype: str, bias: torch.Tensor | None = None,
                act: int = native.EPI_IDENTITY) -> None:
    batch, m, k = a.shape
    n = b.shape[2]
    splits, *_, ws = _plan(a, m, n, k, batch)
    assert ws <= native.GEMM_SCRATCH_BYTES, "the plan must fit the scratch for the comparison to hold"
    st, got = _gemm(a, b, True, bias, act)
    assert st == native.OK, native.last_error()
    st, ref = _gemm(a, b, False, bias, act)
    assert st == native.OK, native.last_error()
    assert torch.equal(got, ref), f"noalloc differs from hmx_gemm ({splits} splits, {ws} workspace bytes)"
    # and the oracle, on a few slices
    for i in sorted({0, batch - 1}):
        exact = R.matmul(to_np(a[i]), to_np(b[i]), bias=None if bias is None else to_np(bias),
                         act="relu" if act == native.EPI_RELU else "identity", out=dtype)
        assert max_rel_error(to_np(got[i]), exact) < (1e-5 if dtype == "f32" else 1e-2)


def test_noalloc_split_k_twice_second_smaller(gpu_device) -> None:
    # f32 split-K bmm: partials in the scratch; then a smaller product whose
    # partials overwrite the start of the same scratch.
    a, b = _operands(4, 64, 96, 8192, "f32", gpu_device)
    assert _plan(a, 64, 96, 8192, 4)[0] > 1
    _check_pair(a, b, "f32")
    a2, b2 = _operands(2, 32, 64, 4096, "f32", gpu_device)
    assert _plan(a2, 32, 64, 4096, 2)[0] > 1
    _check_pair(a2, b2, "f32")


def test_noalloc_bf16_transposed_b_and_epilogue_twice(gpu_device) -> None:
    # bf16 with a row-major B the kernel reads transposed: B^T goes to the
    # scratch first (ragged K, 512+ rows); bias and ReLU fused. Then a smaller
    # one over the same scratch.
    a, b = _operands(1, 600, 333, 4100, "bf16", gpu_device)
    bias = tensor(RNG.normal(0, 1, 333).astype(np.float32), "bf16", gpu_device)
    assert _plan(a, 600, 333, 4100, 1)[4] > 0
    _check_pair(a, b, "bf16", bias, native.EPI_RELU)
    a2, b2 = _operands(1, 520, 100, 1030, "bf16", gpu_device)
    assert _plan(a2, 520, 100, 1030, 1)[4] > 0
    _check_pair(a2, b2, "bf16", bias[:100].contiguous(), native.EPI_RELU)


def test_noalloc_bf16_transposed_a_twice(gpu_device) -> None:
    # bf16 A stored [K, M] is transposed into the scratch first (after B^T
    # where B is read transposed too: ragged K); then a smaller product whose
    # A^T overwrites the start of the same scratch.
    stream = torch.cuda.current_stream(gpu_device).cuda_stream
    lib = native.lib()
    for m, n, k in [(1000, 1500, 777), (600, 520, 640)]:
        at = tensor(RNG.uniform(-1, 1, (k, m)).astype(np.float32), "bf16", gpu_device)
        b = tensor(RNG.uniform(-1, 1, (k, n)).astype(np.float32), "bf16", gpu_device)
        out = [ctypes.c_int() for _ in range(4)]
        ws = ctypes.c_int64()
        native.check(lib.hmx_gemm_plan(native.DTYPE_BF16, m, n, k, 1, 1, native.B_ROW, 0, -1, 0, 0, 0,
                                       native.device_units(gpu_device), native.EPI_IDENTITY,
                                       *[ctypes.byref(o) for o in out], ctypes.byref(ws)), "hmx_gemm_plan")
        assert m * k * 2 <= ws.value <= native.GEMM_SCRATCH_BYTES
        cs = []
        for noalloc in (True, False):
            c = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu_device)
            head = (native.DTYPE_BF16, native.DTYPE_BF16, at.data_ptr(), m, 1, b.data_ptr(), n, native.B_ROW, 0, 0,
                    c.data_ptr(), n, m, n, k, 1, 0, 0, 0, None, None, None, native.DTYPE_F32,
                    native.EPI_IDENTITY, 0.0, None, 0)
            if noalloc:
                st = lib.hmx_gemm_noalloc(*head, 0, 0, 0, stream)
            else:
                w = torch.empty(ws.value, dtype=torch.uint8, device=gpu_device)
                st = lib.hmx_gemm(*head, w.data_ptr(), ws.value, 0, 0, 0, stream)
            torch.cuda.synchronize()
            assert st == native.OK, native.last_error()
            cs.append(c)
        assert torch.equal(cs[0], cs[1])
        exact = R.matmul(to_np(at), to_np(b), True, False, out="bf16")
        assert max_rel_error(to_np(cs[0]), exact) < 1e-2


def test_noalloc_config5_fills_the_scratch(gpu_device) -> None:
    # Config 5's f32 bmm: 16 splits of [16, 256, 256] f32 partials, exactly
    # the scratch's 64 MiB; then a smaller bf16-in bmm.
    a, b = _operands(16, 256, 256, 65536, "f32", gpu_device)
    splits, *_, ws = _plan(a, 256, 256, 65536, 16)
    assert (splits, ws) == (16, native.GEMM_SCRATCH_BYTES)
    _check_pair(a, b, "f32")
    del a, b
    a2, b2 = _operands(8, 256, 256, 16384, "bf16", gpu_device)
    assert _plan(a2, 256, 256, 16384, 8)[0] > 1
    _check_pair(a2, b2, "bf16")


def test_noalloc_refuses_splits_beyond_the_scratch(gpu_device) -> None:
    # 64 splits of [16, 256, 256] f32 partials: 256 MiB > 64 MiB. Refused
    # before anything is enqueued; the output is untouched.
    a, b = _operands(16, 256, 256, 8192, "f32", gpu_device)
    st, c = _gemm(a, b, True, splits=64)
    assert st == native.ERR_INVALID
    assert "scratch" in native.last_error()
    assert torch.isnan(c).all()
    # splits = 0 plans within the scratch and runs.
    st, _ = _gemm(a, b, True)
    assert st == native.OK, native.last_error()


def test_noalloc_program_epilogue_past_the_scratch_size(gpu_device) -> None:
    # An epilogue program that the direct-to-LDS kernel runs fused needs no
    # workspace: a bf16 [8192, 4096] x [4096, 4096] product (its f32 partials
    # would be 128 MiB, twice the scratch) runs through hmx_gemm_noalloc, twice,
    # and equals hmx_gemm; the second call is smaller.
    prog = native.Program()
    prog.count = 2
    prog.code[0] = native.Instr(native.OP["silu"], 1, 0, 0, 0.0, 0.0)
    prog.code[1] = native.Instr(native.OP["mul_c"], 2, 1, 0, 2.0, 0.0)
    prog.result = 2
    for m, n, k in ((8192, 4096, 4096), (4096, 2048, 1024)):
        a, b = _operands(1, m, n, k, "bf16", gpu_device)
        assert _plan(a, m, n, k, 1, native.EPI_PROGRAM)[4] == 0
        st, got = _gemm(a, b, True, act=native.EPI_PROGRAM, program=prog)
        assert st == native.OK, native.last_error()
        st, ref = _gemm(a, b, False, act=native.EPI_PROGRAM, program=prog)
        assert st == native.OK, native.last_error()
        assert torch.equal(got, ref)
        rows = np.arange(0, m, 997)
        exact = R.matmul(to_np(a[0][rows]), to_np(b[0]), act="silu", out="f32") * 2.0
        assert max_rel_error(to_np(got[0][rows]), exact) < 1e-2
        del a, b, got, ref


def test_noalloc_compiles_no_kernel(gpu_device) -> None:
    # hmx_gemm_noalloc calls nothing that allocates, and compiling or loading
    # a kernel at run time would: with an epilogue whose kernel no earlier
    # call compiled it runs the prebuilt kernel (nothing compiled, no compiled
    # launch), bit-equal to hmx_gemm, which compiles it; once compiled, the
    # allocation-free entry point launches it too. Whole 256 x 256 tiles, so
    # both run the 16x16x32 kernel (a program no other test uses).
    prog = native.Program()
    prog.count = 3
    prog.code[0] = native.Instr(native.OP["silu"], 1, 0, 0, 0.0, 0.0)
    prog.code[1] = native.Instr(native.OP["mul_c"], 2, 1, 0, 1.375, 0.0)
    prog.code[2] = native.Instr(native.OP["add_c"], 3, 2, 0, 0.125, 0.0)
    prog.result = 3
    a, b = _operands(1, 4096, 4096, 256, "bf16", gpu_device)
    before = native.jit_info()
    st, got = _gemm(a, b, True, act=native.EPI_PROGRAM, program=prog)
    assert st == native.OK, native.last_error()
    after = native.jit_info()
    assert (after["compiled"], after["launches"]) == (before["compiled"], before["launches"])
    st, ref = _gemm(a, b, False, act=native.EPI_PROGRAM, program=prog)
    assert st == native.OK, native.last_error()
    assert torch.equal(got, ref)
    compiled = native.jit_info()
    if compiled["compiled"] > after["compiled"]:  # run-time compilation is on
        st, again = _gemm(a, b, True, act=native.EPI_PROGRAM, program=prog)
        assert st == native.OK and torch.equal(again, ref)
        last = native.jit_info()
        assert last["compiled"] == compiled["compiled"] and last["launches"] == compiled["launches"] + 1
    rows = np.arange(0, 4096, 997)
    exact = R.matmul(to_np(a[0][rows]), to_np(b[0]), act="silu", out="f32") * 1.375 + 0.125
    assert max_rel_error(to_np(got[0][rows]), exact) < 1e-2
