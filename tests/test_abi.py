"""The C ABI of libhmx without a GPU: the library loads, exports every entry
point ``include/hmx.h`` declares with the signatures the Python binding uses,
refuses bad arguments before touching a device, and plans launches on the host."""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
import re
import subprocess

import pytest

from helion_mlir_backend._compiler import native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hmx.h"


# The refusal tests pass fake device pointers: they must never reach a launch,
# so they run only where no GPU is visible (the CPU suite).
no_device = pytest.mark.skipif(
    __import__("torch").cuda.is_available(), reason="fake pointers: CPU-only refusal test"
)


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not native.available():
        subprocess.run(["make", "-C", str(ROOT / "helion-mlir-xsmm_amd" / "csrc"), "-j8"], check=True,
                       capture_output=True)
    return native.lib()


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^(?:int|const char\*|int64_t|void)\s+\*?(hmx_\w+)\(", text, re.M)


def test_header_declares_the_entry_points() -> None:
    names = declared_functions()
    for name in ("hmx_gemm", "hmx_gemm_plan", "hmx_softmax_rows", "hmx_rmsnorm_rows",
                 "hmx_group_norm_rows", "hmx_row_sum", "hmx_column_sum", "hmx_row_dot",
                 "hmx_matvec", "hmx_elementwise", "hmx_pack", "hmx_last_error",
                 "hmx_abi_version", "hmx_device_check"):
        assert name in names


def test_library_exports_every_declared_symbol(lib: ctypes.CDLL) -> None:
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing
    out = subprocess.run(["nm", "-D", "--defined-only", str(native.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (hmx_\w+)$", out, re.M))
    assert set(declared_functions()) <= exported


def test_binding_covers_the_header() -> None:
    assert set(declared_functions()) == set(native.SIGNATURES)


def test_abi_version(lib: ctypes.CDLL) -> None:
    assert lib.hmx_abi_version() == native.ABI_VERSION == 5


@pytest.mark.parametrize(
    ("name", "args", "message"),
    [
        ("hmx_softmax_rows", (7, 16, 16, 4, 4, None), "unknown dtype"),
        ("hmx_softmax_rows", (0, 16, 16, 4, 0, None), "invalid shape"),
        ("hmx_softmax_rows", (0, None, 16, 4, 4, None), "null operand"),
        ("hmx_rmsnorm_rows", (1, 16, None, 0, 16, -1, 4, 1e-6, None), "invalid shape"),
        ("hmx_group_norm_rows", (0, 16, 16, 16, None, 0, 16, 2, 3, 4, 1e-5, 1, 0, 0.0, None, None),
         "extra op without an extra operand"),
        ("hmx_group_norm_rows", (0, 16, 16, 16, 16, 0, 16, 2, 3, 4, 1e-5, 0, 99, 0.0, None, None),
         "unknown epilogue"),
        ("hmx_group_norm_rows", (0, 16, 16, 16, 16, 0, 16, 2, 3, 4, 1e-5, 0, 8, 0.0, None, None),
         "epilogue program is null"),
        ("hmx_row_sum", (0, 16, 16, 2, 2, 42, 0.0, None, None), "unknown epilogue"),
        ("hmx_elementwise", (9, 0, 16, 16, 4, 0.0, None), "unknown op"),
        ("hmx_pack", (42, 0, 16, 4, 4, 4, 16, 32, 32, 0, None), "unknown kind"),
        ("hmx_pack", (1, 0, 16, 4, 4, 4, 16, 40, 32, 0, None), "multiples of 32"),
        ("hmx_pack", (7, 1, 16, 4, 4, 4, 16, 32, 30, 32, None), "VNNI panels"),
    ],
)
@no_device
def test_invalid_arguments_are_refused(lib: ctypes.CDLL, name: str, args: tuple, message: str) -> None:
    fn = getattr(lib, name)
    assert fn(*args) == native.ERR_INVALID
    assert message in native.last_error()


def _gemm(lib: ctypes.CDLL, **kw: object) -> int:
    args = dict(ab=1, c=1, a=16, lda=64, trans_a=0, b=16, ldb=64, layout=0, panel=0, kpad=0,
                cp=16, ldc=64, m=64, n=64, k=64, batch=1, sa=0, sb=0, sc=0, bias=None,
                scale=None, shift=None, vd=0, epi=0, arg=0.0, prog=None, splits=1, ws=None, wsb=0,
                tm=0, tn=0, tk=0, stream=None)
    args.update(kw)
    prog = args["prog"]
    if isinstance(prog, str):
        p = native.Program()
        p.count = 0 if prog == "empty" else 1
        p.code[0] = native.Instr(99 if prog == "bad_op" else native.OP["relu"], 9 if prog == "bad_reg" else 2, 0, 0,
                                 0.0, 0.0)
        p.result = 2
        args["prog"] = native.program_arg(p)
        return lib.hmx_gemm(*args.values())
    return lib.hmx_gemm(*args.values())


@pytest.mark.parametrize(
    ("kw", "message"),
    [
        ({"ab": 5}, "unknown dtype"),
        ({"layout": 9}, "unknown B layout"),
        ({"ab": 0, "layout": native.B_VNNI_PANELS, "panel": 64, "kpad": 64}, "VNNI layouts"),
        ({"epi": 77}, "unknown epilogue"),
        ({"epi": native.EPI_PROGRAM}, "epilogue program is null"),
        ({"epi": native.EPI_PROGRAM, "prog": "empty"}, "0 instructions"),
        ({"epi": native.EPI_PROGRAM, "prog": "bad_op"}, "unknown opcode"),
        ({"epi": native.EPI_PROGRAM, "prog": "bad_reg"}, "register past"),
        # An unaligned A takes the register-staged kernel, which leaves the
        # program to the split-K reduction and needs the partials.
        ({"epi": native.EPI_PROGRAM, "prog": "ok", "a": 18}, "an epilogue program on these operands needs"),
        ({"lda": 8}, "lda"),
        ({"ldb": 8}, "ldb"),
        ({"ldc": 8}, "ldc"),
        ({"batch": 0}, "invalid shape"),
        ({"a": None}, "null operand"),
        ({"splits": 4, "k": 4096, "lda": 4096}, "split-K needs"),
        ({"layout": native.B_BLOCKED, "kpad": 80}, "multiple of 32"),
        ({"layout": native.B_VNNI_PANELS, "panel": 64, "kpad": 32}, "does not cover"),
        ({"trans_a": 1, "layout": native.B_BLOCKED, "kpad": 64}, "row-major A"),
    ],
)
@no_device
def test_gemm_refuses_bad_arguments(lib: ctypes.CDLL, kw: dict, message: str) -> None:
    assert _gemm(lib, **kw) == native.ERR_INVALID
    assert message in native.last_error()


def _plan(lib: ctypes.CDLL, ab: int, m: int, n: int, k: int, batch: int = 1, splits: int = 0,
          max_ws: int = -1, tiles: tuple[int, int, int] = (0, 0, 0),
          b_layout: int = native.B_ROW, cus: int = 256, trans_a: int = 0,
          epi: int = native.EPI_IDENTITY) -> tuple[int, int, int, int, int]:
    outs = [ctypes.c_int() for _ in range(4)]
    ws = ctypes.c_int64()
    assert lib.hmx_gemm_plan(ab, m, n, k, batch, trans_a, b_layout, splits, max_ws, *tiles, cus, epi,
                             *[ctypes.byref(o) for o in outs], ctypes.byref(ws)) == 0
    return (*[o.value for o in outs], ws.value)


def test_plans_of_the_baseline_configs(lib: ctypes.CDLL) -> None:
    bf16, f32 = native.DTYPE_BF16, native.DTYPE_F32
    # 4096^3 bf16: 256 tiles of 256 x 256 fill the 256 CUs, no split; whole
    # tiles read the row-major B in place, so no workspace.
    assert _plan(lib, bf16, 4096, 4096, 4096) == (1, 256, 256, 64, 0)
    # Ragged M or N with K in whole 32-element stages: the direct-to-LDS kernel
    # reads row-major B in place (no transpose); other ragged shapes with
    # enough rows transpose B once into the workspace.
    assert _plan(lib, bf16, 4000, 4096, 4096) == (1, 256, 256, 64, 0)
    assert _plan(lib, bf16, 4000, 4096, 4100) == (1, 256, 256, 64, 4096 * 4100 * 2)
    assert _plan(lib, bf16, 4000, 4096, 4100, max_ws=0) == (1, 256, 256, 64, 0)
    # Few output rows do not amortize the transpose.
    assert _plan(lib, bf16, 256, 4000, 4100)[4] == 0
    # Few 128 x 128 tiles with K in whole stages split K until the grid holds
    # one workgroup per CU (the workspace holds the f32 partials only).
    assert _plan(lib, bf16, 256, 4000, 4096) == (4, 128, 128, 64, 4 * 256 * 4000 * 4)
    assert _plan(lib, bf16, 1024, 1024, 4096) == (4, 128, 128, 64, 4 * 1024 * 1024 * 4)
    assert _plan(lib, bf16, 1024, 2048, 4096)[:4] == (2, 128, 128, 64)
    # Not past one workgroup per CU, not below 16 stages per chunk, not for
    # small products.
    assert _plan(lib, bf16, 256, 11008, 4096)[0] == 1
    assert _plan(lib, bf16, 384, 384, 2048)[0] == 1
    assert _plan(lib, bf16, 2048, 1024, 2048)[0] == 1
    # Fused linear, 8192 x 11008 x 4096 (B row-major here): 1376 tiles, no split.
    assert _plan(lib, bf16, 8192, 11008, 4096)[:4] == (1, 256, 256, 64)
    # Split-K bmm [16, 256, 65536] @ [16, 65536, 256]: one 256 x 256 tile per
    # slice (each operand read once) x 16 splits = one workgroup per CU; the
    # f32 tile is 32 deep so each A row is read in whole 128-byte lines.
    s, tm, tn, tk, ws = _plan(lib, f32, 256, 256, 65536, batch=16)
    assert (s, tm, tn, tk) == (16, 256, 256, 32) and ws == 16 * 16 * 256 * 256 * 4
    assert _plan(lib, bf16, 256, 256, 65536, batch=16)[:4] == (16, 256, 256, 64)
    # Too few K tiles to fill the GPU by splitting: the small tile.
    assert _plan(lib, f32, 256, 256, 4096, batch=16)[1:3] == (128, 128)
    # A skinny bf16 product against B [N, K] (a decode-shaped linear): the
    # skinny kernel, one workgroup per 32 columns of C, no split or workspace.
    trans = native.B_TRANS
    assert _plan(lib, bf16, 32, 11008, 4096, b_layout=trans) == (1, 32, 32, 64, 0)
    assert _plan(lib, bf16, 1, 4096, 64, b_layout=trans) == (1, 32, 32, 64, 0)
    # One split (what a prepared call passes back) is no split: still skinny.
    assert _plan(lib, bf16, 32, 11008, 4096, splits=1, b_layout=trans) == (1, 32, 32, 64, 0)
    assert _plan(lib, bf16, 64, 11008, 4096, b_layout=trans) == (1, 32, 32, 64, 0)
    # Not skinny: 65 rows, K not in whole 64-element stages, batches, or a
    # caller's splits or tile.
    assert _plan(lib, bf16, 65, 11008, 4096, b_layout=trans)[1] == 128
    assert _plan(lib, bf16, 32, 11008, 4000, b_layout=trans)[1] == 128
    assert _plan(lib, bf16, 32, 11008, 4096, batch=2, b_layout=trans)[1] == 128
    assert _plan(lib, bf16, 32, 11008, 4096, splits=2, b_layout=trans)[:2] == (2, 128)
    assert _plan(lib, bf16, 32, 11008, 4096, tiles=(128, 128, 64), b_layout=trans)[1] == 128
    assert _plan(lib, f32, 32, 11008, 4096, b_layout=trans)[1] != 32
    # The same product with row-major B: 86 tiles of 128 x 128, split four
    # ways (one workgroup per CU at most), f32 partials in the workspace.
    assert _plan(lib, bf16, 32, 11008, 4096) == (4, 128, 128, 64, 4 * 32 * 11008 * 4)
    # The f32 512^3 plumbing case: 16 tiles of 128 x 128 and too few K tiles to
    # split them, so 64 x 64 tiles (64 workgroups), split four ways (one
    # workgroup per CU, four K tiles each).
    assert _plan(lib, f32, 512, 512, 512)[:3] == (4, 64, 64)
    # Small f32 products split at most 16 ways, each chunk at least 4 K tiles.
    assert _plan(lib, f32, 128, 128, 8192)[:3] == (16, 64, 64)
    assert _plan(lib, f32, 512, 512, 128)[:3] == (1, 64, 64)
    assert _plan(lib, f32, 256, 256, 1024)[:3] == (8, 64, 64)
    # Long K on one tile keeps the traffic rule's larger split.
    assert _plan(lib, f32, 64, 64, 65536)[:3] == (256, 128, 128)
    # Split-K fills the CUs with 128 x 128 tiles: they stay.
    assert _plan(lib, f32, 256, 256, 4096, batch=16)[:3] == (4, 128, 128)
    # A request below every f32 tile gets the smallest.
    assert _plan(lib, f32, 512, 512, 512, tiles=(32, 32, 32))[1:4] == (64, 64, 32)


def test_column_sum_plan_and_workspace_check(lib: ctypes.CDLL) -> None:
    def plan(m: int, n: int) -> int:
        ws = ctypes.c_int64(-1)
        assert lib.hmx_column_sum_plan(m, n, ctypes.byref(ws)) == 0
        return ws.value

    # 8 blocks of 512 columns x 128 chunks of 256 rows: [128, 4096] f32 partials.
    assert plan(32768, 4096) == 128 * 4096 * 4
    # Enough column blocks (or too few rows) for one pass: no workspace.
    assert plan(16, 100000) == 0
    assert plan(0, 10) == 0
    # 300 rows, one column block: two chunks of 150 rows.
    assert plan(300, 8) == 2 * 8 * 4
    # A workspace below the plan is refused before anything is enqueued.
    x = ctypes.c_void_p(256)
    y = ctypes.c_void_p(512)
    st = lib.hmx_column_sum(native.DTYPE_F32, x, y, 32768, 4096, ctypes.c_void_p(1024), 4096, None)
    assert st == native.ERR_INVALID and "workspace" in native.last_error()



def test_f32_big_tile_unsplit_plans(lib: ctypes.CDLL) -> None:
    f32 = native.DTYPE_F32
    # Whole 256 x 256 f32 tiles that fill the CUs unsplit, with an epilogue
    # the direct-to-LDS kernel finishes in registers: the big tile, one pass.
    for epi in (native.EPI_IDENTITY, native.EPI_RELU, native.EPI_SILU):
        assert _plan(lib, f32, 4096, 4096, 4096, epi=epi) == (1, 256, 256, 32, 0)
        assert _plan(lib, f32, 8192, 4096, 1024, b_layout=native.B_TRANS, epi=epi) == (1, 256, 256, 32, 0)
    # Other epilogues, K below 8 tiles, fewer tiles than CUs, ragged shapes,
    # transposed A or a caller's tile keep the 128 x 128 tile.
    assert _plan(lib, f32, 4096, 4096, 4096, epi=native.EPI_GELU)[:3] == (1, 128, 128)
    assert _plan(lib, f32, 4096, 4096, 224)[1] == 128
    assert _plan(lib, f32, 4096, 4096, 4096, cus=304)[1] == 128
    assert _plan(lib, f32, 4000, 4096, 4096)[1] == 128
    assert _plan(lib, f32, 4096, 4096, 4096, trans_a=1)[1] == 128
    assert _plan(lib, f32, 4096, 4096, 4096, tiles=(128, 128, 32)) == (1, 128, 128, 32, 0)
    # A plan passed back reproduces itself.
    assert _plan(lib, f32, 4096, 4096, 4096, splits=1, tiles=(256, 256, 32)) == (1, 256, 256, 32, 0)

def test_plan_honours_requests_and_limits(lib: ctypes.CDLL) -> None:
    bf16 = native.DTYPE_BF16
    assert _plan(lib, bf16, 4096, 4096, 4096, tiles=(128, 128, 64))[1:4] == (128, 128, 64)
    # A request below every tile gets the smallest.
    assert _plan(lib, bf16, 4096, 4096, 4096, tiles=(64, 64, 64))[1:3] == (128, 128)
    # Explicit splits, rounded to whole K tiles and no empty chunk.
    s, *_, ws = _plan(lib, bf16, 256, 256, 1000, splits=3)
    assert s == 3 and ws == 3 * 256 * 256 * 4
    assert _plan(lib, bf16, 256, 256, 100, splits=8)[0] == 2  # 2 K tiles: 2 chunks
    # The workspace limit stops the split.
    assert _plan(lib, native.DTYPE_F32, 256, 256, 65536, batch=16, max_ws=0)[0] == 1


# Shapes across every planner branch: whole and ragged tiles, skinny and
# split-K products, long K, batches, transposed A and packed layouts.
_PLAN_SHAPES = [
    (m, n, k, batch)
    for m, n, k, batch in [
        (4096, 4096, 4096, 1), (4000, 4096, 4100, 1), (8192, 11008, 4096, 1), (256, 256, 65536, 16),
        (256, 256, 4096, 16), (512, 512, 512, 1), (128, 128, 8192, 1), (64, 64, 65536, 1),
        (32, 11008, 4096, 1), (64, 4128, 64, 16), (16, 64, 4128, 16), (64, 64, 4128, 16),
        (1000, 4096, 4096, 1), (384, 384, 2048, 1), (256, 256, 1024, 1), (100, 100, 130, 1),
        (1, 1, 1, 1), (37, 45, 19, 3), (600, 333, 129, 1), (2048, 2048, 2048, 1), (96, 96, 100000, 2),
    ]
]
_PLAN_LAYOUTS = [(native.B_ROW, 0), (native.B_TRANS, 0), (native.B_ROW, 1), (native.B_VNNI_PANELS, 0),
                 (native.B_BLOCKED, 0), (native.B_PANELS, 0)]


def test_program_epilogues_plan_their_partials(lib: ctypes.CDLL) -> None:
    bf16, f32 = native.DTYPE_BF16, native.DTYPE_F32
    prog = native.EPI_PROGRAM
    # The direct-to-LDS bf16 kernels run programs fused: no partials. Shapes
    # they do not take, packed B (whose panels the plan does not see) and f32
    # plan f32 partials of the whole output for the reduction that finishes
    # the program; split products plan them anyway.
    assert _plan(lib, bf16, 4096, 4096, 4096, epi=prog) == (1, 256, 256, 64, 0)
    assert _plan(lib, bf16, 8192, 11008, 4096, epi=prog, b_layout=native.B_TRANS)[4] == 0
    assert _plan(lib, bf16, 4000, 4096, 4096, epi=prog)[4] == 0  # ragged M, K in whole stages
    assert _plan(lib, bf16, 4000, 4096, 4100, epi=prog, max_ws=0)[4] == 4000 * 4096 * 4
    assert _plan(lib, bf16, 4096, 4096, 4096, epi=prog, b_layout=native.B_BLOCKED)[4] == 4096 * 4096 * 4
    assert _plan(lib, f32, 4096, 4096, 4096, epi=prog)[4] >= 4096 * 4096 * 4
    assert _plan(lib, f32, 512, 512, 512, epi=prog) == (4, 64, 64, 32, 4 * 512 * 512 * 4)
    # Decode-shaped products never take the skinny kernel with a program.
    assert _plan(lib, bf16, 32, 11008, 4096, b_layout=native.B_TRANS)[:4] == (1, 32, 32, 64)
    assert _plan(lib, bf16, 32, 11008, 4096, b_layout=native.B_TRANS, epi=prog)[1:3] != (32, 32)
    # Named activations plan as before.
    assert _plan(lib, bf16, 4096, 4096, 4096, epi=native.EPI_GELU) == (1, 256, 256, 64, 0)


@pytest.mark.parametrize("epi", [native.EPI_IDENTITY, native.EPI_PROGRAM])
@pytest.mark.parametrize("cus", [256, 304, 80, 32])
@pytest.mark.parametrize("ab", [native.DTYPE_BF16, native.DTYPE_F32])
def test_a_plan_passed_back_is_the_same_plan(lib: ctypes.CDLL, cus: int, ab: int, epi: int) -> None:
    # What a prepared launch does: plan with splits = 0 and no workspace
    # limit, then call hmx_gemm with the plan's splits, tile and workspace.
    # hmx_gemm plans again from those; the two plans must agree, or the kernel
    # that runs is not the one gemm_plan() reports.
    for m, n, k, batch in _PLAN_SHAPES:
        for layout, trans_a in _PLAN_LAYOUTS:
            if ab == native.DTYPE_F32 and layout == native.B_VNNI_PANELS:
                continue
            first = _plan(lib, ab, m, n, k, batch, b_layout=layout, cus=cus, trans_a=trans_a, epi=epi)
            s, tm, tn, tk, ws = first
            again = _plan(lib, ab, m, n, k, batch, splits=s, max_ws=ws, tiles=(tm, tn, tk), b_layout=layout,
                          cus=cus, trans_a=trans_a, epi=epi)
            assert again == first, ((m, n, k, batch, layout, trans_a, cus), first, again)


def test_plans_follow_the_device_cu_count(lib: ctypes.CDLL) -> None:
    bf16, f32 = native.DTYPE_BF16, native.DTYPE_F32
    # 256 CUs: the baseline plans (test_plans_of_the_baseline_configs).
    assert _plan(lib, f32, 256, 256, 65536, batch=16, cus=256)[:4] == (16, 256, 256, 32)
    # 80 CUs: 16 slices x 8 splits already give every CU a workgroup.
    assert _plan(lib, f32, 256, 256, 65536, batch=16, cus=80)[:4] == (8, 256, 256, 32)
    # 304 CUs: one split more than 256 CUs need would overshoot the grid; the
    # 16 x 16 grid underfills, so 32 splits.
    assert _plan(lib, f32, 256, 256, 65536, batch=16, cus=304)[:4] == (32, 256, 256, 32)
    # 4096^3 bf16: 256 whole tiles are enough for 32 or 256 CUs; 304 CUs
    # would leave 48 idle, so 128 x 128 tiles (1024 of them).
    assert _plan(lib, bf16, 4096, 4096, 4096, cus=32)[:3] == (1, 256, 256)
    assert _plan(lib, bf16, 4096, 4096, 4096, cus=256)[:3] == (1, 256, 256)
    assert _plan(lib, bf16, 4096, 4096, 4096, cus=304)[:3] == (1, 128, 128)
    # The f32 512^3 case: 64 tiles of 64 x 64 split until the grid holds one
    # workgroup per CU when they fill at most a quarter of the CUs; on 128
    # CUs they fill half, and the partials would cost more than a quarter of
    # the operand traffic, so no split.
    assert _plan(lib, f32, 512, 512, 512, cus=256)[:3] == (4, 64, 64)
    assert _plan(lib, f32, 512, 512, 512, cus=128)[:3] == (1, 64, 64)


@no_device
def test_noalloc_refuses_a_plan_beyond_its_scratch(lib: ctypes.CDLL) -> None:
    # 64 explicit splits of [16, 256, 256] f32 partials need 256 MiB; the
    # scratch holds 64 MiB: refused on the host, before any device call.
    args = (native.DTYPE_F32, native.DTYPE_F32, 256, 8192, 0, 512, 256, native.B_ROW, 0, 0, 1024, 256,
            256, 256, 8192, 16, 256 * 8192, 8192 * 256, 256 * 256, None, None, None, native.DTYPE_F32,
            native.EPI_IDENTITY, 0.0, None, 64, 0, 0, 0, None)
    assert lib.hmx_gemm_noalloc(*args) == native.ERR_INVALID
    assert "scratch" in native.last_error() and str(native.GEMM_SCRATCH_BYTES) in native.last_error()


@no_device
def test_error_message_is_per_thread(lib: ctypes.CDLL) -> None:
    import threading

    assert lib.hmx_softmax_rows(7, 16, 16, 4, 4, None) == native.ERR_INVALID
    seen = []
    t = threading.Thread(target=lambda: seen.append(native.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "unknown dtype" in native.last_error()


def test_gemm_plan_transposes_a_up_front(lib: ctypes.CDLL) -> None:
    # bf16 A stored [K, M] of 512 or more rows, columns and K is transposed
    # into the workspace (M K 2 bytes, 256-byte rounded), except for whole
    # 256 x 256 tiles that fill the CUs with N up to 4096, which the in-place
    # kernel reads; f32, programs, small shapes and too small a workspace
    # read it in place. The plan reproduces itself when passed back.
    if os.environ.get("HMX_GEMM_TRANSPOSE_A", "").startswith("0"):
        pytest.skip("HMX_GEMM_TRANSPOSE_A=0 turns the transpose off")
    bf16, f32 = native.DTYPE_BF16, native.DTYPE_F32
    at = lambda m, k: -(-m * k * 2 // 256) * 256  # noqa: E731
    cases = [((3000, 3000, 3000), True), ((1000, 4096, 4096), True), ((8192, 8192, 4096), True),
             ((2048, 2048, 2048), True), ((4096, 4096, 4096), False), ((511, 4096, 4096), False),
             ((4096, 4096, 500), False)]
    def as_transposed(ab, m, n, k, **kw):
        # The plan of row-major A (same splits and tile) plus A^T's bytes.
        plan = _plan(lib, ab, m, n, k, trans_a=1, **kw)
        plain = _plan(lib, ab, m, n, k, **kw)
        return plan[:4] == plain[:4] and plan[4] == plain[4] + at(m, k)

    for (m, n, k), transposed in cases:
        s, tm, tn, tk, ws = _plan(lib, bf16, m, n, k, trans_a=1)
        assert as_transposed(bf16, m, n, k) == transposed, ((m, n, k), ws)
        assert _plan(lib, bf16, m, n, k, splits=s, max_ws=ws, tiles=(tm, tn, tk), trans_a=1) == (s, tm, tn, tk, ws)
        if transposed:
            # no room for A^T: read in place
            assert _plan(lib, bf16, m, n, k, max_ws=at(m, k) - 256, trans_a=1)[4] < at(m, k)
    assert not as_transposed(f32, 3000, 3000, 3000)
    assert not as_transposed(bf16, 3000, 3000, 3000, epi=native.EPI_PROGRAM)
