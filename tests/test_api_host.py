"""Host-side behaviour of the plugin surface without a GPU: target resolution
(``HELION_MLIR_TARGET`` gains ``gpu``), operand gates and their errors, epilogue
fusion codes, the GEMM plan, the output pool and the bench's one-GPU guard."""

from __future__ import annotations

import functools
import subprocess
import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

import helion_mlir_backend as B
import helion_mlir_utils as U
from helion_mlir_backend._compiler import native
from helion_mlir_backend._compiler.support.errors import UnsupportedTargetError
from helion_mlir_utils._gpu import epilogue_code
from helion_mlir_utils.matmul import _packed_layout

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(autouse=True)
def _auto_target(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.delenv("HELION_MLIR_TARGET", raising=False)


def test_devices_resolve_to_targets() -> None:
    assert B.resolve_target(torch.device("cpu")).name == "cpu"
    assert B.resolve_target(torch.device("cuda")).name == "gpu"
    assert B.resolve_target(torch.device("cuda", 0), "auto").name == "gpu"
    assert B.resolve_target(None, "gpu").name == "gpu"
    with pytest.raises(UnsupportedTargetError, match="meta tensors"):
        B.resolve_target(torch.device("meta"))
    with pytest.raises(ValueError, match="unknown MLIR target 'tpu'"):
        B.resolve_target(torch.device("cpu"), "tpu")


@pytest.mark.parametrize("value", ["gpu", "cpu", "auto", ""])
def test_environment_names_the_target(monkeypatch: pytest.MonkeyPatch, value: str) -> None:
    monkeypatch.setenv("HELION_MLIR_TARGET", value)
    expected = value if value in ("gpu", "cpu") else "cpu"
    assert B.resolve_target(torch.device("cpu")).name == expected


def test_unknown_target_in_environment_is_rejected(monkeypatch: pytest.MonkeyPatch) -> None:
    monkeypatch.setenv("HELION_MLIR_TARGET", "xpu")
    with pytest.raises(ValueError, match="HELION_MLIR_TARGET='xpu'"):
        B.resolve_target(torch.device("cpu"))


def test_gpu_target_pipelines() -> None:
    gpu = B.get_target("gpu")
    assert gpu.resolve_pipeline(None) == "hip"
    with pytest.raises(ValueError, match="pipeline 'opt' for the MLIR target 'gpu'"):
        gpu.resolve_pipeline("opt")
    with pytest.raises(NotImplementedError, match="only CUDA is supported"):
        gpu.check_tensor("x", torch.empty(2))


def test_install_without_helion_and_compile_api() -> None:
    assert B.install() is False  # Helion is not importable here
    with pytest.raises(UnsupportedTargetError, match="helion_mlir_utils"):
        B.compile_mlir(object(), [torch.empty(2)])


def test_cpu_tensors_are_refused_loudly() -> None:
    a, b = torch.randn(8, 8), torch.randn(8, 8)
    assert not U.supports(a, b)
    with pytest.raises(ValueError, match="does not support these operands"):
        U.matmul(a, b)
    with pytest.raises(ValueError, match="ROCm device"):
        U.softmax(a)
    with pytest.raises(ValueError, match="ROCm device"):
        U.rms_norm(a)
    with pytest.raises(ValueError, match="ROCm device"):
        U.relu(a)
    with pytest.raises(ValueError, match="does not support"):
        U.matvec(a, torch.randn(8, 1))
    assert not U.supports_matvec(a, torch.randn(8, 1))


def test_bmm_mismatch_raises_like_torch() -> None:
    a = torch.randn(3, 64, 64)
    with pytest.raises(RuntimeError, match="batch2"):
        U.bmm(a, torch.randn(1, 64, 64))
    with pytest.raises(RuntimeError, match="batch2"):
        U.bmm(a, torch.randn(3, 32, 64))


def test_shape_errors_come_first() -> None:
    with pytest.raises(ValueError, match="2-D"):
        U.softmax(torch.randn(2, 3, 4))
    with pytest.raises(ValueError, match="divisible by 3 groups"):
        U.group_norm(torch.randn(4, 8), 3, torch.ones(8), torch.zeros(8), 1e-5)
    with pytest.raises(ValueError, match="f32 vector"):
        U.row_dot(torch.randn(4, 8), torch.randn(8, dtype=torch.float64))


def test_epilogue_codes() -> None:
    assert epilogue_code(U.identity_epilogue) == (native.EPI_IDENTITY, 0.0, None)
    assert epilogue_code(torch.relu)[0] == native.EPI_RELU
    assert epilogue_code(F.silu)[0] == native.EPI_SILU
    assert epilogue_code(torch.sigmoid)[0] == native.EPI_SIGMOID
    assert epilogue_code(F.gelu)[0] == native.EPI_GELU
    assert epilogue_code(functools.partial(F.gelu, approximate="tanh"))[0] == native.EPI_GELU_TANH
    assert epilogue_code(functools.partial(F.leaky_relu, negative_slope=0.3)) == (native.EPI_LEAKY_RELU, 0.3, None)
    assert epilogue_code(U.Activation("leaky_relu", 0.2)) == (native.EPI_LEAKY_RELU, 0.2, None)
    # Other elementwise callables are traced into programs; one named
    # activation of the input keeps its code.
    code, _, program = epilogue_code(lambda x: x * 3)
    assert code == native.EPI_PROGRAM and program.count == 1
    assert epilogue_code(lambda x: F.gelu(x, approximate="tanh"))[:2] == (native.EPI_GELU_TANH, 0.0)
    assert epilogue_code(lambda x: x.float())[0] == native.EPI_IDENTITY
    with pytest.raises(ValueError, match="cannot fuse"):
        epilogue_code(lambda x: x.sum())

    def double(x: torch.Tensor) -> torch.Tensor:
        return torch.tanh(x)

    U.register_epilogue(double, "tanh")
    assert epilogue_code(double)[0] == native.EPI_TANH


def test_activation_objects_compute_what_they_fuse() -> None:
    x = torch.randn(100, dtype=torch.float64)
    torch.testing.assert_close(U.Activation("silu")(x), F.silu(x))
    torch.testing.assert_close(U.Activation("gelu_tanh")(x), F.gelu(x, approximate="tanh"))
    torch.testing.assert_close(U.Activation("leaky_relu", 0.2)(x), F.leaky_relu(x, 0.2))
    with pytest.raises(ValueError, match="unknown activation"):
        U.Activation("swish")


def test_packed_layouts_are_recognised_and_checked() -> None:
    a16 = torch.randn(40, 100).bfloat16()
    assert _packed_layout(a16, torch.empty(2, 64, 64, 2, dtype=torch.bfloat16), 70)[:3] == (native.B_VNNI_PANELS, 64, 128)
    assert _packed_layout(a16, torch.empty(3, 4, 32, 32, dtype=torch.bfloat16), 70)[0] == native.B_BLOCKED
    assert _packed_layout(a16, torch.empty(3, 4, 16, 32, 2, dtype=torch.bfloat16), 70)[0] == native.B_BLOCKED_VNNI
    assert _packed_layout(a16, torch.empty(2, 100, 64, dtype=torch.bfloat16), 70)[0] == native.B_PANELS
    with pytest.raises(ValueError, match="VNNI-packed RHS"):
        _packed_layout(a16, torch.empty(2, 50, 64, 2, dtype=torch.bfloat16), 70)
    with pytest.raises(ValueError, match="incompatible"):
        _packed_layout(a16, torch.empty(3, 3, 32, 32, dtype=torch.bfloat16), 70)
    with pytest.raises(ValueError, match="block shape"):
        _packed_layout(a16, torch.empty(3, 4, 16, 64, dtype=torch.bfloat16), 70)


def test_gemm_plan_of_the_baseline_configs() -> None:
    assert U.gemm_plan(torch.bfloat16, 4096, 4096, 4096) == {
        "splits": 1, "tile_m": 256, "tile_n": 256, "tile_k": 64, "workspace_bytes": 0}
    assert U.gemm_plan(torch.float32, 256, 256, 65536, batch=16)["splits"] >= 16
    # A decode-shaped linear (B [N, K]): the skinny kernel, no split.
    assert U.gemm_plan(torch.bfloat16, 32, 11008, 4096, trans_b=True) == {
        "splits": 1, "tile_m": 32, "tile_n": 32, "tile_k": 64, "workspace_bytes": 0}
    assert U.tall_output_tiles(8192, 11008, 4096) == (256, 256, 64)
    assert U.vnni_panel(128, 4096) == 256


def test_output_pool_api() -> None:
    from helion_mlir_backend import output_pool

    t = output_pool.empty((4, 5), dtype=torch.float32, device=torch.device("cpu"))
    assert t.shape == (4, 5)
    assert output_pool.empty_like(t, dtype=torch.bfloat16).dtype == torch.bfloat16
    stats = output_pool.output_pool_stats()
    assert set(stats) >= {"hits", "misses", "free_blocks", "free_bytes", "max_bytes"}
    B.set_output_pool(1 << 30)
    assert output_pool.enabled()


def test_bench_refuses_more_than_one_gpu() -> None:
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_explain_reports_the_library() -> None:
    info = B.explain()
    assert info["library_built"] in (True, False)
    assert "native_calls" in info
