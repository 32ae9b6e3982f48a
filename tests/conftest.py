"""Test setup: import paths, the ``gpu`` marker and shared fixtures.

``-m "not gpu"`` runs everywhere (oracle pins, host logic, the C ABI's
exports and argument checks); ``-m gpu`` runs the parity tests of the gfx950
kernels against the CPU oracle and needs a ROCm device and a built
``libhmx.so`` -- on a GPU box a missing library fails the tests rather than
skipping them.
"""

from __future__ import annotations

from pathlib import Path
import sys

import pytest

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT, ROOT / "helion-mlir-xsmm_amd"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libhmx.so")


@pytest.fixture(scope="session")
def gpu_device():
    """``cuda:0`` after checking it is a gfx950 the library runs on."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    from helion_mlir_backend._compiler import native

    device = torch.device("cuda", 0)
    native.ensure_device(device)  # raises if the library is missing or the GPU is not gfx950
    return device
