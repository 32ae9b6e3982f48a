"""The BASELINE configurations as seeded synthetic inputs.

Inputs are drawn on the CPU with ``torch.Generator().manual_seed(seed)`` in
f32 (then cast), in a fixed order, so the GPU kernels, the CPU oracle and the
CPU baseline all see identical values:

1. f32 ``matmul`` ``A[512,512] @ B[512,512]``, U[-1,1], seed 0 (A first).
2. Row softmax + RMSNorm ``X[32768,4096]`` N(0, std 2) (bf16 and f32), seed 1;
   RMSNorm weight ``[4096]`` U[0.5,1.5] drawn after X, eps 1e-6.
3. bf16 GEMM ``A[4096,4096] @ B[4096,4096]`` U[-1,1], seed 2.
4. Fused linear ``SiLU(X @ W^T + b)``: X ``[8192,4096]`` N(0,1), W
   ``[11008,4096]`` N(0,0.02), b ``[11008]`` N(0,0.02), bf16, seed 3, drawn X, W, b.
5. Split-K bmm ``A[16,256,65536] @ B[16,65536,256]`` U[-1,1] f32 (and bf16), seed 4.

``scale`` shrinks every extent by that factor (for tests that need the same
distributions at small sizes).
"""

from __future__ import annotations

import torch

CONFIGS = {
    1: "f32 matmul 512^3",
    2: "softmax + RMSNorm [32768, 4096]",
    3: "bf16 GEMM 4096^3",
    4: "fused linear SiLU(X @ W^T + b) 8192 x 11008 x 4096",
    5: "split-K bmm [16, 256, 65536] @ [16, 65536, 256]",
}


def _uniform(g: torch.Generator, shape: tuple[int, ...]) -> torch.Tensor:
    return torch.rand(shape, generator=g, dtype=torch.float32) * 2.0 - 1.0


def _normal(g: torch.Generator, shape: tuple[int, ...], std: float) -> torch.Tensor:
    return torch.randn(shape, generator=g, dtype=torch.float32) * std


def config1(scale: int = 1) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(0)
    n = 512 // scale
    return {"a": _uniform(g, (n, n)), "b": _uniform(g, (n, n))}


def config2(dtype: torch.dtype = torch.bfloat16, scale: int = 1) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(1)
    x = _normal(g, (32768 // scale, 4096 // scale), 2.0)
    w = torch.rand((4096 // scale,), generator=g, dtype=torch.float32) + 0.5
    return {"x": x.to(dtype), "weight": w.to(dtype), "eps": 1e-6}


def config3(scale: int = 1) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(2)
    n = 4096 // scale
    return {"a": _uniform(g, (n, n)).to(torch.bfloat16), "b": _uniform(g, (n, n)).to(torch.bfloat16)}


def config4(scale: int = 1) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(3)
    m, n, k = 8192 // scale, 11008 // scale, 4096 // scale
    x = _normal(g, (m, k), 1.0).to(torch.bfloat16)
    w = _normal(g, (n, k), 0.02).to(torch.bfloat16)
    b = _normal(g, (n,), 0.02).to(torch.bfloat16)
    return {"x": x, "w": w, "b": b}


def config5(dtype: torch.dtype = torch.float32, scale: int = 1, batch: int = 16) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(4)
    m, n, k = 256 // scale, 256 // scale, 65536 // scale
    a = _uniform(g, (batch, m, k)).to(dtype)
    b = _uniform(g, (batch, k, n)).to(dtype)
    return {"a": a, "b": b}
