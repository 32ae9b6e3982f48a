#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X, in the driver's JSON-line format.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one call of the public entry point on inputs already resident in
HBM. The default workload is BASELINE config 3, the bf16 GEMM 4096^3
(``helion_mlir_utils.matmul``), whose TFLOP/s is ``value``; the same run also
measures config 2's softmax and RMSNorm (bf16, [32768, 4096]) in HBM GB/s and
reports them under ``components``. Other workloads (``--workload``) exist for
profiling one kernel at a time: gemm, gemm_f32c, gemm_prepacked, linear,
softmax, softmax_f32, rmsnorm, rmsnorm_f32, bmm, bmm_bf16, matmul_f32, and the
rest of the memory-bound API on BASELINE tensors: layernorm, groupnorm,
row_sum, column_sum, row_dot, matvec, relu, pack_vnni.

Timing: W untimed steps (and more, untimed, until the GPU has run 50 ms of
them: its clocks ramp up under load), then K steps bracketed by ``torch.cuda.synchronize()``
and HIP events recorded on the stream the kernels run on (torch's current
stream, which the library launches on); ``value`` spans all K steps. A second
pass of K steps gives each step its own event pair, recorded by the step's
first and last kernels themselves (``hmx_time_launches``):
``roofline.achieved`` is the algorithmic work per launch of the dominant
kernel over the mean of those pairs (its average launch duration, as a kernel
trace measures it). ``roofline.traffic`` is the bytes per launch that left the L2 caches for the
memory fabric, measured with rocprofv3 counters (``profiles/traffic.json``:
the L2's read requests to memory by size, and WRITE_SIZE); reads that hit the
256 MB last-level cache (MALL) in front of HBM count too, so for operands
that fit it the figure is L2-miss traffic, an upper bound on HBM bytes. Null
when not measured. ``cpu_baseline`` times the same math on the host with
torch (one thread per usable core: the process's CPU affinity, capped by
OMP_NUM_THREADS) on a bounded sample of the workload, with the CPU oracle
(``oracle/restate.py``, numpy) on the same sample beside it.
"""

from __future__ import annotations

import argparse
import gc
import json
import os
from pathlib import Path
import platform
import sys
import time

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "helion-mlir-xsmm_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "bf16 GEMM TFLOP/s (4096³) + softmax/RMSNorm HBM GB/s, % of MI355X roofline"
# MI355X published peaks: dense bf16 MFMA, dense f32 MFMA, HBM3E.
PEAK_BF16_TFLOPS = 2500.0
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_cores() -> int:
    """Host cores this process may use: its CPU affinity, capped by
    OMP_NUM_THREADS when that is set (a GPU box's share of its host)."""
    cores = len(os.sched_getaffinity(0))
    try:
        cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    except ValueError:
        pass
    return max(cores, 1)


def _torch_cpu(fn, work: float, budget_s: float = 10.0) -> tuple[float, int, int]:
    """(work units per second, reps, threads) of ``fn`` run by torch on the
    host with one thread per usable core."""
    import torch

    threads = _cpu_cores()
    torch.set_num_threads(threads)
    rate, reps = _time_cpu(fn, work, budget_s=budget_s)
    return rate, reps, threads


def _blas_limited(threads: int):
    """numpy's BLAS limited to ``threads`` threads (a context manager)."""
    try:
        from threadpoolctl import threadpool_limits

        return threadpool_limits(limits=threads, user_api="blas")
    except Exception:  # noqa: BLE001 - no limiter: numpy runs as configured
        import contextlib

        return contextlib.nullcontext()


class Workload:
    """One benchmarked entry point: ``step()`` runs it once on resident inputs."""

    name: str
    description: str
    unit: str  # "TFLOP/s" or "GB/s"
    bound: str  # "mfma" or "hbm"
    peak: float
    work: float  # algorithmic flops or bytes per step
    dtype: str
    kernel: str  # the dominant kernel's name (rocprof)
    library_kernels: bool = True  # a step enqueues libhmx kernels
    config: dict

    def step(self) -> object:
        raise NotImplementedError

    def cpu_baseline(self) -> dict:
        raise NotImplementedError


def _time_cpu(fn, work_per_call: float, budget_s: float = 10.0, max_reps: int = 50) -> tuple[float, int]:
    """(throughput in work units per second, reps) of ``fn`` after one warm-up,
    repeated until ``budget_s`` seconds of CPU work or ``max_reps``."""
    fn()
    reps, start = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        elapsed = time.perf_counter() - start
        if elapsed >= budget_s or reps >= max_reps:
            return work_per_call * reps / elapsed, reps


class Gemm(Workload):
    def __init__(self, device, out_dtype_name: str = "bf16", prepacked: bool = False) -> None:
        import torch

        import helion_mlir_utils as U
        import hmx_workloads as W

        cfg = W.config3()
        self.cpu_a, self.cpu_b = cfg["a"], cfg["b"]
        self.a, self.b = cfg["a"].to(device), cfg["b"].to(device)
        self.out_dtype = torch.bfloat16 if out_dtype_name == "bf16" else torch.float32
        self.U = U
        self.prepacked = U.pack_b_blocked_vnni(self.b) if prepacked else None
        m = n = k = 4096
        self.name = "gemm_prepacked" if prepacked else ("gemm" if out_dtype_name == "bf16" else "gemm_f32c")
        self.description = "bf16 GEMM 4096^3 (config 3)" + (", B pre-packed (pack_b_blocked_vnni)" if prepacked else "")
        self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_BF16_TFLOPS
        self.work = 2.0 * m * n * k
        self.dtype = "bf16"
        # Row-major and blocked VNNI B both run the 16x16x32 direct-to-LDS kernel.
        self.kernel = "gemm_bf16_mi16_kernel"
        self.config = {"workload": self.description, "m": m, "n": n, "k": k, "a": "bf16 row-major",
                       "b": "bf16 row-major" if not prepacked else "bf16 [N/32,K/32,16,32,2]",
                       "c": out_dtype_name, "seed": 2, "values": "U[-1,1]"}

    def step(self):
        if self.prepacked is not None:
            return self.U.matmul_prepacked_b(self.a, self.prepacked, 4096)
        return self.U.matmul(self.a, self.b, out_dtype=self.out_dtype)

    def cpu_baseline(self) -> dict:
        """torch's CPU bf16 matmul (oneDNN, f32 accumulation) on the first
        512 rows of A -- the restatement the reference's CPU path is timed
        as -- and, beside it, the numpy oracle on the same rows."""
        import torch

        from oracle import restate as R

        rows = 512
        a16, b16 = self.cpu_a[:rows].contiguous(), self.cpu_b
        work = 2.0 * rows * 4096 * 4096
        rate, reps, threads = _torch_cpu(lambda: torch.matmul(a16, b16), work)
        a, b = a16.float().numpy(), b16.float().numpy()
        with _blas_limited(threads):
            o_rate, o_reps = _time_cpu(lambda: R.matmul(a, b, out="bf16"), work, budget_s=5.0)
        return {"value": rate / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
                "sample": f"torch.matmul bf16 on the CPU (oneDNN, f32 accumulate) of A[:{rows}] @ B, 4096 x 4096 "
                          f"B, {reps} reps, {threads} threads, {_cpu_model()}",
                "oracle": {"value": o_rate / 1e12, "unit": "TFLOP/s",
                           "sample": f"oracle.restate.matmul (numpy f32 BLAS) on the same rows, {o_reps} reps"}}


class GemmLongK(Workload):
    """bf16 GEMM 4096 x 4096 x K through the library: config 3's kernel at
    other depths (K = 16384: the steady state, where the per-launch fixed
    cost -- first loads, the epilogue's C writes -- is a quarter as large a
    share as at K = 4096; the sweep over K separates the two)."""

    def __init__(self, device, k: int = 16384) -> None:
        import torch

        import helion_mlir_utils as U

        g = torch.Generator().manual_seed(2)
        m = n = 4096
        self.a = (torch.rand(m, k, generator=g) * 2 - 1).to(torch.bfloat16).to(device)
        self.b = (torch.rand(k, n, generator=g) * 2 - 1).to(torch.bfloat16).to(device)
        self.U = U
        self.name = "gemm_longk" if k == 16384 else f"gemm_k{k}"
        self.description = f"bf16 GEMM 4096 x 4096 x {k} (config 3 kernel, K = {k})"
        self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_BF16_TFLOPS
        self.work = 2.0 * m * n * k
        self.dtype = "bf16"
        self.kernel = "gemm_bf16_mi16_kernel"
        self.config = {"workload": self.description, "m": m, "n": n, "k": k, "seed": 2, "values": "U[-1,1]"}

    def step(self):
        return self.U.matmul(self.a, self.b)

    def cpu_baseline(self) -> dict:
        return {"value": None, "unit": "TFLOP/s", "cores": 0, "kind": "port", "sample": "none (steady-state probe)"}


class VendorGemm(Workload):
    """torch.matmul (hipBLASLt) on config 3's operands, or on the long-K
    shape: the vendor library's kernel as a reference point for clock and
    MFMA-utilisation counters, not a hot-path op."""

    def __init__(self, device, k: int = 4096) -> None:
        import torch

        g = torch.Generator().manual_seed(2)
        m = n = 4096
        self.a = (torch.rand(m, k, generator=g) * 2 - 1).to(torch.bfloat16).to(device)
        self.b = (torch.rand(k, n, generator=g) * 2 - 1).to(torch.bfloat16).to(device)
        self.name = "gemm_hipblaslt" if k == 4096 else "gemm_longk_hipblaslt"
        self.description = f"torch.matmul (hipBLASLt) bf16 4096 x 4096 x {k} (reference point)"
        self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_BF16_TFLOPS
        self.work = 2.0 * m * n * k
        self.dtype = "bf16"
        self.kernel = "Cijk"
        self.library_kernels = False
        self.config = {"workload": self.description, "m": m, "n": n, "k": k, "seed": 2, "values": "U[-1,1]"}

    def step(self):
        return self.a @ self.b

    def cpu_baseline(self) -> dict:
        return {"value": None, "unit": "TFLOP/s", "cores": 0, "kind": "port", "sample": "none (reference point)"}


class Linear(Workload):
    def __init__(self, device) -> None:
        import torch
        import torch.nn.functional as F

        import helion_mlir_utils as U
        import hmx_workloads as W

        cfg = W.config4()
        self.cpu = cfg
        x, w, b = (cfg[k].to(device) for k in ("x", "w", "b"))
        layer = torch.nn.Linear(4096, 11008, device=device, dtype=torch.bfloat16)
        with torch.no_grad():
            layer.weight.copy_(w)
            layer.bias.copy_(b)
        self.x, self.layer, self.U, self.F = x, layer, U, F
        self.cache = None
        self.name = "linear"
        self.description = "fused linear SiLU(X @ W^T + b), 8192 x 11008 x 4096 (config 4)"
        self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_BF16_TFLOPS
        self.work = 2.0 * 8192 * 11008 * 4096
        self.dtype = "bf16"
        # 256x256 tiles over the first 10240 columns (five rounds), then 256x128 tiles over the last 768.
        self.kernel = "gemm_bf16_mi16_rounds_kernel (256x256 rounds and the 256x128 tail, one launch)"
        self.config = {"workload": self.description, "m": 8192, "n": 11008, "k": 4096, "seed": 3}

    def step(self):
        import torch

        with torch.no_grad():
            y, self.cache = self.U.linear(self.x, self.layer, self.F.silu, cache=self.cache)
        return y

    def cpu_baseline(self) -> dict:
        """torch's CPU bf16 F.linear + SiLU (oneDNN) on the first 256 of 8192
        rows, and the numpy oracle on the same rows."""
        import torch
        import torch.nn.functional as F

        from oracle import restate as R

        rows = 256
        x16, w16, b16 = self.cpu["x"][:rows].contiguous(), self.cpu["w"], self.cpu["b"]
        work = 2.0 * rows * 11008 * 4096
        rate, reps, threads = _torch_cpu(lambda: F.silu(F.linear(x16, w16, b16).float()).to(torch.bfloat16), work)
        x, w, b = x16.float().numpy(), w16.float().numpy(), b16.float().numpy()
        with _blas_limited(threads):
            o_rate, o_reps = _time_cpu(lambda: R.matmul(x, w, False, True, b, act="silu", out="bf16"), work,
                                       budget_s=5.0)
        return {"value": rate / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
                "sample": f"torch F.linear bf16 + SiLU on the CPU (oneDNN) of the first {rows} of 8192 rows, "
                          f"{reps} reps, {threads} threads, {_cpu_model()}",
                "oracle": {"value": o_rate / 1e12, "unit": "TFLOP/s",
                           "sample": f"oracle.restate.matmul (numpy) on the same rows, {o_reps} reps"}}


class LinearDecode(Linear):
    """Config 4's layer at decode shape: the first 32 rows of X, so the step
    streams W once (HBM-bound; the skinny kernel)."""

    ROWS = 32

    def __init__(self, device) -> None:
        super().__init__(device)
        r = self.ROWS
        self.x = self.x[:r].contiguous()
        self.name = "linear_decode"
        self.description = f"fused linear SiLU(X @ W^T + b), {r} x 11008 x 4096 (config 4's layer, {r} rows)"
        self.unit, self.bound, self.peak = "GB/s", "hbm", PEAK_HBM_GBS
        # W, X and b read once, Y written once.
        self.work = 2.0 * (11008 * 4096 + r * 4096 + 11008 + r * 11008)
        self.kernel = "gemm_bf16_skinny_kernel"
        self.config = {"workload": self.description, "m": r, "n": 11008, "k": 4096, "seed": 3}

    def cpu_baseline(self) -> dict:
        import torch
        import torch.nn.functional as F

        x16, w16, b16 = self.cpu["x"][: self.ROWS].contiguous(), self.cpu["w"], self.cpu["b"]
        rate, reps, threads = _torch_cpu(lambda: F.silu(F.linear(x16, w16, b16).float()).to(torch.bfloat16),
                                         self.work)
        return {"value": rate / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"torch F.linear bf16 + SiLU on the CPU (oneDNN) of the whole {self.ROWS}-row problem, "
                          f"{reps} reps, {threads} threads, {_cpu_model()}"}


class RowOp(Workload):
    def __init__(self, device, op: str, dtype_name: str) -> None:
        import torch

        import helion_mlir_utils as U
        import hmx_workloads as W

        dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float32
        cfg = W.config2(dtype)
        self.cpu = cfg
        self.x, self.w, self.eps = cfg["x"].to(device), cfg["weight"].to(device), cfg["eps"]
        self.U, self.op = U, op
        m, n = map(int, self.x.shape)
        esz = self.x.element_size()
        self.name = op + ("" if dtype_name == "bf16" else "_f32")
        self.description = f"row {op} [{m}, {n}] {dtype_name} (config 2)"
        self.unit, self.bound, self.peak = "GB/s", "hbm", PEAK_HBM_GBS
        self.work = 2.0 * m * n * esz + (n * esz if op == "rmsnorm" else 0)  # one read + one write
        self.dtype = dtype_name
        # bf16 RMSNorm rows run two to a workgroup (rmsnorm_cached2).
        self.kernel = ("softmax_cached" if op == "softmax"
                       else "rmsnorm_cached2" if dtype_name == "bf16" else "rmsnorm_cached")
        self.config = {"workload": self.description, "m": m, "n": n, "seed": 1, "values": "N(0, std 2)"}
        if op == "rmsnorm":
            self.config["eps"] = self.eps

    def step(self):
        if self.op == "softmax":
            return self.U.softmax(self.x)
        return self.U.rms_norm(self.x, self.w, self.eps)

    def cpu_baseline(self) -> dict:
        """torch on the host (f32 inside, one rounding to the input dtype, as
        the kernels compute) over the first 4096 rows, and the numpy oracle
        on the same rows."""
        import torch

        from oracle import restate as R

        rows = 4096
        xt = self.cpu["x"][:rows].contiguous()
        wt = self.cpu["weight"].float()
        dtype, eps = xt.dtype, self.eps
        if self.op == "softmax":
            def fn():
                return torch.softmax(xt.float(), -1).to(dtype)
        else:
            def fn():
                xf = xt.float()
                return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps) * wt).to(dtype)
        work = self.work * rows / self.x.shape[0]
        rate, reps, threads = _torch_cpu(fn, work, budget_s=5.0)
        x = xt.float().numpy()
        w = wt.numpy()
        out = self.dtype
        ofn = (lambda: R.softmax(x, out)) if self.op == "softmax" else (lambda: R.rms_norm(x, w, eps, out))
        o_rate, o_reps = _time_cpu(ofn, work, budget_s=3.0)
        name = "softmax" if self.op == "softmax" else "rms_norm"
        return {"value": rate / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"torch {name} on the CPU (f32 inside) of the first {rows} of {self.x.shape[0]} rows, "
                          f"{reps} reps, {threads} threads, {_cpu_model()}",
                "oracle": {"value": o_rate / 1e9, "unit": "GB/s", "cores": 1,
                           "sample": f"oracle.restate.{name} (numpy, one thread) on the same rows, {o_reps} reps"}}


class MemOp(Workload):
    """The rest of the memory-bound API, each on a BASELINE tensor: LayerNorm,
    GroupNorm (32 groups), row_sum, column_sum, row_dot, matvec and relu on
    config 2's X ([32768, 4096] bf16), and the VNNI weight pack
    (``pack_b_vnni_t``, 64-column panels) of config 4's W ([11008, 4096] bf16).
    ``work`` is one HBM read of each input and one write of each output."""

    def __init__(self, device, op: str) -> None:
        import torch

        import helion_mlir_utils as U
        import hmx_workloads as W

        self.U, self.op = U, op
        g = torch.Generator().manual_seed(5)
        if op == "pack_vnni":
            self.cpu = {"w": W.config4()["w"]}
            self.w = self.cpu["w"].to(device)
            n, k = map(int, self.w.shape)
            self.work = 2.0 * n * k * 2
            self.description = f"pack_b_vnni_t [{n}, {k}] bf16, 64-column panels (config 4's weight)"
            self.kernel = "pack_kernel"
            self.config = {"workload": self.description, "n": n, "k": k, "panel": 64, "seed": 3}
        else:
            cfg = W.config2(torch.bfloat16)
            x = cfg["x"]
            m, n = map(int, x.shape)
            vec = torch.randn(n, generator=g)
            self.cpu = {"x": x, "w": cfg["weight"].float(), "b": vec * 0.1, "v": vec}
            self.x = x.to(device)
            self.w32 = self.cpu["w"].to(device)
            self.b32 = self.cpu["b"].to(device)
            self.v32 = vec.to(device)
            self.v16 = vec.to(torch.bfloat16).reshape(n, 1).to(device)
            rw = 2.0 * m * n  # X once, bf16
            self.work = {"layernorm": 2 * rw + 8 * n, "groupnorm": 2 * rw + 8 * n, "row_sum": rw + 2 * m,
                         "column_sum": rw + 4 * n, "row_dot": rw + 4 * n + 2 * m, "matvec": rw + 2 * n + 2 * m,
                         "relu": 2 * rw}[op]
            self.kernel = {"layernorm": "group_norm_rows", "groupnorm": "group_norm_rows",
                           "row_sum": "row_reduce", "column_sum": "column_partial_kernel + column_final_kernel", "row_dot": "row_reduce",
                           "matvec": "row_reduce", "relu": "elementwise_kernel"}[op]
            self.description = f"{op} [{m}, {n}] bf16 (config 2's X)"
            self.config = {"workload": self.description, "m": m, "n": n, "seed": 1, "values": "N(0, std 2)"}
        self.name = op
        self.unit, self.bound, self.peak = "GB/s", "hbm", PEAK_HBM_GBS
        self.dtype = "bf16"

    def step(self):
        U = self.U
        if self.op == "pack_vnni":
            return U.pack_b_vnni_t(self.w, 64)
        if self.op == "layernorm":
            return U.layer_norm(self.x, self.w32, self.b32, 1e-5)
        if self.op == "groupnorm":
            return U.group_norm(self.x, 32, self.w32, self.b32, 1e-5)
        if self.op == "row_sum":
            return U.row_sum(self.x)
        if self.op == "column_sum":
            return U.column_sum(self.x)
        if self.op == "row_dot":
            return U.row_dot(self.x, self.v32)
        if self.op == "matvec":
            return U.matvec(self.x, self.v16)
        return U.relu(self.x)

    def cpu_baseline(self) -> dict:
        from oracle import restate as R

        if self.op == "pack_vnni":
            rows = 1024
            w = self.cpu["w"][:rows].float().numpy()
            rate, reps = _time_cpu(lambda: R.pack_b_vnni_t(w, 64), self.work * rows / self.w.shape[0])
            return {"value": rate / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                    "sample": f"oracle.restate.pack_b_vnni_t on the first {rows} of {self.w.shape[0]} rows, "
                              f"{reps} reps, {_cpu_model()}"}
        rows = 4096
        x = self.cpu["x"][:rows].float().numpy()
        w, b, v = (self.cpu[k].numpy() for k in ("w", "b", "v"))
        fn = {"layernorm": lambda: R.group_norm(x, 1, w, b, 1e-5, out="bf16"),
              "groupnorm": lambda: R.group_norm(x, 32, w, b, 1e-5, out="bf16"),
              "row_sum": lambda: R.row_sum(x, out="bf16"),
              "column_sum": lambda: R.column_sum(x),
              "row_dot": lambda: R.row_dot(x, v, out="bf16"),
              "matvec": lambda: R.matvec(x, v, out="bf16"),
              "relu": lambda: R.relu(x, out="bf16")}[self.op]
        rate, reps = _time_cpu(fn, self.work * rows / self.x.shape[0])
        return {"value": rate / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"oracle.restate ({self.op}) on the first {rows} of {self.x.shape[0]} rows, {reps} reps, "
                          f"{_cpu_model()}"}


class Bmm(Workload):
    def __init__(self, device, dtype_name: str) -> None:
        import torch

        import helion_mlir_utils as U
        import hmx_workloads as W

        dtype = torch.float32 if dtype_name == "f32" else torch.bfloat16
        cfg = W.config5(dtype)
        self.cpu = cfg
        self.a, self.b = cfg["a"].to(device), cfg["b"].to(device)
        self.U = U
        self.plan = U.gemm_plan(dtype, 256, 256, 65536, batch=16)
        self.name = "bmm" if dtype_name == "f32" else "bmm_bf16"
        self.description = (f"split-K bmm [16,256,65536] @ [16,65536,256] {dtype_name}-in, f32 out, "
                            f"S={self.plan['splits']} (config 5)")
        if dtype_name == "f32":
            self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_F32_TFLOPS
            self.kernel = "gemm_f32_dma_kernel + splitk_reduce_kernel"
        else:
            self.unit, self.bound, self.peak = "GB/s", "hbm", PEAK_HBM_GBS
            self.kernel = "gemm_bf16_dma64_kernel + splitk_reduce_kernel"
        self.flops = 2.0 * 16 * 256 * 256 * 65536
        esz = 4 if dtype_name == "f32" else 2
        self.bytes = 16 * (256 * 65536 * 2) * esz + 16 * 256 * 256 * 4
        self.work = self.flops if self.unit == "TFLOP/s" else self.bytes
        self.dtype = dtype_name
        self.config = {"workload": self.description, "batch": 16, "m": 256, "n": 256, "k": 65536,
                       "splits": self.plan["splits"], "seed": 4, "values": "U[-1,1]"}

    def step(self):
        import torch

        return self.U.bmm(self.a, self.b, out_dtype=torch.float32)

    def cpu_baseline(self) -> dict:
        """torch.bmm on the CPU (f32 out) of 2 of the 16 batch slices, and the
        numpy oracle's split-K bmm of one slice."""
        import torch

        from oracle import restate as R

        a2, b2 = self.cpu["a"][:2].contiguous(), self.cpu["b"][:2].contiguous()
        if a2.dtype == torch.bfloat16:
            def fn():
                return torch.bmm(a2, b2).float()
        else:
            def fn():
                return torch.bmm(a2, b2)
        rate, reps, threads = _torch_cpu(fn, self.work / 8)
        a = self.cpu["a"][:1].float().numpy()
        b = self.cpu["b"][:1].float().numpy()
        s = self.plan["splits"]
        with _blas_limited(threads):
            o_rate, o_reps = _time_cpu(lambda: R.split_k_bmm(a, b, s), self.work / 16, budget_s=5.0, max_reps=20)
        scale = 1e12 if self.unit == "TFLOP/s" else 1e9
        return {"value": rate / scale, "unit": self.unit, "cores": threads, "kind": "port",
                "sample": f"torch.bmm on the CPU of 2 of 16 batch slices, {reps} reps, {threads} threads, "
                          f"{_cpu_model()}",
                "oracle": {"value": o_rate / scale, "unit": self.unit,
                           "sample": f"oracle.restate.split_k_bmm of 1 slice, S={s}, {o_reps} reps"}}


class MatmulF32(Workload):
    def __init__(self, device) -> None:
        import helion_mlir_utils as U
        import hmx_workloads as W

        cfg = W.config1()
        self.cpu = cfg
        self.a, self.b = cfg["a"].to(device), cfg["b"].to(device)
        self.U = U
        self.name = "matmul_f32"
        self.description = "f32 matmul 512^3 (config 1)"
        self.unit, self.bound, self.peak = "TFLOP/s", "mfma", PEAK_F32_TFLOPS
        self.work = 2.0 * 512**3
        self.dtype = "f32"
        self.kernel = "gemm_f32_kernel + splitk_reduce_kernel"
        self.config = {"workload": self.description, "m": 512, "n": 512, "k": 512, "seed": 0,
                       "block_sizes": [64, 64, 64]}

    def step(self):
        return self.U.matmul(self.a, self.b, block_sizes=[64, 64, 64])

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import restate as R

        at, bt = self.cpu["a"], self.cpu["b"]
        torch.set_num_threads(_cpu_cores())
        rate, reps = _time_cpu(lambda: torch.matmul(at, bt), self.work, budget_s=5.0, max_reps=2000)
        a, b = at.numpy(), bt.numpy()
        with _blas_limited(_cpu_cores()):
            o_rate, o_reps = _time_cpu(lambda: R.matmul(a, b), self.work, budget_s=3.0, max_reps=2000)
        return {"value": rate / 1e12, "unit": "TFLOP/s", "cores": _cpu_cores(), "kind": "port",
                "sample": f"torch.matmul 512^3 f32 on the CPU, {reps} reps, {_cpu_cores()} threads, {_cpu_model()}",
                "oracle": {"value": o_rate / 1e12, "unit": "TFLOP/s",
                           "sample": f"oracle.restate.matmul 512^3 f32 (numpy), {o_reps} reps"}}


class Copy(Workload):
    """A plain device copy of known size (torch's copy kernel): the calibration
    point for the rocprofv3 traffic counters, not a hot-path op."""

    def __init__(self, device) -> None:
        import torch

        self.x = torch.empty((32768, 8192), dtype=torch.bfloat16, device=device).fill_(1.0)
        self.y = torch.empty_like(self.x)
        self.name = "copy"
        self.description = "device copy of 512 MiB (counter calibration)"
        self.unit, self.bound, self.peak = "GB/s", "hbm", PEAK_HBM_GBS
        self.work = 2.0 * self.x.numel() * 2
        self.dtype = "bf16"
        self.kernel = "copy"
        self.library_kernels = False
        self.config = {"workload": self.description, "bytes_read": self.x.numel() * 2, "bytes_written": self.x.numel() * 2}

    def step(self):
        return self.y.copy_(self.x)

    def cpu_baseline(self) -> dict:
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": "none (calibration workload)"}


MEM_OPS = ("layernorm", "groupnorm", "row_sum", "column_sum", "row_dot", "matvec", "relu", "pack_vnni")


def make(name: str, device) -> Workload:
    return {
        "gemm": lambda: Gemm(device),
        "gemm_f32c": lambda: Gemm(device, "f32"),
        "gemm_prepacked": lambda: Gemm(device, prepacked=True),
        "gemm_longk": lambda: GemmLongK(device),
        **{f"gemm_k{k}": (lambda k=k: GemmLongK(device, k)) for k in (1024, 2048, 8192)},
        "gemm_hipblaslt": lambda: VendorGemm(device),
        "gemm_longk_hipblaslt": lambda: VendorGemm(device, 16384),
        "linear": lambda: Linear(device),
        "linear_decode": lambda: LinearDecode(device),
        "softmax": lambda: RowOp(device, "softmax", "bf16"),
        "softmax_f32": lambda: RowOp(device, "softmax", "f32"),
        "rmsnorm": lambda: RowOp(device, "rmsnorm", "bf16"),
        "rmsnorm_f32": lambda: RowOp(device, "rmsnorm", "f32"),
        "bmm": lambda: Bmm(device, "f32"),
        "bmm_bf16": lambda: Bmm(device, "bf16"),
        "matmul_f32": lambda: MatmulF32(device),
        "copy": lambda: Copy(device),
        **{op: (lambda op=op: MemOp(device, op)) for op in MEM_OPS},
    }[name]()


# Untimed load before the timed region (seconds of back-to-back steps).
SETTLE_S = 0.05
LAUNCH_PASSES = 3


def measure(w: Workload, steps: int, warmup: int) -> dict:
    """:func:`_measure` with Python's cyclic garbage collector paused, as
    ``timeit`` does: a full collection in the middle of a pass stalls the host
    for tens of milliseconds (39 ms seen between two launches of the pre-packed
    GEMM), the GPU idles meanwhile, and the passes after it run at the lower
    clock it comes back from."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        return _measure(w, steps, warmup)
    finally:
        if was:
            gc.enable()


def _measure(w: Workload, steps: int, warmup: int) -> dict:
    """Step time (ms) over ``steps`` timed steps, and the average duration of
    one step's kernels, both from HIP events on the stream the library
    launches on (torch's current stream).

    ``ms`` spans the timed region: a pair of events around exactly ``steps``
    back-to-back steps, with nothing else on the stream. Before it, after the
    ``warmup`` steps, untimed steps continue until the GPU has been busy for
    SETTLE_S: the clocks ramp up over the first ~10 ms of load (a timed
    region started right after 10 warmup steps of the 4096^3 GEMM measures
    ~130 us per step, the next one ~116 us).

    ``launch_ms`` comes from further passes of ``steps`` steps after it. For
    each step a pair of events is armed in the library
    (``hmx_time_launches``): the first kernel of the step records the start
    event as it begins and its last kernel the stop event as it ends, so the
    mean of a pass's pairs is the GPU time of the step's kernels without host
    time -- what a kernel trace reports. A pass now and then runs every
    kernel 5-15 % slower than the plain pass just before it (seen on either
    GEMM workload, in the first pass of a process or a later one), so there
    are LAUNCH_PASSES passes: ``launch_ms`` is the lowest pass mean and
    ``launch_passes_ms`` lists them all. Kernels that
    record events are dispatched later than plain launches (a 16 us kernel
    then takes ~43 us per step instead of 16 us), which is why the step time
    comes from the uninstrumented pass. Workloads that launch no library
    kernel (the calibration copy) bracket each step with plain event records.
    """
    import torch

    from helion_mlir_backend._compiler import native

    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    chunk = 1
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(chunk):
            w.step()
        torch.cuda.synchronize()
        chunk = min(2 * chunk, 1024)
    begin = torch.cuda.Event(enable_timing=True)
    finish = torch.cuda.Event(enable_timing=True)
    begin.record()
    for _ in range(steps):
        w.step()
    finish.record()
    torch.cuda.synchronize()
    ms = begin.elapsed_time(finish) / steps

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    armed = w.library_kernels
    if armed:
        for ev in starts + ends:  # creates the events; the kernels re-record them
            ev.record()
        torch.cuda.synchronize()
    passes = []
    for _ in range(LAUNCH_PASSES):
        for i in range(steps):
            if armed:
                native.time_launches(starts[i], ends[i])
                w.step()
            else:
                starts[i].record()
                w.step()
                ends[i].record()
        if armed:
            native.time_launches(None, None)
        torch.cuda.synchronize()
        passes.append(sum(a.elapsed_time(b) for a, b in zip(starts, ends)) / steps)
    scale = 1e12 if w.unit == "TFLOP/s" else 1e9
    value = w.work / (ms * 1e-3) / scale
    return {"ms": ms, "launch_ms": min(passes), "launch_passes_ms": passes, "value": value,
            "frac": value / w.peak}


def traffic_of(name: str) -> float | None:
    """HBM bytes per launch of the step's kernels, from the rocprofv3 counter
    runs recorded in profiles/traffic.json (L2-to-memory read requests by size,
    WRITE_SIZE)."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        entry = json.loads(path.read_text()).get(name)
    except (OSError, ValueError):
        return None
    if not entry or entry.get("bytes_per_launch") is None:
        return None
    return float(entry["bytes_per_launch"])


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="gemm")
    parser.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    parser.add_argument("--no-components", action="store_true", help="skip the softmax/RMSNorm lines")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (every box here has one GPU; "
              "the path is measured on one GPU's share at its real shape)", file=sys.stderr)
        return 2

    import torch

    device = torch.device("cuda", 0)
    print(f"bench: workload={args.workload} steps={args.steps} warmup={args.warmup}", file=sys.stderr, flush=True)
    w = make(args.workload, device)
    result = measure(w, args.steps, args.warmup)
    print(f"bench: {w.name} {result['ms']:.4f} ms/step {result['value']:.1f} {w.unit}, "
          f"{result['launch_ms']:.4f} ms/launch", file=sys.stderr, flush=True)

    # The launch time spans all of a step's kernels: one launch, or two for the
    # split-K bmm (split GEMM + fixed-order reduction), the linear's whole-round
    # split (256 x 256 head + 256 x 128 tail) and column_sum (partials + sum).
    per_launch_ms = result["launch_ms"]
    achieved = w.work / (per_launch_ms * 1e-3) / (1e12 if w.unit == "TFLOP/s" else 1e9)
    roofline = {
        "bound": w.bound,
        "achieved": round(achieved, 2),
        "peak": w.peak,
        "unit": w.unit,
        "frac": round(achieved / w.peak, 4),
        "traffic": traffic_of(w.name),
        "kernel": w.kernel,
        "launch_ms": round(per_launch_ms, 5),
        "launch_passes_ms": [round(x, 5) for x in result["launch_passes_ms"]],
    }
    line = {
        "metric": METRIC,
        "value": round(result["value"], 2),
        "unit": w.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(result["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic (seeded, BASELINE config distributions)",
        "config": w.config,
        "roofline": roofline,
    }
    if args.workload == "gemm" and not args.no_components:
        components = {}
        for name in ("softmax", "rmsnorm"):
            cw = make(name, device)
            r = measure(cw, args.steps, args.warmup)
            achieved_c = cw.work / (r["launch_ms"] * 1e-3) / 1e9
            components[name + "_bf16"] = {
                "value": round(r["value"], 1), "unit": "GB/s", "frac": round(r["frac"], 4),
                "ms_per_step": round(r["ms"], 5),
                "roofline": {"bound": "hbm", "achieved": round(achieved_c, 1), "peak": PEAK_HBM_GBS,
                             "unit": "GB/s", "frac": round(achieved_c / PEAK_HBM_GBS, 4),
                             "traffic": traffic_of(cw.name), "kernel": cw.kernel,
                             "launch_ms": round(r["launch_ms"], 5)},
                "config": cw.config,
            }
            print(f"bench: {name} {r['ms']:.4f} ms/step {r['value']:.1f} GB/s", file=sys.stderr, flush=True)
            if not args.no_cpu_baseline:
                components[name + "_bf16"]["cpu_baseline"] = cw.cpu_baseline()
            del cw
        line["components"] = components
    if not args.no_cpu_baseline:
        print("bench: timing the CPU oracle baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = w.cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
