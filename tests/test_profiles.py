"""The profile summariser (``helion-mlir-xsmm_amd/hmx_profiles.py``) on
synthetic rocprofv3 counter output: the K-sweep fit recovers the fixed cost
and rate it was built from, and the clock columns are the counters' ratios."""

from __future__ import annotations

import csv
from pathlib import Path

import pytest

import hmx_profiles as P

XCC, SIMDS = 8, 1024
KERNEL = "void hmx::(anonymous namespace)::gemm_bf16_mi16_kernel<1, 0, true, false, 256, 256, 8, 2>(hmx::GemmArgs)"


def _run(root: Path, name: str, dur_us: float, ghz: float, busy: float, dispatches: int = 60,
         window_kcycles: float = 0.0) -> None:
    # busy: the MFMA share of the kernel's own cycles; the GRBM counter also
    # counts window_kcycles outside the kernel's timestamps.
    run = root / name
    run.mkdir(parents=True)
    with open(run / "run_agent_info.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Name", "Num_Xcc", "Simd_Count"])
        w.writeheader()
        w.writerow({"Name": "gfx950", "Num_Xcc": XCC, "Simd_Count": SIMDS})
    cycles = dur_us * 1e3 * ghz  # per XCD, inside the kernel
    with open(run / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Counter_Name",
                               "Counter_Value"])
        w.writeheader()
        t = 1_000_000
        for d in range(dispatches):
            end = t + int(round(dur_us * 1e3))
            for counter, value in (("GRBM_GUI_ACTIVE", (cycles + window_kcycles * 1e3) * XCC),
                                   ("SQ_VALU_MFMA_BUSY_CYCLES", busy * cycles * SIMDS)):
                w.writerow({"Dispatch_Id": d, "Kernel_Name": KERNEL, "Start_Timestamp": t, "End_Timestamp": end,
                            "Counter_Name": counter, "Counter_Value": value})
            t = end + 5000


def test_line_fit_is_least_squares() -> None:
    f, s = P._line_fit([1.0, 2.0, 3.0, 4.0], [3.0, 5.1, 6.9, 9.0])
    assert s == pytest.approx(1.98, abs=1e-12) and f == pytest.approx(1.05, abs=1e-12)


def test_kfit_recovers_fixed_cost_and_rate(tmp_path: Path) -> None:
    fixed_us, per_k_us = 6.2, 0.0216  # duration = fixed + per_k * K
    fixed_cyc, ratio, ghz, window = 9000.0, 0.25, 2.0, 30.0  # other cycles = fixed + ratio * MFMA cycles
    names = {1024: "gemm_k1024", 2048: "gemm_k2048", 4096: "gemm", 8192: "gemm_k8192", 16384: "gemm_longk"}
    for k, name in names.items():
        dur = fixed_us + per_k_us * k
        cyc = dur * 1e3 * ghz
        mfma = (cyc - fixed_cyc) / (1 + ratio)  # so that cyc - mfma = fixed + ratio * mfma
        _run(tmp_path, name, dur, ghz, mfma / cyc, window_kcycles=window)
    _run(tmp_path, "linear", 500.0, ghz, 0.6)  # not a K point: ignored
    text = P.kfit_summary(tmp_path, "title", "cmd")
    rows = [ln for ln in text.splitlines() if ln.startswith("| ") and ln[2].isdigit()]
    assert [int(r.split("|")[1]) for r in rows] == sorted(names)
    assert f"Duration = {fixed_us:.2f} us + {per_k_us * 1e3:.3f} us per 1000 of K" in text
    assert f"{2 * 4096 * 4096 / per_k_us / 1e6:.0f} TFLOP/s" in text
    assert f"GRBM cycles = {window:.1f} kcycles + {ghz:.3f} GHz x duration" in text
    assert f"Other cycles = {fixed_cyc / 1e3:.2f} kcycles + {ratio:.3f} x MFMA cycles" in text
    # The clock table takes the window off: every depth at the true clock.
    table = P.clock_summary(tmp_path, "t", "c")
    for name in names.values():
        row = next(ln for ln in table.splitlines() if ln.startswith(f"| {name} |"))
        assert float(row.split("|")[5]) == pytest.approx(ghz, abs=1e-3)


def test_clock_columns_are_counter_ratios(tmp_path: Path) -> None:
    _run(tmp_path, "gemm", 98.0, 2.2, 0.6)
    name, dur, clk, busy = P._clock_rows(tmp_path / "gemm", 50)
    assert name == KERNEL
    assert dur == pytest.approx(98.0) and clk == pytest.approx(2.2) and busy == pytest.approx(0.6)


def test_clock_summary_row(tmp_path: Path) -> None:
    _run(tmp_path, "gemm", 98.0, 2.2, 0.6, dispatches=60)
    text = P.clock_summary(tmp_path, "t", "c")
    # No K sweep in the root: no window to take off, the clock is the raw ratio.
    assert ("| gemm | `void gemm_bf16_mi16_kernel<1, 0, true, false, 256, 256, 8, 2>(GemmArgs` | 50 | 98.0 | 2.200 | "
            "0.600 | 1.320 | 2.200 |") in text


def _trace(root: Path, durations_us: list[float], per_step: int = 1) -> Path:
    run = root / "kt"
    run.mkdir(parents=True)
    with open(run / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        t = 1_000_000
        for d in durations_us:
            for q in range(per_step):
                end = t + int(round(d * 1e3 / per_step))
                name = KERNEL if q == 0 else KERNEL.replace("gemm_bf16_mi16_kernel", f"reduce_{q}")
                w.writerow({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": end})
                t = end
            t += 9000
    with open(run / "run_kernel_stats.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": KERNEL, "Calls": len(durations_us), "AverageNs": 1e5, "MinNs": 9e4, "MaxNs": 1.1e5,
                    "Percentage": 100.0})
    (root / "bench.log").write_text("bench: gemm 0.0990 ms/step 1388.3 TFLOP/s, 0.0960 ms/launch\n")
    return run


def test_pass_means_split_the_tail() -> None:
    # settle steps, then the plain pass (20 x 96), then passes at 95, 110, 94
    spans = [120.0] * 7 + [96.0] * 20 + [95.0] * 20 + [110.0] * 20 + [94.0] * 20
    plain, armed = P.pass_means(spans, 20)
    assert plain == [96.0] * 20
    assert armed == pytest.approx([95.0, 110.0, 94.0])
    assert P.pass_means(spans[-30:], 20) == (spans[-30:], [])


def test_trace_summary_reports_the_lowest_pass(tmp_path: Path) -> None:
    # one slow pass (the second) must not set the kernel time; two kernels a
    # step are one span from the first's start to the second's end
    durations = [130.0] * 5 + [96.0] * 20 + [95.0] * 20 + [112.0] * 20 + [94.5] * 20
    run = _trace(tmp_path, durations, per_step=2)
    spans = P.step_spans(P._rows(run / "run_kernel_trace.csv"), 2)
    assert spans == pytest.approx(durations, abs=1e-3)
    text = P.trace_summary("gemm", run, tmp_path / "bench.log", "T", "cmd")
    assert "means 95.00, 112.00, 94.50 us" in text
    assert "(the lowest pass mean, bench.py's launch_ms): 94.50 us" in text
    assert "mean 96.00 us, min 96.00 us" in text
