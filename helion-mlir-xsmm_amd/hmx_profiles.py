"""Turns rocprofv3 output of ``bench.py`` runs into the summaries kept under
``profiles/``: a kernel-trace table per workload, and the HBM traffic per
launch from counter runs.

    python helion-mlir-xsmm_amd/hmx_profiles.py trace WORKLOAD TRACE_DIR BENCH_LOG OUT.md "TITLE" "COMMAND"
    python helion-mlir-xsmm_amd/hmx_profiles.py traffic PMC_ROOT OUT.json
    python helion-mlir-xsmm_amd/hmx_profiles.py clock PMC_ROOT OUT.md "TITLE" "COMMAND"
    python helion-mlir-xsmm_amd/hmx_profiles.py kfit PMC_ROOT OUT.md "TITLE" "COMMAND"

``TRACE_DIR`` holds ``run_kernel_trace.csv`` and ``run_kernel_stats.csv`` of
``rocprofv3 --kernel-trace --stats -o run -f csv -- python3 bench.py
--workload WORKLOAD --steps S ...``; ``BENCH_LOG`` is that run's stderr (the
``bench:`` lines). ``PMC_ROOT`` holds one directory per counter run, named
``<tag>_<workload>`` (tag ``rd``: ``TCC_EA0_RDREQ_{32B,64B,128B}_sum``; tag
``wr``: ``WRITE_SIZE``), each with ``run_counter_collection.csv``. For
``clock``, ``PMC_ROOT`` holds one directory per workload, each a counter run
with ``GRBM_GUI_ACTIVE`` and ``SQ_VALU_MFMA_BUSY_CYCLES`` (and its
``run_agent_info.csv``): the clock each GEMM dispatch ran at and the share of
SIMD cycles its MFMA unit was busy. ``kfit`` reads such runs of the 4096 x
4096 x K GEMM workloads (``gemm_k<K>``, ``gemm`` = 4096, ``gemm_longk`` =
16384) and fits, by least squares over K, the duration against K and each
SIMD's cycles outside the MFMA unit against its MFMA cycles: the intercepts
are the per-launch fixed cost.
"""

from __future__ import annotations

import collections
import csv
import json
from pathlib import Path
import re
import sys

_NS = re.compile(r"hmx::(\(anonymous namespace\)::)?")


def kernel_name(name: str, limit: int = 160) -> str:
    """A kernel's demangled name without the library's namespaces, cut to
    ``limit`` characters (torch's own kernels have names of several KB)."""
    name = _NS.sub("", name)
    return name if len(name) <= limit else name[: limit - 3] + "..."


def _rows(path: Path) -> list[dict]:
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


PASSES = 3  # bench.py's event-armed passes after its timed plain pass (LAUNCH_PASSES)


def step_spans(lib: list[dict], per_step: int) -> list[float]:
    """First kernel start to last kernel end (us) of each step, ``per_step``
    consecutive library kernels a step."""
    return [(int(lib[i + per_step - 1]["End_Timestamp"]) - int(lib[i]["Start_Timestamp"])) / 1e3
            for i in range(0, len(lib) - per_step + 1, per_step)]


def pass_means(spans: list[float], steps: int, passes: int = PASSES) -> tuple[list[float], list[float]]:
    """The steps of the timed plain pass and the means of the ``passes``
    event-armed passes after it: bench.py ends with the plain pass's
    ``steps`` steps followed by ``passes`` passes of ``steps`` steps."""
    tail = spans[-(passes + 1) * steps:]
    if len(tail) < (passes + 1) * steps:
        return tail, []
    plain, armed = tail[:steps], tail[steps:]
    return plain, [sum(armed[i * steps:(i + 1) * steps]) / steps for i in range(passes)]


def trace_summary(workload: str, trace_dir: Path, bench_log: Path, title: str, command: str,
                  steps: int = 20) -> str:
    """The markdown summary of one kernel-trace run: every kernel's calls and
    durations; the mean step span (first kernel start to last kernel end) of
    the library kernels in bench.py's timed plain pass and in each of its
    event-armed passes, and the lowest pass mean, which is what bench.py
    reports as ``launch_ms`` (a pass now and then runs every kernel 5-15 %
    slower than the others)."""
    trace = sorted(_rows(trace_dir / "run_kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    stats = _rows(trace_dir / "run_kernel_stats.csv")
    log = bench_log.read_text()
    bench_line = next((ln for ln in log.splitlines() if ln.startswith("bench:") and "ms/step" in ln), "")
    lib = [r for r in trace if "hmx::" in r["Kernel_Name"] and "pack" not in r["Kernel_Name"]]
    # kernels per step: the distinct library kernels of the last step's pattern
    names = list(dict.fromkeys(r["Kernel_Name"] for r in lib[-8:]))
    per_step = max(1, len(names))
    spans = step_spans(lib, per_step)
    plain, armed = pass_means(spans, steps)
    out = [f"# {title}: kernel trace", "", "Command:", "", "```", command, "```", "",
           "| Kernel | Calls | Average (us) | Min (us) | Max (us) | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in stats:
        out.append(f"| `{kernel_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    out += ["", "Calls include the warmup and the untimed settle steps bench.py runs before its timed region.", ""]
    if armed:
        out.append(f"Step spans ({per_step} library kernel(s) per step; first kernel start to last kernel end): "
                   f"the timed plain pass of {len(plain)} steps, mean {sum(plain) / len(plain):.2f} us, min "
                   f"{min(plain):.2f} us; the {len(armed)} event-armed passes after it, means "
                   + ", ".join(f"{a:.2f}" for a in armed)
                   + f" us. Kernel time per step (the lowest pass mean, bench.py's launch_ms): {min(armed):.2f} us.")
        out.append("")
    elif plain:
        out.append(f"The last {len(plain)} steps ({per_step} library kernel(s) per step; first kernel start to "
                   f"last kernel end): mean {sum(plain) / len(plain):.2f} us, min {min(plain):.2f} us per step.")
        out.append("")
    if bench_line:
        out += ["bench.py under the profiler (ms/step: the timed plain pass; ms/launch: the step's kernels, timed "
                f"by events they record themselves): `{bench_line}`", ""]
    return "\n".join(out)


def traffic(pmc_root: Path) -> dict:
    """Bytes per launch leaving L2 for the memory fabric, per workload: reads
    from the L2's memory read requests by size, writes from WRITE_SIZE (KiB),
    for the last dispatch of each kernel."""
    result: dict = collections.defaultdict(lambda: {"kernels": collections.defaultdict(dict)})
    for run in sorted(p for p in pmc_root.iterdir() if p.is_dir()):
        tag, _, workload = run.name.partition("_")
        path = run / "run_counter_collection.csv"
        if not path.is_file() or tag not in ("rd", "wr"):
            continue
        last: dict[tuple[str, str], tuple[int, float]] = {}
        dispatches: dict[str, set] = collections.defaultdict(set)
        for r in _rows(path):
            key = (kernel_name(r["Kernel_Name"]), r["Counter_Name"])
            disp = int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0)
            dispatches[key[0]].add(disp)
            if key not in last or disp >= last[key][0]:
                last[key] = (disp, float(r["Counter_Value"]))
        # The step's kernels run on every step; kernels of the workload's
        # set-up (input copies, a one-time pack) run once or twice.
        most = max((len(d) for d in dispatches.values()), default=0)
        per_kernel: dict[str, float] = collections.defaultdict(float)
        for (kernel, counter), (_, value) in last.items():
            if len(dispatches[kernel]) < most / 2:
                continue
            if tag == "rd":
                size = {"TCC_EA0_RDREQ_32B_sum": 32, "TCC_EA0_RDREQ_64B_sum": 64,
                        "TCC_EA0_RDREQ_128B_sum": 128}.get(counter)
                if size:
                    per_kernel[kernel] += size * value
            elif counter.startswith("WRITE_SIZE"):
                per_kernel[kernel] += 1024 * value
        for kernel, value in per_kernel.items():
            result[workload]["kernels"][kernel]["read_bytes" if tag == "rd" else "write_bytes"] = int(value)
    out = {}
    for workload, entry in sorted(result.items()):
        kernels = {k: dict(v) for k, v in entry["kernels"].items()}
        total = sum(v.get("read_bytes", 0) + v.get("write_bytes", 0) for v in kernels.values())
        out[workload] = {"kernels": kernels, "bytes_per_launch": total}
    method = {
        "read_bytes": "32 * TCC_EA0_RDREQ_32B_sum + 64 * TCC_EA0_RDREQ_64B_sum + 128 * TCC_EA0_RDREQ_128B_sum "
                      "(requests from L2 to the memory fabric, by size: HBM and MALL hits alike)",
        "write_bytes": "WRITE_SIZE * 1024",
        "dispatch": "the last dispatch of each kernel that runs on every step (set-up kernels excluded); "
                    "bytes_per_launch sums the step's kernels",
    }
    copy = out.get("copy")
    if copy:
        moved = 32768 * 8192 * 2  # the copy workload reads and writes 512 MiB
        rd = sum(v.get("read_bytes", 0) for v in copy["kernels"].values())
        wr = sum(v.get("write_bytes", 0) for v in copy["kernels"].values())
        method["calibration"] = (f"copy workload (torch copy of 512 MiB): read {rd / moved:.4f}, write "
                                 f"{wr / moved:.4f} of the bytes moved")
    out["_method"] = method
    return out


def _clock_rows(run: Path, last: int) -> tuple[str, float, float, float] | None:
    """(kernel, mean duration in us, clock in GHz, MFMA-busy share) of the
    last ``last`` dispatches of the longest-running kernel of one counter
    run, or None without one."""
    path = run / "run_counter_collection.csv"
    if not path.is_file():
        return None
    agent = next((r for r in _rows(run / "run_agent_info.csv") if r.get("Name", "").startswith("gfx")), {})
    xcc, simds = int(agent.get("Num_Xcc", 8)), int(agent.get("Simd_Count", 1024))
    disp: dict[int, dict] = collections.defaultdict(dict)
    for r in _rows(path):
        d = disp[int(r["Dispatch_Id"])]
        d["name"] = r["Kernel_Name"]
        d["dur"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        d[r["Counter_Name"]] = float(r["Counter_Value"])
    totals: dict[str, float] = collections.defaultdict(float)
    for d in disp.values():
        totals[d["name"]] += d["dur"]
    name = max(totals, key=totals.get)
    rows = [d for _, d in sorted(disp.items()) if d["name"] == name][-last:]
    dur = sum(d["dur"] for d in rows) / len(rows)
    clocks = [d["GRBM_GUI_ACTIVE"] / xcc / (d["dur"] * 1e3) for d in rows]
    busy = [d["SQ_VALU_MFMA_BUSY_CYCLES"] / simds / (d["GRBM_GUI_ACTIVE"] / xcc) for d in rows]
    return name, dur, sum(clocks) / len(rows), sum(busy) / len(rows)


def _dispatches(run: Path, name: str) -> int:
    """The number of dispatches of kernel ``name`` in a counter run."""
    return len({r["Dispatch_Id"] for r in _rows(run / "run_counter_collection.csv") if r["Kernel_Name"] == name})


def _line_fit(xs: list[float], ys: list[float]) -> tuple[float, float]:
    """Least-squares (intercept, slope) of ys against xs."""
    n = len(xs)
    mx, my = sum(xs) / n, sum(ys) / n
    sxx = sum((x - mx) ** 2 for x in xs)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sxx
    return my - slope * mx, slope


def kfit_summary(pmc_root: Path, title: str, command: str, last: int = 50) -> str:
    """The K sweep of the 4096 x 4096 x K GEMM. Per K: the duration, and per
    XCD the GRBM_GUI_ACTIVE cycles, per SIMD the MFMA-busy cycles. Then three
    least-squares lines over K: duration against K (the intercept is the
    per-launch fixed cost); GRBM cycles against duration (the slope is the
    clock; the intercept, cycles the counter adds outside the kernel's own
    timestamps, is why the cycles over the duration overstate the clock of
    short kernels); and, at the fitted clock, each SIMD's cycles outside the
    MFMA unit against its MFMA cycles."""
    pts = _k_points(pmc_root, last)
    ks = [p[0] for p in pts]
    durs = [p[2] for p in pts]
    grbm = [p[3] * p[2] * 1e3 for p in pts]  # cycles per XCD
    mfma = [p[4] * g for p, g in zip(pts, grbm)]  # busy cycles per SIMD
    out = [f"# {title}", "", "Command:", "", "```", command, "```", ""]
    if len(pts) < 2:
        return "\n".join(out + ["(fewer than two depths)"]) + "\n"
    f0, s0 = _line_fit(ks, durs)
    c0, ghz = _line_fit(durs, [g / 1e3 for g in grbm])  # kcycles against us: slope in GHz
    other = [ghz * d * 1e3 - m for d, m in zip(durs, mfma)]
    f1, s1 = _line_fit(mfma, other)
    out += ["| K | Kernel | Duration (us) | TFLOP/s | GRBM kcycles / XCD | GRBM / duration (GHz) | MFMA kcycles / SIMD |"
            " MFMA busy at the fitted clock |", "|---|---|---|---|---|---|---|---|"]
    for (k, name, dur, _clk, _util), g, m in zip(pts, grbm, mfma):
        out.append(f"| {k} | `{kernel_name(name)[:60]}` | {dur:.1f} | {2 * 4096 * 4096 * k / dur / 1e6:.0f} | "
                   f"{g / 1e3:.1f} | {g / 1e3 / dur:.3f} | {m / 1e3:.1f} | {m / (ghz * dur * 1e3):.3f} |")
    out += ["",
            f"Duration = {f0:.2f} us + {s0 * 1e3:.3f} us per 1000 of K (least squares over {len(pts)} depths): "
            f"the K-proportional part runs at {2 * 4096 * 4096 / s0 / 1e6:.0f} TFLOP/s, and the fixed {f0:.2f} us "
            f"per launch is {100 * f0 / (f0 + s0 * 4096):.1f} % of the 4096^3 launch.",
            f"GRBM cycles = {c0:.1f} kcycles + {ghz:.3f} GHz x duration: the clock is {ghz:.3f} GHz, and the "
            f"counter adds {c0:.1f} kcycles per dispatch ({c0 / ghz:.1f} us at that clock) outside the kernel's "
            f"timestamps.",
            f"Other cycles = {f1 / 1e3:.2f} kcycles + {s1:.3f} x MFMA cycles per SIMD (at {ghz:.3f} GHz): the K "
            f"loop spends {s1:.3f} cycles outside the MFMA unit per MFMA cycle, and each launch "
            f"{f1 / 1e3:.2f} kcycles ({f1 / ghz / 1e3:.1f} us) more."]
    return "\n".join(out) + "\n"


def _k_points(pmc_root: Path, last: int) -> list[tuple]:
    """(K, kernel, duration, GRBM cycles / duration, MFMA busy) of the 4096 x
    4096 x K GEMM runs in ``pmc_root``, by K."""
    names = {"gemm": 4096, "gemm_longk": 16384}
    pts = []
    for run in sorted(p for p in pmc_root.iterdir() if p.is_dir()):
        k = names.get(run.name) or (int(run.name[6:]) if run.name.startswith("gemm_k") else None)
        got = _clock_rows(run, last) if k else None
        if got:
            pts.append((k, *got))
    return sorted(pts)


def counter_window(pmc_root: Path, last: int = 50) -> tuple[float, float] | None:
    """(kcycles per XCD the GRBM counter adds outside a kernel's timestamps,
    the clock in GHz): the least-squares line of GRBM cycles against duration
    over the K-sweep runs in ``pmc_root``; None with fewer than two."""
    pts = _k_points(pmc_root, last)
    if len(pts) < 2:
        return None
    return _line_fit([p[2] for p in pts], [p[3] * p[2] for p in pts])


def clock_summary(pmc_root: Path, title: str, command: str, last: int = 50) -> str:
    """Per workload (a directory of ``pmc_root``): over the last ``last``
    dispatches of its longest-running kernel, the mean duration, the clock
    and the MFMA-busy share of SIMD cycles (SQ_VALU_MFMA_BUSY_CYCLES, summed
    over the SIMDs, over the XCD's cycles times the SIMD count). The clock is
    GRBM_GUI_ACTIVE cycles (counted once per XCD) over the duration, less the
    cycles the counter adds outside the kernel's timestamps when the K-sweep
    runs in the same root give them (``counter_window``); the raw ratio is
    shown beside it."""
    window = counter_window(pmc_root, last)
    c0 = window[0] * 1e3 if window else 0.0
    out = [f"# {title}", "", "Command:", "", "```", command, "```", ""]
    if window:
        out += [f"The GRBM counter adds {window[0]:.1f} kcycles per dispatch outside the kernel's timestamps "
                f"(least squares of its cycles against the duration over the 4096 x 4096 x K runs, slope "
                f"{window[1]:.3f} GHz); the clock column takes them off, the raw column does not.", ""]
    out += ["| Workload | Kernel | Dispatches | Duration (us) | Clock (GHz) | MFMA busy | Busy x clock | Raw GRBM / duration (GHz) |",
            "|---|---|---|---|---|---|---|---|"]
    for run in sorted(p for p in pmc_root.iterdir() if p.is_dir()):
        got = _clock_rows(run, last)
        if got is None:
            continue
        name, dur, raw, util_raw = got
        cycles = raw * dur * 1e3  # per XCD, raw
        clk = (cycles - c0) / (dur * 1e3)
        util = util_raw * cycles / (cycles - c0)
        out.append(f"| {run.name} | `{kernel_name(name)[:70]}` | {min(last, _dispatches(run, name))} | {dur:.1f} | "
                   f"{clk:.3f} | {util:.3f} | {clk * util:.3f} | {raw:.3f} |")
    return "\n".join(out) + "\n"


def main(argv: list[str]) -> int:
    if len(argv) >= 7 and argv[1] == "trace":
        _, _, workload, trace_dir, log, out, title, command = argv[:8]
        Path(out).write_text(trace_summary(workload, Path(trace_dir), Path(log), title, command))
        return 0
    if len(argv) == 6 and argv[1] == "kfit":
        Path(argv[3]).write_text(kfit_summary(Path(argv[2]), argv[4], argv[5]))
        return 0
    if len(argv) == 6 and argv[1] == "clock":
        Path(argv[3]).write_text(clock_summary(Path(argv[2]), argv[4], argv[5]))
        return 0
    if len(argv) == 4 and argv[1] == "traffic":
        Path(argv[3]).write_text(json.dumps(traffic(Path(argv[2])), indent=1, sort_keys=True) + "\n")
        return 0
    print(__doc__, file=sys.stderr)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv))
