"""Turns rocprofv3 output of ``bench.py`` runs into the summaries kept under
``profiles/``: a kernel-trace table per workload, and the HBM traffic per
launch from counter runs.

    python helion-mlir-xsmm_amd/hmx_profiles.py trace WORKLOAD TRACE_DIR BENCH_LOG OUT.md "TITLE" "COMMAND"
    python helion-mlir-xsmm_amd/hmx_profiles.py traffic PMC_ROOT OUT.json
    python helion-mlir-xsmm_amd/hmx_profiles.py clock PMC_ROOT OUT.md "TITLE" "COMMAND"

``TRACE_DIR`` holds ``run_kernel_trace.csv`` and ``run_kernel_stats.csv`` of
``rocprofv3 --kernel-trace --stats -o run -f csv -- python3 bench.py
--workload WORKLOAD --steps S ...``; ``BENCH_LOG`` is that run's stderr (the
``bench:`` lines). ``PMC_ROOT`` holds one directory per counter run, named
``<tag>_<workload>`` (tag ``rd``: ``TCC_EA0_RDREQ_{32B,64B,128B}_sum``; tag
``wr``: ``WRITE_SIZE``), each with ``run_counter_collection.csv``. For
``clock``, ``PMC_ROOT`` holds one directory per workload, each a counter run
with ``GRBM_GUI_ACTIVE`` and ``SQ_VALU_MFMA_BUSY_CYCLES`` (and its
``run_agent_info.csv``): the clock each GEMM dispatch ran at and the share of
SIMD cycles its MFMA unit was busy.
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


def trace_summary(workload: str, trace_dir: Path, bench_log: Path, title: str, command: str,
                  steps: int = 20) -> str:
    """The markdown summary of one kernel-trace run: every kernel's calls and
    durations, and the mean span (first kernel start to last kernel end) of
    the library kernels of the last ``steps`` steps -- bench.py's second,
    event-armed pass."""
    trace = sorted(_rows(trace_dir / "run_kernel_trace.csv"), key=lambda r: int(r["Start_Timestamp"]))
    stats = _rows(trace_dir / "run_kernel_stats.csv")
    log = bench_log.read_text()
    bench_line = next((ln for ln in log.splitlines() if ln.startswith("bench:") and "ms/step" in ln), "")
    lib = [r for r in trace if "hmx::" in r["Kernel_Name"] and "pack" not in r["Kernel_Name"]]
    # kernels per step: the distinct library kernels of the last step's pattern
    names = list(dict.fromkeys(r["Kernel_Name"] for r in lib[-8:]))
    per_step = max(1, len(names))
    tail = lib[-steps * per_step:]
    spans = []
    for i in range(0, len(tail) - per_step + 1, per_step):
        group = tail[i:i + per_step]
        spans.append((int(group[-1]["End_Timestamp"]) - int(group[0]["Start_Timestamp"])) / 1e3)
    out = [f"# {title}: kernel trace", "", "Command:", "", "```", command, "```", "",
           "| Kernel | Calls | Average (us) | Min (us) | Max (us) | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in stats:
        out.append(f"| `{kernel_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |")
    out += ["", "Calls include the warmup and the untimed settle steps bench.py runs before its timed region.", ""]
    if spans:
        out.append(f"The last {len(spans)} steps ({per_step} library kernel(s) per step; first kernel start to "
                   f"last kernel end): mean {sum(spans) / len(spans):.2f} us, min {min(spans):.2f} us per step.")
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


def clock_summary(pmc_root: Path, title: str, command: str, last: int = 50) -> str:
    """Per workload (a directory of ``pmc_root``): over the last ``last``
    dispatches of its longest-running kernel, the mean duration, the clock
    (GRBM_GUI_ACTIVE cycles, counted once per XCD, over the duration), the
    MFMA-busy share of SIMD cycles (SQ_VALU_MFMA_BUSY_CYCLES, summed over the
    SIMDs, over the XCD's cycles times the SIMD count) and their product, the
    MFMA cycles per SIMD per nanosecond."""
    out = [f"# {title}", "", "Command:", "", "```", command, "```", "",
           "| Workload | Kernel | Dispatches | Duration (us) | Clock (GHz) | MFMA busy | Busy x clock |",
           "|---|---|---|---|---|---|---|"]
    for run in sorted(p for p in pmc_root.iterdir() if p.is_dir()):
        path = run / "run_counter_collection.csv"
        if not path.is_file():
            continue
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
        clk, util = sum(clocks) / len(rows), sum(busy) / len(rows)
        out.append(f"| {run.name} | `{kernel_name(name)[:70]}` | {len(rows)} | {dur:.1f} | {clk:.3f} | "
                   f"{util:.3f} | {clk * util:.3f} |")
    return "\n".join(out) + "\n"


def main(argv: list[str]) -> int:
    if len(argv) >= 7 and argv[1] == "trace":
        _, _, workload, trace_dir, log, out, title, command = argv[:8]
        Path(out).write_text(trace_summary(workload, Path(trace_dir), Path(log), title, command))
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
