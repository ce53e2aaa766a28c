"""Per-kernel counter report from rocprofv3 CSV output.

The counterpart of the reference's benchmark/parse_ncu_report.py, which reads an Nsight Compute
report and prints, per kernel, speed-of-light percentages, occupancy, registers and shared
memory, stall reasons, FLOPs from FFMA counts and DRAM bytes from sectors
(parse_ncu_report.py:53-102).  Here the inputs are rocprofv3 output directories written with
``-d DIR -o NAME -f csv``:

* ``--trace DIR``: a ``--kernel-trace --stats`` run (``*_kernel_stats.csv``): calls and mean
  duration per kernel.  With ``--trace-window SKIP:COUNT`` the means come from
  ``*_kernel_trace.csv`` over those dispatches of each kernel (a benchmark's timed steps).
* ``--pmc DIR`` (repeatable): ``--pmc`` runs (``*_counter_collection.csv``) with any counters;
  each counter is averaged per kernel over its dispatches.  One run may hold at most 8 SQ and
  4 TCC counters, so the counters below take several runs.
* ``--calibrate-fetch DIR --calibrate-write DIR --calibrate-bytes N``: FETCH_SIZE and
  WRITE_SIZE runs of a plain device copy of N bytes (``bench.py --copy-calibration-mib``).
  They give the factors that turn the two counters (KiB per dispatch) into HBM bytes.

Derived per kernel, when the counters it needs were collected:

==========================  =====================================================================
executed MFMA FLOP          SQ_INSTS_VALU_MFMA_MOPS_F32 x 512 (FP32 MFMA; one MOP = 512 FLOP)
MFMA utilisation            SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs)
clock under load            GRBM_GUI_ACTIVE / XCDs / that PMC run's duration (>= 0.2 ms)
achieved TFLOP/s            executed MFMA FLOP / mean duration (trace)
HBM bytes                   FETCH_SIZE x 1024 x f_fetch + WRITE_SIZE x 1024 x f_write
HBM GB/s                    HBM bytes / mean duration
arithmetic intensity        executed MFMA FLOP / HBM bytes
LDS bank-conflict rate      SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
scratch (spill) bytes       Scratch_Size of the dispatch
==========================  =====================================================================

GRBM_GUI_ACTIVE counts cycles on every XCD and is summed over them; the SQ counters are summed
over all SIMDs.  The report is Markdown with a machine-readable tail
(``traffic_bytes_per_launch[kernel] = ...`` and friends) that bench.py reads back.

Usage::

    python -m cuda_transformer_amd.rocprof_report --title T --trace DIR --pmc DIR [--pmc DIR ...]
        [--calibrate-fetch DIR --calibrate-write DIR --calibrate-bytes N] [--command CMD ...]
        [--out FILE.md]
"""
from __future__ import annotations

import argparse
import csv
import statistics
import sys
from dataclasses import dataclass, field
from pathlib import Path

MOP_FLOPS_F32 = 512  # FLOP per unit of SQ_INSTS_VALU_MFMA_MOPS_F32
MIN_CLOCK_MS = 0.2   # shortest kernel whose GRBM_GUI_ACTIVE gives a clock estimate


def _one(directory: Path, suffix: str) -> Path:
    hits = sorted(Path(directory).glob(f"*{suffix}"))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return hits[0]


def short_name(name: str) -> str:
    """The function name of a kernel.  rocprofv3's truncated names (-T) are already short, but
    it leaves names it cannot demangle (e.g. templates over __bf16, "DF16b") mangled; for those
    the last identifier of the Itanium nested name is taken, so template instances merge into
    one row as they do for demangled names."""
    if not name.startswith("_Z"):
        return name
    i = 3 if name.startswith("_ZN") else 2
    last = name
    while i < len(name) and name[i].isdigit():
        j = i
        while j < len(name) and name[j].isdigit():
            j += 1
        n = int(name[i:j])
        last = name[j:j + n]
        i = j + n
    return last


def read_kernel_stats(directory) -> dict[str, dict]:
    """{kernel: {calls, avg_ns, total_ns, share}} from a --kernel-trace --stats run."""
    out: dict[str, dict] = {}
    with open(_one(directory, "_kernel_stats.csv")) as f:
        for r in csv.DictReader(f):
            k = short_name(r["Name"])
            o = out.setdefault(k, {"calls": 0, "total_ns": 0.0, "share": 0.0})
            o["calls"] += int(r["Calls"])
            o["total_ns"] += float(r["TotalDurationNs"])
            o["share"] += float(r["Percentage"])
            o["avg_ns"] = o["total_ns"] / o["calls"]
    return out


def read_trace_window(directory, skip: int, count: int) -> dict[str, dict]:
    """{kernel: {calls, avg_ns, all_calls, all_avg_ns}} over dispatches [skip, skip + count) of
    each kernel, in start order, from a --kernel-trace run (``*_kernel_trace.csv``): the
    dispatches a benchmark timed, without its warm-up or later phases."""
    per: dict[str, list[tuple[int, int]]] = {}
    with open(_one(directory, "_kernel_trace.csv")) as f:
        for r in csv.DictReader(f):
            per.setdefault(short_name(r["Kernel_Name"]), []).append(
                (int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out = {}
    for k, ds in per.items():
        ds.sort()
        durs = [e - s for s, e in ds]
        win = durs[skip:skip + count]
        if win:
            out[k] = {"calls": len(win), "avg_ns": statistics.fmean(win),
                      "all_calls": len(durs), "all_avg_ns": statistics.fmean(durs)}
    return out


def read_counters(directory) -> tuple[dict[str, dict[str, float]], dict[str, dict]]:
    """({kernel: {counter: mean per dispatch}}, {kernel: dispatch info}) from a --pmc run."""
    vals: dict[str, dict[str, list[float]]] = {}
    info: dict[str, dict] = {}
    spans: dict[str, dict[str, int]] = {}  # kernel -> dispatch id -> duration (ns)
    with open(_one(directory, "_counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            k = short_name(r["Kernel_Name"])
            vals.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            info.setdefault(k, {"lds": int(r["LDS_Block_Size"]), "scratch": int(r["Scratch_Size"]),
                                "workgroup": int(r["Workgroup_Size"]), "grid": int(r["Grid_Size"])})
            spans.setdefault(k, {})[r["Dispatch_Id"]] = (int(r["End_Timestamp"])
                                                        - int(r["Start_Timestamp"]))
    for k, d in spans.items():
        info[k]["pmc_ms"] = statistics.fmean(d.values()) / 1e6
    return {k: {c: statistics.fmean(v) for c, v in cs.items()} for k, cs in vals.items()}, info


def read_agent(directory) -> dict:
    """The GPU agent's properties (CU / SIMD / XCD counts, clock) from *_agent_info.csv."""
    with open(_one(directory, "_agent_info.csv")) as f:
        for r in csv.DictReader(f):
            if r.get("Agent_Type", "").upper() == "GPU":
                return {"name": r["Name"], "cus": int(r["Cu_Count"]), "simds": int(r["Simd_Count"]),
                        "xcds": int(r["Num_Xcc"]), "max_clock_mhz": float(r["Max_Engine_Clk_Fcompute"])}
    raise ValueError(f"no GPU agent in {directory}")


def calibration(fetch_dir, write_dir, nbytes: int) -> tuple[float, float, str]:
    """(f_fetch, f_write, copy kernel name): bytes moved per KiB counted for a plain copy."""
    f, _ = read_counters(fetch_dir)
    w, _ = read_counters(write_dir)
    name = next((k for k in f if "copy" in k.lower()), None)
    if name is None or name not in w:
        raise ValueError("no copy kernel in the calibration runs")
    kib = nbytes / 1024
    return kib / f[name]["FETCH_SIZE"], kib / w[name]["WRITE_SIZE"], name


@dataclass
class KernelRow:
    name: str
    calls: int | None = None
    avg_ms: float | None = None
    share: float | None = None
    counters: dict[str, float] = field(default_factory=dict)
    info: dict = field(default_factory=dict)
    mfma_flop: float | None = None
    mfma_util: float | None = None
    clock_ghz: float | None = None
    tflops: float | None = None
    hbm_bytes: float | None = None
    hbm_gbps: float | None = None
    intensity: float | None = None
    lds_conflict_rate: float | None = None


def build_rows(trace=None, pmc=(), calib=None, agent=None, window=None) -> list[KernelRow]:
    """Join the trace and the PMC runs per kernel and derive the figures of the module doc.
    window = (skip, count) takes each kernel's mean duration over those dispatches only."""
    stats = read_kernel_stats(trace) if trace else {}
    if trace and window:
        win = read_trace_window(trace, *window)
        for k, w in win.items():
            stats.setdefault(k, {"share": None})
            stats[k].update(calls=w["calls"], avg_ns=w["avg_ns"], all_calls=w["all_calls"],
                            all_avg_ns=w["all_avg_ns"])
    counters: dict[str, dict[str, float]] = {}
    infos: dict[str, dict] = {}
    grbm_ms: dict[str, float] = {}  # duration of the dispatches GRBM_GUI_ACTIVE was read on
    for d in pmc:
        c, i = read_counters(d)
        for k, v in c.items():
            counters.setdefault(k, {}).update(v)
            if "GRBM_GUI_ACTIVE" in v and i[k]["pmc_ms"] > 0:
                grbm_ms[k] = i[k]["pmc_ms"]
        for k, v in i.items():
            infos.setdefault(k, v)
        if agent is None:
            try:
                agent = read_agent(d)
            except (FileNotFoundError, ValueError):
                pass
    names = list(stats) + [k for k in counters if k not in stats]
    rows = []
    for n in names:
        r = KernelRow(n, counters=counters.get(n, {}), info=infos.get(n, {}))
        if n in stats:
            r.calls, r.avg_ms, r.share = stats[n]["calls"], stats[n]["avg_ns"] / 1e6, stats[n]["share"]
            if "all_avg_ns" in stats[n]:
                r.info = {**r.info, "all_calls": stats[n]["all_calls"],
                          "all_avg_ms": stats[n]["all_avg_ns"] / 1e6}
        c = r.counters
        if "SQ_INSTS_VALU_MFMA_MOPS_F32" in c:
            r.mfma_flop = c["SQ_INSTS_VALU_MFMA_MOPS_F32"] * MOP_FLOPS_F32
            if r.avg_ms:
                r.tflops = r.mfma_flop / (r.avg_ms * 1e-3) / 1e12
        if agent and "GRBM_GUI_ACTIVE" in c and c["GRBM_GUI_ACTIVE"] > 0:
            cycles = c["GRBM_GUI_ACTIVE"] / agent["xcds"]
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                r.mfma_util = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * agent["simds"])
            # GRBM_GUI_ACTIVE includes dispatch overhead: a clock estimate needs a long kernel,
            # timed in the same run as the counter
            if grbm_ms.get(n, 0.0) >= MIN_CLOCK_MS:
                r.clock_ghz = cycles / (grbm_ms[n] * 1e-3) / 1e9
        if calib and "FETCH_SIZE" in c and "WRITE_SIZE" in c:
            r.hbm_bytes = 1024 * (c["FETCH_SIZE"] * calib[0] + c["WRITE_SIZE"] * calib[1])
            if r.avg_ms:
                r.hbm_gbps = r.hbm_bytes / (r.avg_ms * 1e-3) / 1e9
            if r.mfma_flop:
                r.intensity = r.mfma_flop / r.hbm_bytes
        if c.get("SQ_LDS_IDX_ACTIVE"):
            r.lds_conflict_rate = c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_LDS_IDX_ACTIVE"]
        rows.append(r)
    return rows


def _fmt(v, spec, unit=""):
    return "-" if v is None else format(v, spec) + unit


def render(rows: list[KernelRow], title: str, commands=(), calib=None, agent=None,
           window=None) -> str:
    lines = [f"# {title}", ""]
    if commands:
        lines += ["Commands (run from /tmp with TMPDIR=/tmp; R = repository root):", "", "```",
                  *commands, "```", ""]
    if agent:
        lines += [f"Device: {agent['name']}, {agent['cus']} CUs / {agent['simds']} SIMDs on "
                  f"{agent['xcds']} XCDs, {agent['max_clock_mhz']:.0f} MHz max.", ""]
    if window:
        lines += [f"Mean durations are over dispatches {window[0]}..{window[0] + window[1] - 1} of each "
                  f"kernel in launch order (the timed window); all-dispatch means follow the table.",
                  ""]
    if calib:
        lines += [f"HBM calibration: a plain copy ({calib[2]}) gives FETCH_SIZE x {calib[0]:.3f} "
                  f"and WRITE_SIZE x {calib[1]:.3f} (bytes moved per KiB counted).", ""]
    lines += ["| kernel | calls | mean ms | share | MFMA TFLOP/s | MFMA util | clock GHz | "
              "HBM GB | HBM GB/s | FLOP/B | LDS conflict | LDS B | scratch B |",
              "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        lines.append(
            f"| {r.name} | {_fmt(r.calls, 'd')} | {_fmt(r.avg_ms, '.4f')} | "
            f"{_fmt(r.share, '.1f', '%')} | {_fmt(r.tflops, '.1f')} | "
            f"{_fmt(None if r.mfma_util is None else 100 * r.mfma_util, '.1f', '%')} | "
            f"{_fmt(r.clock_ghz, '.2f')} | {_fmt(None if r.hbm_bytes is None else r.hbm_bytes / 1e9, '.3f')} | "
            f"{_fmt(r.hbm_gbps, '.0f')} | {_fmt(r.intensity, '.1f')} | "
            f"{_fmt(None if r.lds_conflict_rate is None else 100 * r.lds_conflict_rate, '.2f', '%')} | "
            f"{r.info.get('lds', '-')} | {r.info.get('scratch', '-')} |")
    if window:
        lines += ["", "| kernel | all dispatches | mean ms over all |", "|---|---|---|"]
        lines += [f"| {r.name} | {r.info['all_calls']} | {r.info['all_avg_ms']:.4f} |"
                  for r in rows if "all_calls" in r.info]
    tail = []
    for r in rows:
        if r.hbm_bytes is not None:
            tail.append(f"traffic_bytes_per_launch[{r.name}] = {r.hbm_bytes:.6e}")
        if r.mfma_flop is not None:
            tail.append(f"mfma_flop_per_launch[{r.name}] = {r.mfma_flop:.6e}")
        if r.mfma_util is not None:
            tail.append(f"mfma_util[{r.name}] = {r.mfma_util:.4f}")
        if r.avg_ms is not None:
            tail.append(f"mean_ms[{r.name}] = {r.avg_ms:.6f}")
    if tail:
        lines += ["", "Machine-readable:", "", "```", *tail, "```"]
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description="per-kernel report from rocprofv3 CSV directories")
    p.add_argument("--title", default="rocprofv3 kernel report")
    p.add_argument("--trace")
    p.add_argument("--pmc", action="append", default=[])
    p.add_argument("--calibrate-fetch")
    p.add_argument("--calibrate-write")
    p.add_argument("--calibrate-bytes", type=int)
    p.add_argument("--command", action="append", default=[],
                   help="a command that produced the inputs, quoted into the report")
    p.add_argument("--trace-window", metavar="SKIP:COUNT",
                   help="mean durations over dispatches [SKIP, SKIP+COUNT) of each kernel")
    p.add_argument("--out")
    a = p.parse_args(argv)
    window = tuple(int(x) for x in a.trace_window.split(":")) if a.trace_window else None
    calib = None
    if a.calibrate_fetch and a.calibrate_write and a.calibrate_bytes:
        calib = calibration(a.calibrate_fetch, a.calibrate_write, a.calibrate_bytes)
    agent = None
    for d in [*a.pmc, *([a.trace] if a.trace else [])]:
        try:
            agent = read_agent(d)
            break
        except (FileNotFoundError, ValueError):
            continue
    rows = build_rows(a.trace, a.pmc, calib, agent, window)
    text = render(rows, a.title, a.command, calib, agent, window)
    if a.out:
        Path(a.out).write_text(text)
    else:
        sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
