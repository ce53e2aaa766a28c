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
executed MFMA FLOP          SQ_INSTS_VALU_MFMA_MOPS_{F32,BF16,F16} x 512 (one MOP = 512 FLOP)
MFMA utilisation            SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs)
clock under load            GRBM_GUI_ACTIVE / XCDs / that PMC run's duration (>= 0.2 ms)
achieved TFLOP/s            executed MFMA FLOP / mean duration (trace)
HBM bytes                   FETCH_SIZE x 1024 x f_fetch + WRITE_SIZE x 1024 x f_write
HBM GB/s                    HBM bytes / mean duration
arithmetic intensity        executed MFMA FLOP / HBM bytes
LDS bank-conflict rate      SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
scratch (spill) bytes       Scratch_Size of the dispatch
registers                   2 x VGPR_Count, 2 x Accum_VGPR_Count (AGPRs), SGPR_Count of the
                            dispatch (rocprofv3 reports half the VGPR allocation on gfx950)
theoretical waves / SIMD    min(8, 512 // (VGPRs + AGPRs, each rounded up to 8),
                            LDS: (163840 // LDS_Block_Size) workgroups per CU x waves per
                            workgroup / 4 SIMDs), with the limiting resource named
achieved waves / SIMD       4 x SQ_WAVE_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs)
wave states                 SQ_ACTIVE_INST_ANY (issuing), SQ_WAIT_ANY (waiting on a dependency:
                            s_waitcnt on memory, barriers), SQ_WAIT_INST_ANY (ready but not
                            issued: pipe busy), SQ_WAIT_INST_LDS, and the issuing time by unit
                            (SQ_ACTIVE_INST_VALU / _LDS / _VMEM / _SCA / _MISC), each as a share
                            of SQ_WAVE_CYCLES (all in quad-cycles)
memory / fetch latency      rocprofv3's derived metrics VmemLatency, LdsLatency and
                            InstrFetchLatency: the in-flight instruction level (SQ_INST_LEVEL_VMEM,
                            _LDS, SQ_IFETCH_LEVEL) accumulated every cycle over the instructions
                            issued (SQ_INSTS_VMEM, _LDS, SQ_IFETCH), i.e. the mean cycles a
                            vector-memory, LDS or instruction-fetch request is outstanding (one
                            --pmc pass each)
==========================  =====================================================================

The reference parser splits stalls into memory dependency, pipe busy, barrier and instruction
fetch (parse_ncu_report.py:71-80).  Here: memory dependency = the dependency-wait share with the
VMEM / LDS latencies beside it; pipe busy = the issue-wait share; instruction fetch =
InstrFetchLatency.  gfx950's counter set has no barrier-wait counter (SQ_WAIT_ANY counts s_waitcnt
and s_barrier waits together), and PC sampling, which would give per-reason stalls, is not
available on the pool this was measured on; barrier waits are therefore measured with clock reads
around the barrier in an instrumented build, not by this report.

MFMA FLOPs count the FP32, BF16 and FP16 MOPS counters that were collected (512 FLOP each).
The wave-state and occupancy figures are rocprofv3's counterparts of the reference parser's
achieved occupancy, registers per thread and stall breakdown (parse_ncu_report.py:60-80).

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

MOP_FLOPS_F32 = 512  # FLOP per unit of SQ_INSTS_VALU_MFMA_MOPS_{F32,BF16,F16}
MOPS_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                 "SQ_INSTS_VALU_MFMA_MOPS_F16")
MIN_CLOCK_MS = 0.2   # shortest kernel whose GRBM_GUI_ACTIVE gives a clock estimate
# gfx950 (CDNA4) resources per SIMD / CU that bound occupancy
VGPR_FILE = 512      # unified VGPR + AGPR entries per lane of a SIMD
VGPR_GRANULE = 8
MAX_WAVES_PER_SIMD = 8
LDS_PER_CU = 160 * 1024
SIMDS_PER_CU = 4
# wave-state counters, reported as shares of SQ_WAVE_CYCLES
WAVE_STATES = (("issue", "SQ_ACTIVE_INST_ANY"), ("dep_wait", "SQ_WAIT_ANY"),
               ("issue_wait", "SQ_WAIT_INST_ANY"), ("lds_issue_wait", "SQ_WAIT_INST_LDS"),
               ("valu", "SQ_ACTIVE_INST_VALU"), ("lds", "SQ_ACTIVE_INST_LDS"),
               ("vmem", "SQ_ACTIVE_INST_VMEM"), ("salu", "SQ_ACTIVE_INST_SCA"),
               ("branch", "SQ_ACTIVE_INST_MISC"))
# derived latency metrics (cycles), reported as they are
LATENCIES = (("vmem", "VmemLatency"), ("lds", "LdsLatency"), ("ifetch", "InstrFetchLatency"))


def _round_up(x: int, g: int) -> int:
    return -(-x // g) * g


def theoretical_waves(vgpr: int, agpr: int, lds: int, workgroup: int) -> tuple[int, str]:
    """(waves per SIMD, limiting resource) for one kernel on gfx950: the unified register
    file (VGPRs and AGPRs, each allocated in granules of 8, from 512 per lane), the 160 KiB of
    LDS per CU shared by whole workgroups (a workgroup's waves spread over the 4 SIMDs), and the
    8 wave slots of a SIMD."""
    regs = _round_up(max(vgpr, 1), VGPR_GRANULE) + _round_up(agpr, VGPR_GRANULE)
    limits = {"slots": MAX_WAVES_PER_SIMD, "vgpr": VGPR_FILE // regs}
    if lds > 0:
        waves_per_wg = -(-max(workgroup, 1) // 64)
        limits["lds"] = (LDS_PER_CU // lds) * waves_per_wg // SIMDS_PER_CU
    which = min(limits, key=lambda k: (limits[k], k != "slots"))
    return limits[which], which


def _one(directory: Path, suffix: str) -> Path:
    hits = sorted(Path(directory).glob(f"*{suffix}"))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return hits[0]


def short_name(name: str) -> str:
    """The function name of a kernel.  Demangled names lose the return type, this library's
    namespaces and the argument list, and keep their template arguments (which tell the tile
    and row-length variants apart): "void cta::(anonymous namespace)::k<64, true>(float*)" ->
    "k<64, true>".  rocprofv3's truncated names (-T) are already short.  Names it cannot
    demangle (e.g. templates over __bf16, "DF16b") stay mangled; for those the last identifier
    of the Itanium nested name is taken, with its template arguments decoded where they are
    integer, boolean or floating-point types and literals (so instances stay apart)."""
    if not name.startswith("_Z"):
        n = name[5:] if name.startswith("void ") else name
        n = n.replace("(anonymous namespace)::", "")
        depth = 0
        for i, ch in enumerate(n):
            if ch == "<":
                depth += 1
            elif ch == ">":
                depth -= 1
            elif ch == "(" and depth == 0:
                n = n[:i]
                break
        return n.replace("cta::", "")
    i = 3 if name.startswith("_ZN") else 2
    last = name
    while i < len(name) and name[i].isdigit():
        j = i
        while j < len(name) and name[j].isdigit():
            j += 1
        n = int(name[i:j])
        last = name[j:j + n]
        i = j + n
    if i < len(name) and name[i] == "I":
        args = _template_args(name, i + 1)
        if args is not None:
            last += "<" + ", ".join(args) + ">"
    return last


_TYPE_CODES = {"DF16b": "bf16", "DF16_": "f16", "f": "float", "d": "double", "i": "int",
               "j": "unsigned", "b": "bool"}


def _template_args(name: str, i: int) -> list[str] | None:
    """Decode the Itanium template arguments starting at name[i] (after the 'I') up to the
    closing 'E': literals L<type><value>E of integer and boolean types, and the builtin types of
    _TYPE_CODES.  None when anything else appears."""
    out = []
    while i < len(name) and name[i] != "E":
        if name[i] == "L":
            t = name[i + 1]
            j = name.find("E", i + 2)
            if t not in "bijlm" or j < 0:
                return None
            v = name[i + 2:j].replace("n", "-")
            out.append(("true" if v == "1" else "false") if t == "b" else v)
            i = j + 1
            continue
        for code, text in _TYPE_CODES.items():
            if name.startswith(code, i):
                out.append(text)
                i += len(code)
                break
        else:
            return None
    return out


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


def read_trace_window(directory, skip: int, count: int,
                      per_step: dict[str, int] | None = None) -> dict[str, dict]:
    """{kernel: {calls, avg_ns, all_calls, all_avg_ns}} over dispatches [skip, skip + count) of
    each kernel, in start order, from a --kernel-trace run (``*_kernel_trace.csv``): the
    dispatches a benchmark timed, without its warm-up or later phases.  skip and count count
    steps; a kernel launched k times per step (per_step[kernel] = k, e.g. once per head chunk)
    takes dispatches [k skip, k (skip + count)); a per_step key names a kernel by its short name
    or by the base identifier before its template arguments (exact match, never a substring:
    fa2_bwd_dq_kernel does not match fa2_bwd_dq_ds_kernel<...>)."""
    per: dict[str, list[tuple[int, int]]] = {}
    with open(_one(directory, "_kernel_trace.csv")) as f:
        for r in csv.DictReader(f):
            per.setdefault(short_name(r["Kernel_Name"]), []).append(
                (int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out = {}
    for k, ds in per.items():
        ds.sort()
        durs = [e - s for s, e in ds]
        ps = per_step or {}
        mult = ps.get(k, ps.get(k.split("<", 1)[0], 1))
        win = durs[mult * skip:mult * (skip + count)]
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
                                "workgroup": int(r["Workgroup_Size"]), "grid": int(r["Grid_Size"]),
                                **_regs(r)})
            spans.setdefault(k, {})[r["Dispatch_Id"]] = (int(r["End_Timestamp"])
                                                        - int(r["Start_Timestamp"]))
    for k, d in spans.items():
        info[k]["pmc_ms"] = statistics.fmean(d.values()) / 1e6
    return {k: {c: statistics.fmean(v) for c, v in cs.items()} for k, cs in vals.items()}, info


# rocprofv3 reports VGPR_Count on gfx950 as half the allocation: kernels the compiler reports
# at 145, 140 and 256 VGPRs (-Rpass-analysis=kernel-resource-usage) appear as 76, 72 and 128
# (152, 144 and 256 allocated in granules of 8, halved), and only the doubled counts give the
# occupancy the SQ counters measure (3, 3 and 2 waves per SIMD).  AGPRs are taken the same way.
REG_COUNT_SCALE = 2


def _regs(r) -> dict:
    return {"vgpr": REG_COUNT_SCALE * int(r.get("VGPR_Count") or 0),
            "agpr": REG_COUNT_SCALE * int(r.get("Accum_VGPR_Count") or 0),
            "sgpr": int(r.get("SGPR_Count") or 0)}


def read_trace_info(directory) -> dict[str, dict]:
    """{kernel: {lds, scratch, workgroup, grid, vgpr, agpr, sgpr}} of each kernel's first
    dispatch in a --kernel-trace run (``*_kernel_trace.csv``); {} without one."""
    hits = sorted(Path(directory).glob("*_kernel_trace.csv"))
    out: dict[str, dict] = {}
    if not hits:
        return out
    with open(hits[0]) as f:
        for r in csv.DictReader(f):
            k = short_name(r["Kernel_Name"])
            if k in out or "LDS_Block_Size" not in r:
                continue
            wg = 1
            for axis in ("X", "Y", "Z"):
                wg *= int(r.get(f"Workgroup_Size_{axis}") or 1)
            out[k] = {"lds": int(r["LDS_Block_Size"]), "scratch": int(r["Scratch_Size"]),
                      "workgroup": wg, **_regs(r)}
    return out


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
    waves_theory: int | None = None
    waves_limit: str | None = None
    waves_achieved: float | None = None
    wave_states: dict[str, float] = field(default_factory=dict)
    latencies: dict[str, float] = field(default_factory=dict)


def build_rows(trace=None, pmc=(), calib=None, agent=None, window=None,
               per_step=None) -> list[KernelRow]:
    """Join the trace and the PMC runs per kernel and derive the figures of the module doc.
    window = (skip, count) takes each kernel's mean duration over those steps' dispatches only
    (per_step: dispatches per step of kernels launched more than once a step)."""
    stats = read_kernel_stats(trace) if trace else {}
    if trace and window:
        win = read_trace_window(trace, *window, per_step)
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
    if trace:
        for k, v in read_trace_info(trace).items():
            infos.setdefault(k, v)
    names = list(stats) + [k for k in counters if k not in stats]
    rows = []
    for n in names:
        r = KernelRow(n, counters=counters.get(n, {}), info=infos.get(n, {}))
        if "vgpr" in r.info:
            r.waves_theory, r.waves_limit = theoretical_waves(
                r.info["vgpr"], r.info["agpr"], r.info["lds"], r.info["workgroup"])
        if n in stats:
            r.calls, r.avg_ms, r.share = stats[n]["calls"], stats[n]["avg_ns"] / 1e6, stats[n]["share"]
            if "all_avg_ns" in stats[n]:
                r.info = {**r.info, "all_calls": stats[n]["all_calls"],
                          "all_avg_ms": stats[n]["all_avg_ns"] / 1e6}
        c = r.counters
        if any(m in c for m in MOPS_COUNTERS):
            r.mfma_flop = sum(c.get(m, 0.0) for m in MOPS_COUNTERS) * MOP_FLOPS_F32
            if r.avg_ms:
                r.tflops = r.mfma_flop / (r.avg_ms * 1e-3) / 1e12
        if c.get("SQ_WAVE_CYCLES"):
            r.wave_states = {key: c[ctr] / c["SQ_WAVE_CYCLES"] for key, ctr in WAVE_STATES
                             if ctr in c}
        if agent and "GRBM_GUI_ACTIVE" in c and c["GRBM_GUI_ACTIVE"] > 0:
            cycles = c["GRBM_GUI_ACTIVE"] / agent["xcds"]
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                r.mfma_util = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (cycles * agent["simds"])
            if "SQ_WAVE_CYCLES" in c:
                r.waves_achieved = 4 * c["SQ_WAVE_CYCLES"] / (cycles * agent["simds"])
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
        r.latencies = {key: c[ctr] for key, ctr in LATENCIES if ctr in c}
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
                  f"kernel in launch order (the timed window; kernels dispatched k times a step: "
                  f"k times those indices); all-dispatch means follow the table.", ""]
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
    occ = [r for r in rows if r.waves_theory is not None or r.wave_states]
    if occ:
        pct = lambda v: _fmt(None if v is None else 100 * v, ".1f", "%")  # noqa: E731
        lines += ["", "Registers, occupancy and wave states (shares of wave-cycles; issue + "
                  "dependency wait + issue wait need not sum to 100%: a wave can be in none):", "",
                  "| kernel | VGPR | AGPR | SGPR | waves/SIMD theory (limit) | waves/SIMD achieved | "
                  "issuing | dep. wait | issue wait | LDS issue wait | VALU+MFMA | LDS | VMEM | "
                  "SALU | branch |",
                  "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
        for r in occ:
            w = r.wave_states
            theory = "-" if r.waves_theory is None else f"{r.waves_theory} ({r.waves_limit})"
            lines.append(
                f"| {r.name} | {r.info.get('vgpr', '-')} | {r.info.get('agpr', '-')} | "
                f"{r.info.get('sgpr', '-')} | {theory} | {_fmt(r.waves_achieved, '.2f')} | "
                f"{pct(w.get('issue'))} | {pct(w.get('dep_wait'))} | {pct(w.get('issue_wait'))} | "
                f"{pct(w.get('lds_issue_wait'))} | {pct(w.get('valu'))} | {pct(w.get('lds'))} | "
                f"{pct(w.get('vmem'))} | {pct(w.get('salu'))} | {pct(w.get('branch'))} |")
    lat = [r for r in rows if r.latencies]
    if lat:
        lines += ["", "Memory and instruction-fetch latency (mean cycles a request is outstanding):",
                  "", "| kernel | VMEM latency | LDS latency | instruction-fetch latency |",
                  "|---|---|---|---|"]
        for r in lat:
            lines.append(f"| {r.name} | {_fmt(r.latencies.get('vmem'), '.0f')} | "
                         f"{_fmt(r.latencies.get('lds'), '.0f')} | "
                         f"{_fmt(r.latencies.get('ifetch'), '.0f')} |")
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
        if r.waves_theory is not None:
            tail.append(f"waves_per_simd_theory[{r.name}] = {r.waves_theory}")
        if r.waves_achieved is not None:
            tail.append(f"waves_per_simd_achieved[{r.name}] = {r.waves_achieved:.3f}")
        for key, v in r.wave_states.items():
            tail.append(f"wave_state_{key}[{r.name}] = {v:.4f}")
        for key, v in r.latencies.items():
            tail.append(f"latency_{key}_cycles[{r.name}] = {v:.1f}")
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
    p.add_argument("--per-step", action="append", default=[], metavar="KERNEL=K",
                   help="KERNEL is dispatched K times per step: its window is K times wider")
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
    per_step = {k: int(v) for k, v in (x.rsplit("=", 1) for x in a.per_step)}
    rows = build_rows(a.trace, a.pmc, calib, agent, window, per_step)
    text = render(rows, a.title, a.command, calib, agent, window)
    if a.out:
        Path(a.out).write_text(text)
    else:
        sys.stdout.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
