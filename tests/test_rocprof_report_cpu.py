"""The rocprofv3 counter report (cuda_transformer_amd/rocprof_report.py) on synthetic CSVs whose
derived figures are known in closed form: MFMA utilisation, clock, executed FLOPs, HBM bytes
through the copy calibration, arithmetic intensity and LDS conflict rate."""
import csv

import pytest

from cuda_transformer_amd import rocprof_report as rr

PMC_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
              "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
              "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
              "Counter_Value", "Start_Timestamp", "End_Timestamp"]
AGENT = {"Agent_Type": "GPU", "Name": "gfx950", "Cu_Count": "256", "Simd_Count": "1024",
         "Num_Xcc": "8", "Max_Engine_Clk_Fcompute": "2400"}


def _pmc(d, name, rows):
    """rows: [(kernel, counter, value), ...] -> d/<name>_counter_collection.csv + agent info."""
    d.mkdir(parents=True, exist_ok=True)
    with open(d / f"{name}_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(PMC_HEADER)
        for i, (k, c, v) in enumerate(rows):
            # every dispatch lasts 2 ms (its timestamps), the span the clock is measured over
            w.writerow([i, i, "Agent 1", 1, 1, 1, 1024, 7, k, 256, 4096, 0, 128, 0, 32, c, v,
                        10_000_000 * i, 10_000_000 * i + 2_000_000])
    with open(d / f"{name}_agent_info.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(AGENT))
        w.writeheader()
        w.writerow({**AGENT, "Agent_Type": "CPU", "Name": "host"})
        w.writerow(AGENT)
    return d


def _trace(d, kernels):
    d.mkdir(parents=True, exist_ok=True)
    with open(d / "t_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                    "StdDev"])
        for k, calls, avg in kernels:
            w.writerow([k, calls, calls * avg, avg, 50.0, avg, avg, 0])
    return d


def test_derived_figures(tmp_path):
    ms = 2.0
    xcds, simds, clock = 8, 1024, 2.25e9
    cycles = clock * ms * 1e-3                       # per XCD
    mops = 4.0e8                                     # -> 2.048e11 FLOP
    busy = 0.75 * cycles * simds
    trace = _trace(tmp_path / "trace", [("k_mfma", 3, ms * 1e6), ("k_copyish", 3, 1e6)])
    mf = _pmc(tmp_path / "mfma", "m", [
        ("k_mfma", "GRBM_GUI_ACTIVE", cycles * xcds), ("k_mfma", "GRBM_GUI_ACTIVE", cycles * xcds),
        ("k_mfma", "SQ_VALU_MFMA_BUSY_CYCLES", busy), ("k_mfma", "SQ_INSTS_VALU_MFMA_MOPS_F32", mops),
        ("k_mfma", "SQ_LDS_BANK_CONFLICT", 5.0), ("k_mfma", "SQ_LDS_IDX_ACTIVE", 100.0)])
    fe = _pmc(tmp_path / "fetch", "f", [("k_mfma", "FETCH_SIZE", 1000.0), ("k_copyish", "FETCH_SIZE", 10.0)])
    wr = _pmc(tmp_path / "write", "w", [("k_mfma", "WRITE_SIZE", 500.0), ("k_copyish", "WRITE_SIZE", 10.0)])
    cf = _pmc(tmp_path / "cf", "c", [("__amd_rocclr_copyBuffer", "FETCH_SIZE", 512.0)])
    cw = _pmc(tmp_path / "cw", "c", [("__amd_rocclr_copyBuffer", "WRITE_SIZE", 1024.0)])
    calib = rr.calibration(cf, cw, 1 << 20)          # 1024 KiB moved each way
    assert calib[0] == pytest.approx(2.0) and calib[1] == pytest.approx(1.0)
    agent = rr.read_agent(mf)
    assert agent["xcds"] == 8 and agent["simds"] == 1024
    rows = {r.name: r for r in rr.build_rows(trace, [mf, fe, wr], calib, agent)}
    r = rows["k_mfma"]
    assert r.calls == 3 and r.avg_ms == pytest.approx(ms)
    assert r.mfma_flop == pytest.approx(mops * 512)
    assert r.tflops == pytest.approx(mops * 512 / (ms * 1e-3) / 1e12)
    assert r.mfma_util == pytest.approx(0.75)
    assert r.clock_ghz == pytest.approx(2.25)
    assert r.hbm_bytes == pytest.approx(1024 * (1000 * 2.0 + 500 * 1.0))
    assert r.intensity == pytest.approx(r.mfma_flop / r.hbm_bytes)
    assert r.lds_conflict_rate == pytest.approx(0.05)
    assert rows["k_copyish"].mfma_flop is None and rows["k_copyish"].mfma_util is None

    text = rr.render(list(rows.values()), "T", ["cmd"], calib, agent)
    assert "traffic_bytes_per_launch[k_mfma] = 2.560000e+06" in text
    assert "mfma_util[k_mfma] = 0.7500" in text
    assert "| k_mfma | 3 | 2.0000 |" in text


def test_cli_writes_report(tmp_path):
    trace = _trace(tmp_path / "trace", [("k", 1, 1e6)])
    pmc = _pmc(tmp_path / "p", "p", [("k", "SQ_INSTS_VALU_MFMA_MOPS_F32", 1.0)])
    out = tmp_path / "r.md"
    assert rr.main(["--title", "X", "--trace", str(trace), "--pmc", str(pmc), "--out", str(out),
                    "--command", "rocprofv3 ..."]) == 0
    text = out.read_text()
    assert text.startswith("# X") and "mfma_flop_per_launch[k] = 5.120000e+02" in text


def test_missing_inputs_raise(tmp_path):
    with pytest.raises(FileNotFoundError):
        rr.read_kernel_stats(tmp_path)
    no_copy = _pmc(tmp_path / "n", "n", [("k", "FETCH_SIZE", 1.0)])
    with pytest.raises(ValueError):
        rr.calibration(no_copy, no_copy, 1024)


def test_trace_window(tmp_path):
    d = tmp_path / "tr"
    d.mkdir()
    with open(d / "x_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        # dispatches of k in launch order: 9, 1, 2, 3, 9 (ms); written out of order
        for i, dur in reversed(list(enumerate([9, 1, 2, 3, 9]))):
            w.writerow(["k", i * 100_000_000, i * 100_000_000 + dur * 1_000_000])
    with open(d / "x_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs",
                    "StdDev"])
        w.writerow(["k", 5, 24e6, 4.8e6, 100.0, 1e6, 9e6, 0])
    win = rr.read_trace_window(d, 1, 3)
    assert win["k"]["calls"] == 3 and win["k"]["avg_ns"] == pytest.approx(2e6)
    # two dispatches a step: step 1 is dispatches 2..3 (2, 3 ms)
    win2 = rr.read_trace_window(d, 1, 1, {"k": 2})
    assert win2["k"]["calls"] == 2 and win2["k"]["avg_ns"] == pytest.approx(2.5e6)
    assert win["k"]["all_calls"] == 5 and win["k"]["all_avg_ns"] == pytest.approx(4.8e6)
    (row,) = rr.build_rows(d, window=(1, 3))
    assert row.avg_ms == pytest.approx(2.0) and row.calls == 3
    text = rr.render([row], "T", window=(1, 3))
    assert "dispatches 1..3" in text and "| k | 5 | 4.8000 |" in text


def test_short_name_of_mangled_kernels():
    """rocprofv3 leaves kernels over __bf16 mangled; the report shortens them like the rest."""
    from cuda_transformer_amd.rocprof_report import short_name

    mangled = ("_ZN3cta12_GLOBAL__N_119fa2_fwd_bf16_kernelILi64ELb0EEEvPKDF16bS3_S3_PDF16bPfiiii"
               "NS0_11RowStridesBES6_S6_fff")
    assert short_name(mangled) == "fa2_fwd_bf16_kernel<64, false>"
    dkdv = ("_ZN3cta12_GLOBAL__N_124fa2_bwd_dkdv_half_kernelIDF16bLi64ELb1ELi8ELi64ELi2ELb0EEEv"
            "PKT_S4_S4_S4_PKfS6_PS2_S7_S7_iiiiiNS0_11RowStridesHES8_S8_S8_S8_ff")
    assert short_name(dkdv) == "fa2_bwd_dkdv_half_kernel<bf16, 64, true, 8, 64, 2, false>"
    f16 = "_ZN3cta12_GLOBAL__N_122fa2_bwd_dq_half_kernelIDF16_Li32ELb0EEEvPKT_"
    assert short_name(f16) == "fa2_bwd_dq_half_kernel<f16, 32, false>"
    # an argument it cannot decode leaves the bare identifier
    assert short_name("_ZN3cta1kINS_3FooEEEvv") == "k"
    assert short_name("_Z6foobarv") == "foobar"
    assert short_name("fa2_fwd_kernel") == "fa2_fwd_kernel"
    assert short_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
    demangled = ("void cta::(anonymous namespace)::gemm_kernel<cta::(anonymous namespace)::"
                 "GemmTile<128, 64, 16, 2, 2>, 0, 0, 0>(cta::GemmOperand, float*)")
    assert short_name(demangled) == "gemm_kernel<GemmTile<128, 64, 16, 2, 2>, 0, 0, 0>"
    assert short_name("cta::(anonymous namespace)::gelu_fwd_kernel(float const*, long)") == \
        "gelu_fwd_kernel"


def test_theoretical_occupancy():
    """gfx950: 512 unified VGPR+AGPR entries per lane, granule 8; 160 KiB LDS per CU; 8 slots."""
    assert rr.theoretical_waves(256, 0, 0, 256) == (2, "vgpr")
    assert rr.theoretical_waves(250, 0, 0, 256) == (2, "vgpr")      # 250 -> 256 allocated
    assert rr.theoretical_waves(168, 0, 0, 256) == (3, "vgpr")
    assert rr.theoretical_waves(128, 0, 0, 256) == (4, "vgpr")
    assert rr.theoretical_waves(80, 48, 0, 256) == (4, "vgpr")       # 80 + 48 = 128 entries
    assert rr.theoretical_waves(32, 0, 0, 64) == (8, "slots")
    # 36 KiB of LDS per 4-wave workgroup: 4 workgroups per CU -> 4 waves per SIMD
    assert rr.theoretical_waves(64, 0, 36 * 1024, 256) == (4, "lds")
    # 64 KiB per 8-wave workgroup: 2 workgroups per CU -> 16 waves over 4 SIMDs = 4
    assert rr.theoretical_waves(40, 0, 64 * 1024, 512) == (4, "lds")


def test_wave_states_and_achieved_occupancy(tmp_path):
    xcds, simds, cycles = 8, 1024, 1.0e6               # cycles per XCD
    wave_quads = 2.5 * cycles * simds / 4              # 2.5 waves resident per SIMD on average
    rows = [("k", "GRBM_GUI_ACTIVE", cycles * xcds), ("k", "SQ_WAVE_CYCLES", wave_quads),
            ("k", "SQ_ACTIVE_INST_ANY", 0.4 * wave_quads), ("k", "SQ_WAIT_ANY", 0.3 * wave_quads),
            ("k", "SQ_WAIT_INST_ANY", 0.2 * wave_quads), ("k", "SQ_ACTIVE_INST_VALU", 0.25 * wave_quads),
            ("k", "SQ_INSTS_VALU_MFMA_MOPS_BF16", 10.0), ("k", "SQ_INSTS_VALU_MFMA_MOPS_F32", 1.0)]
    d = _pmc(tmp_path / "ws", "w", rows)
    (r,) = rr.build_rows(None, [d], None, rr.read_agent(d))
    assert r.waves_achieved == pytest.approx(2.5)
    assert r.wave_states["issue"] == pytest.approx(0.4)
    assert r.wave_states["dep_wait"] == pytest.approx(0.3)
    assert r.wave_states["issue_wait"] == pytest.approx(0.2)
    assert r.wave_states["valu"] == pytest.approx(0.25)
    assert "lds" not in r.wave_states
    assert r.mfma_flop == pytest.approx(11.0 * 512)
    # registers from the dispatch (VGPR_Count 128 = 256 allocated, LDS 4096 B, 256 threads)
    assert (r.info["vgpr"], r.info["agpr"], r.info["sgpr"]) == (256, 0, 32)
    assert (r.waves_theory, r.waves_limit) == (2, "vgpr")
    text = rr.render([r], "T", agent=rr.read_agent(d))
    assert "| k | 256 | 0 | 32 | 2 (vgpr) | 2.50 | 40.0% | 30.0% | 20.0% | - | 25.0% |" in text
    assert "waves_per_simd_achieved[k] = 2.500" in text and "wave_state_dep_wait[k] = 0.3000" in text


def test_registers_from_kernel_trace(tmp_path):
    d = tmp_path / "kt"
    d.mkdir()
    cols = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
            "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size",
            "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X",
            "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
    with open(d / "x_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        w.writerow(["KERNEL_DISPATCH", "Agent 1", 1, 0, 1, 1, 3, "kern", 1, 0, 2_000_000, 36864,
                    20, 128, 0, 96, 256, 1, 1, 4096, 1, 1])
    with open(d / "x_kernel_stats.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs",
                    "MaxNs", "StdDev"])
        w.writerow(["kern", 1, 2e6, 2e6, 100.0, 2e6, 2e6, 0])
    (r,) = rr.build_rows(d)
    assert r.info["vgpr"] == 256 and r.info["scratch"] == 20 and r.info["workgroup"] == 256
    assert (r.waves_theory, r.waves_limit) == (2, "vgpr")


def test_trace_window_per_step_matches_exact_names(tmp_path):
    """A per-step multiplier applies to the kernel it names (short name or base identifier),
    not to another kernel whose name contains it."""
    from cuda_transformer_amd import rocprof_report as rr

    d = tmp_path / "trace"
    d.mkdir()
    rows = [("fa2_bwd_dq_kernel", 0), ("fa2_bwd_dq_ds_kernel<64, true>", 0),
            ("fa2_bwd_dq_ds_kernel<64, true>", 0)] * 4
    with open(d / "run_kernel_trace.csv", "w") as f:
        f.write("Kernel_Name,Start_Timestamp,End_Timestamp\n")
        for t, (k, _) in enumerate(rows):
            f.write(f'"{k}",{10 * t},{10 * t + 1 + t}\n')
    win = rr.read_trace_window(d, 1, 2, {"fa2_bwd_dq_ds_kernel": 2})
    assert win["fa2_bwd_dq_kernel"]["calls"] == 2          # not widened by the ds multiplier
    assert win["fa2_bwd_dq_ds_kernel<64, true>"]["calls"] == 4
    win = rr.read_trace_window(d, 1, 2, {"fa2_bwd_dq": 2})  # a substring names nothing
    assert win["fa2_bwd_dq_kernel"]["calls"] == 2 and win["fa2_bwd_dq_ds_kernel<64, true>"]["calls"] == 2


def test_latency_metrics_are_reported(tmp_path):
    """rocprofv3's derived VmemLatency / LdsLatency / InstrFetchLatency (cycles), each from its
    own --pmc pass, land in the latency table and the machine-readable tail as collected."""
    lat_v = _pmc(tmp_path / "v", "v", [("k", "VmemLatency", 570.0), ("k", "VmemLatency", 590.0)])
    lat_l = _pmc(tmp_path / "l", "l", [("k", "LdsLatency", 49.0)])
    lat_i = _pmc(tmp_path / "i", "i", [("k", "InstrFetchLatency", 30.0), ("j", "InstrFetchLatency", 7.0)])
    rows = rr.build_rows(pmc=[lat_v, lat_l, lat_i])
    by = {r.name: r for r in rows}
    assert by["k"].latencies == {"vmem": 580.0, "lds": 49.0, "ifetch": 30.0}
    assert by["j"].latencies == {"ifetch": 7.0}
    text = rr.render(rows, "T")
    assert "| k | 580 | 49 | 30 |" in text and "| j | - | - | 7 |" in text
    assert "latency_vmem_cycles[k] = 580.0" in text
