"""The rocprofv3 counter backend without a GPU: pass limits, the command line,
CSV parsing and the derived figures, on synthetic profiler output.

The CSV layouts are rocprofv3's (one row per dispatch and counter in
``*_counter_collection.csv``, one row per dispatch in ``*_kernel_trace.csv``).
The derived-figure checks use the counts a 2048x4096x4096 fp16 GEMM launch
recorded on MI355X: 67,108,864 MFMA busy cycles and 31,171,758 busy CU
cycles must give 53.8% MFMA utilisation, and 134,217,728 f16 MOPS must give
exactly the 2*M*N*K FLOPs.
"""

from __future__ import annotations

import csv

import pytest

from kernelforge.profiling import rocprof

COUNTER_HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id",
                  "Thread_Id", "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size",
                  "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count",
                  "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
TRACE_HEADER = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id",
                "Kernel_Id", "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp",
                "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count",
                "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X",
                "Grid_Size_Y", "Grid_Size_Z"]
GEMM = "void kf::(anonymous namespace)::gemm_direct_kernel<_Float16, 128, 256, 8, 0, 3>(kf::GemmArgs)"
FILL = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>>(int)"


def _counter_csv(path, rows):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(COUNTER_HEADER)
        for did, kernel, name, value in rows:
            w.writerow([did, did, "Agent 1", 1, 7, 7, 131072, 3, kernel, 512, 65536, 0, 128, 128,
                        40, name, f"{value:.6f}", 1000, 66000])


def test_passes_fit_one_hardware_pass():
    for name, counters in rocprof.PASSES.items():
        rocprof.check_pass(counters)  # every shipped pass is within the limits
    rocprof.check_pass(("FETCH_SIZE",))
    with pytest.raises(ValueError, match="TCC 5 > 4"):
        rocprof.check_pass(("FETCH_SIZE", "WRITE_SIZE"))
    with pytest.raises(ValueError, match="SQ 9 > 8"):
        rocprof.check_pass(tuple(f"SQ_X{i}" for i in range(9)))
    with pytest.raises(ValueError, match="GRBM 3 > 2"):
        rocprof.check_pass(("GRBM_COUNT", "GRBM_GUI_ACTIVE", "GRBM_GUI_ACTIVE_sum"))


def test_command_puts_the_program_right_after_the_separator():
    target = ["/usr/bin/python3", "-m", "kernelforge.cli.main", "profile", "matmul"]
    cmd = rocprof.build_command(target, counters=("FETCH_SIZE",), out_dir="/tmp/o", name="fetch")
    assert cmd[:3] == ["rocprofv3", "--pmc", "FETCH_SIZE"]
    assert cmd[cmd.index("--") + 1:] == target
    assert "--kernel-trace" not in cmd  # counters and tracing never share a run
    trace = rocprof.build_command(target, counters=(), out_dir="/tmp/o", name="trace")
    assert "--kernel-trace" in trace and "--pmc" not in trace
    assert rocprof.self_command(["env"])[1:3] == ["-m", "kernelforge.cli.main"]
    with pytest.raises(ValueError, match="exceeds"):
        rocprof.build_command(target, counters=("FETCH_SIZE", "WRITE_SIZE"), out_dir="o", name="x")


def test_counter_csv_groups_by_dispatch_and_picks_the_last_library_launch(tmp_path):
    path = tmp_path / "mfma_counter_collection.csv"
    rows = []
    for did, kernel in ((1, FILL), (2, GEMM), (3, FILL), (4, GEMM)):
        scale = 1.0 if did == 4 else 0.5
        rows += [(did, kernel, "SQ_BUSY_CU_CYCLES", 31_171_758 * scale),
                 (did, kernel, "SQ_VALU_MFMA_BUSY_CYCLES", 67_108_864 * scale),
                 (did, kernel, "SQ_INSTS_VALU_MFMA_MOPS_F16", 134_217_728 * scale)]
    _counter_csv(path, rows)
    dispatches = rocprof.parse_counter_csv(path)
    assert [d.dispatch_id for d in dispatches] == [1, 2, 3, 4]
    measured = rocprof.measured_dispatch(dispatches)
    assert measured.dispatch_id == 4 and measured.kernel == GEMM
    assert measured.counters["SQ_BUSY_CU_CYCLES"] == 31_171_758
    assert (measured.vgprs, measured.agprs, measured.lds_bytes) == (128, 128, 65536)

    launch = rocprof.LaunchCounters()
    launch.absorb(measured, timed=False)
    assert launch.duration_us is None  # counter runs never supply the duration
    assert launch.mfma_utilisation == pytest.approx(0.538, abs=5e-4)
    assert launch.mfma_flops == 2 * 2048 * 4096 * 4096
    assert rocprof.measured_dispatch([d for d in dispatches if d.kernel == FILL]) is None
    # The profiler reports the GEMM kernels by their mangled names.
    mangled = "_ZN2kf4gemm18gemm_direct_kernelIDF16_Li128ELi256ELi8ELi0ELi3EEEvNS0_4ArgsE"
    assert rocprof.is_library_kernel(mangled) and not rocprof.is_library_kernel(FILL)


def test_trace_csv_supplies_duration_and_launch_shape(tmp_path):
    path = tmp_path / "trace_kernel_trace.csv"
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(TRACE_HEADER)
        w.writerow(["KERNEL_DISPATCH", "Agent 1", 1, 0, 7, 9, 3, GEMM, 9, 5_000, 70_400, 65536, 0,
                    128, 128, 40, 512, 1, 1, 131072, 1, 1])
    (d,) = rocprof.parse_trace_csv(path)
    assert d.duration_us == pytest.approx(65.4) and d.grid == 131072 and d.workgroup == 512
    launch = rocprof.LaunchCounters()
    launch.absorb(d, timed=True)
    launch.counters["SQ_BUSY_CU_CYCLES"] = 31_171_758
    # 31,171,758 cycles over 256 CUs in 65.4 us: the 1.86 GHz shader clock.
    assert launch.shader_clock_ghz(256) == pytest.approx(1.862, abs=2e-3)


def test_vgpr_field_reads_half_the_gfx950_allocation():
    # .vgpr_count of this library's code objects against the VGPR_Count that
    # rocprofv3 recorded for the same kernels on an MI355X: (allocated, field).
    for allocated, field in ((223, 112), (256, 128), (56, 28), (79, 40)):
        assert rocprof.allocated_vgprs(field) == -(-allocated // 8) * 8
    launch = rocprof.LaunchCounters(kernel=GEMM, grid=131072, workgroup=512, vgprs=112)
    text = rocprof.RocprofRun([["rocprofv3"]], [0], launch).render(
        flops=1, algorithmic_bytes=1, peak_tflops=1, peak_gbps=1, cu_count=256, memory_bound=False)
    assert "224 / 0 / 0 B (VGPR_Count 112 x 2)" in text


def test_hbm_bytes_use_the_copy_calibration():
    launch = rocprof.LaunchCounters(counters={"FETCH_SIZE": 1024.0, "WRITE_SIZE": 2048.0})
    assert launch.hbm_bytes == (2.0 * 1024 + 1.0 * 2048) * 1024
    assert rocprof.LaunchCounters(counters={"FETCH_SIZE": 1.0}).hbm_bytes is None


def test_render_prices_against_the_peaks():
    launch = rocprof.LaunchCounters(kernel=GEMM, grid=131072, workgroup=512, duration_us=65.4,
                                    counters={"SQ_BUSY_CU_CYCLES": 31_171_758.0,
                                              "SQ_VALU_MFMA_BUSY_CYCLES": 67_108_864.0,
                                              "FETCH_SIZE": 52_000.0, "WRITE_SIZE": 16_384.0})
    run = rocprof.RocprofRun([["rocprofv3", "--kernel-trace"]], [0], launch)
    text = run.render(flops=68_719_476_736, algorithmic_bytes=67_108_864, peak_tflops=2516.6,
                      peak_gbps=8000.0, cu_count=256, memory_bound=False)
    assert run.ok
    assert "1050.8 TFLOP/s = 41.8% of peak" in text
    assert "MFMA busy" in text and "53.8%" in text and "1.86 GHz" in text
    assert "x algorithmic" in text and "bound: MFMA" in text
    empty = rocprof.RocprofRun([["rocprofv3"]], [1], None, "boom")
    assert not empty.ok and "no dispatch" in empty.render(
        flops=1, algorithmic_bytes=1, peak_tflops=1, peak_gbps=1, cu_count=1, memory_bound=True)


def test_unknown_pass_is_refused_before_anything_runs(monkeypatch, tmp_path):
    monkeypatch.setattr(rocprof, "rocprof_available", lambda: True)
    with pytest.raises(ValueError, match="unknown counter passes"):
        rocprof.run(["python"], out_dir=tmp_path, passes=("bogus",))


def test_profile_child_argv_keeps_the_shape_and_the_cache():
    from kernelforge.cli.main import build_parser, nsight_child_argv, profile_child_argv

    args = build_parser().parse_args(["profile", "matmul", "--backend", "rocprof", "-m", "512",
                                      "-n", "1024", "-k", "256", "--cache", "/tmp/kf.json"])
    child = profile_child_argv(args)
    assert child[:2] == ["profile", "matmul"]
    for flag, value in (("-m", "512"), ("-n", "1024"), ("-k", "256"), ("--cache", "/tmp/kf.json")):
        assert child[child.index(flag) + 1] == value
    assert child[-2:] == ["--backend", "launch-once"] and "--no-db" in child
    assert child.count("--backend") == 1
    assert nsight_child_argv is profile_child_argv
    args = build_parser().parse_args(["profile", "vector_add", "--elements", "99", "--no-cache"])
    child = profile_child_argv(args)
    assert child[child.index("--elements") + 1] == "99" and "--no-cache" in child


def test_nsight_backend_reports_unavailable(capsys):
    from kernelforge.cli.main import main

    assert main(["profile", "matmul", "--backend", "nsight"]) == 2
    assert "ncu not found" in capsys.readouterr().err


@pytest.mark.parametrize("dtype,peak", (("fp32", "157.3"), ("fp16", "2516.6")))
def test_profile_prices_each_dtype_against_its_own_mfma_peak(monkeypatch, capsys, dtype, peak):
    from kernelforge.cli.main import main

    launch = rocprof.LaunchCounters(kernel=GEMM, grid=131072, workgroup=512, duration_us=500.0)
    monkeypatch.setattr(rocprof, "rocprof_available", lambda: True)
    monkeypatch.setattr(rocprof, "run", lambda *a, **k: rocprof.RocprofRun([["rocprofv3"]], [0], launch))
    assert main(["profile", "matmul", "-m", "2048", "-n", "4096", "-k", "4096", "--dtype", dtype,
                 "--backend", "rocprof", "--no-cache"]) == 0
    # 68,719,476,736 FLOP in 500 us = 137.4 TFLOP/s.
    tflops = 68_719_476_736 / 500e-6 / 1e12
    assert f"{tflops:.1f} TFLOP/s = {100 * tflops / float(peak):.1f}% of peak" in capsys.readouterr().out


def _fake_passes(monkeypatch, results):
    """Make rocprof.run's passes return ``results[name] = (rc, log)`` and write a
    counter or trace file holding one GEMM dispatch, as rocprofv3 would."""
    monkeypatch.setattr(rocprof, "rocprof_available", lambda: True)

    def fake(command, timeout):
        out_dir = command[command.index("-d") + 1]
        name = command[command.index("-o") + 1]
        from pathlib import Path

        Path(out_dir).mkdir(parents=True, exist_ok=True)
        if "--pmc" in command:
            _counter_csv(Path(out_dir) / f"{name}_counter_collection.csv",
                         [(4, GEMM, c, 1000.0) for c in command[command.index("--pmc") + 1:
                                                               command.index("--output-format")]])
        else:
            with open(Path(out_dir) / f"{name}_kernel_trace.csv", "w", newline="") as fh:
                w = csv.writer(fh)
                w.writerow(TRACE_HEADER)
                w.writerow(["KERNEL_DISPATCH", "Agent 1", 1, 0, 7, 4, 3, GEMM, 4, 5_000, 70_400,
                            65536, 0, 128, 128, 40, 512, 1, 1, 131072, 1, 1])
        return results[name]

    monkeypatch.setattr(rocprof, "_run_pass", fake)


def test_a_profiler_segfault_after_a_finished_program_is_reported_not_hidden(monkeypatch, tmp_path):
    """rocprofv3 can end on SIGSEGV in its own teardown once the program it ran
    has exited and its files are written. Such a pass is used, and the run
    carries and prints what happened; the raw status is kept."""
    import signal

    segv = int(signal.SIGSEGV)
    _fake_passes(monkeypatch, {
        "trace": (0, f"...\n{rocprof.CHILD_DONE}\n"),
        "fetch": (-segv, f"...\n{rocprof.CHILD_DONE}\n"),
    })
    run = rocprof.run(["python"], out_dir=tmp_path, passes=("trace", "fetch"))
    assert run.ok and run.returncodes == [0, 0] and run.raw_returncodes == [0, -segv]
    assert len(run.notes) == 1 and "SIGSEGV" in run.notes[0] and "'fetch'" in run.notes[0]
    text = run.render(flops=1, algorithmic_bytes=1, peak_tflops=1, peak_gbps=1, cu_count=256,
                      memory_bound=False)
    assert "note: pass 'fetch': rocprofv3 exited on SIGSEGV" in text


@pytest.mark.parametrize("status", (-11, 139))
def test_a_profiler_segfault_before_the_program_finished_fails_the_profile(monkeypatch, tmp_path,
                                                                           status):
    """Without the child's completion line the same signal is a failure: the
    pass's status stands and the profile is not ok, whatever the files hold."""
    _fake_passes(monkeypatch, {"trace": (0, rocprof.CHILD_DONE), "mfma": (status, "partial")})
    run = rocprof.run(["python"], out_dir=tmp_path, passes=("trace", "mfma"))
    assert not run.ok and run.returncodes == [0, status]
    assert "before the profiled program finished" in run.notes[0]


def test_a_failed_pass_ends_the_profile_even_when_its_files_hold_the_launch(monkeypatch, tmp_path):
    """A pass whose status stands as a failure starts no further pass on the GPU,
    and its counters are not merged into the result."""
    ran = []
    _fake_passes(monkeypatch, {"trace": (0, rocprof.CHILD_DONE), "mfma": (-11, "partial"),
                               "fetch": (0, rocprof.CHILD_DONE)})
    inner = rocprof._run_pass
    monkeypatch.setattr(rocprof, "_run_pass", lambda c, t: (ran.append(c[c.index("-o") + 1]), inner(c, t))[1])
    run = rocprof.run(["python"], out_dir=tmp_path, passes=("trace", "mfma", "fetch"))
    assert ran == ["trace", "mfma"] and not run.ok and run.returncodes == [0, -11]
    assert run.launch is not None and not run.launch.counters


def test_the_launch_once_child_prints_the_completion_line_last():
    """The parent recognises a finished child by this line; it must be what
    _launch_once prints after its measured launch has synchronised."""
    import inspect

    from kernelforge.cli import main as cli

    src = inspect.getsource(cli._launch_once)
    assert src.index("torch.cuda.synchronize") < src.index("print(CHILD_DONE")
