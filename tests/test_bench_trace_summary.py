"""bench.py --trace-summary on a synthetic rocprofv3 kernel trace (CPU only): each configuration's
figures come from its kernel's first run of back-to-back dispatches (runs are cut at gaps above
2 ms), its last `steps` dispatches; a later, longer run of the same kernel (the default run's c2
power sample on zeroed operands) is not the configuration's timing; c5 M=1 and M=8 share a kernel
and take its runs in order; runs shorter than `steps` are dropped."""
import csv

import bench

C2 = "void tvk::gemm_dma_kernel<tvk::GemmCfg<signed char, 256, 256, 2, 4, 0, 1>, false>(tvk::GemmDesc, int, int, int, int)"
GEMV = "_ZN3tvk16gemv_mfma_kernelIDF16bLi4ELi2ELi8EEEvNS_8GemvArgsE"


def _write(path, runs):
    """runs: (kernel name, start ns, count, duration ns, gap ns between dispatches)."""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, t0, n, dur, gap in runs:
            for i in range(n):
                s = t0 + i * (dur + gap)
                w.writerow({"Kernel_Name": name, "Start_Timestamp": s, "End_Timestamp": s + dur})


def test_first_run_not_the_longest(tmp_path):
    p = tmp_path / "run_kernel_trace.csv"
    _write(p, [
        (C2, 0, 3, 60_000, 1_000),                 # a correctness call: shorter than steps, dropped
        (C2, 10_000_000, 45, 50_000, 1_000),       # c2's settle, warm-up and timed launches
        (GEMV, 40_000_000, 30, 18_000, 500),       # c5 M=1
        (GEMV, 50_000_000, 25, 20_000, 500),       # c5 M=8
        (C2, 90_000_000, 4000, 42_000, 500),       # the power sample on zeros: longer, later
    ])
    out = bench.trace_summary(str(p), 20)
    assert out["c2"]["avg_ns"] == 50_000 and out["c2"]["run_dispatches"] == 45
    assert out["c5m1"]["avg_ns"] == 18_000 and out["c5m1"]["run_dispatches"] == 30
    assert out["c5m8"]["avg_ns"] == 20_000 and out["c5m8"]["run_dispatches"] == 25
    assert all(v["dispatches"] == 20 for v in out.values())
