#!/usr/bin/env python3
"""Benchmark of the MI355X HIP backend for Tensorvia's ops::Mul (matmul) path.

One "step" is one ops::Mul call (one kernel launch) on device-resident, seeded synthetic inputs.
The JSON line's ``value`` is configuration c2 (int8 A[4096,4096] @ B[4096,4096] -> int8 wrap):
BASELINE.json's configs[1], the config the bench contract quotes at N=1 (configs[0], c1, is the
reference's README shape, which its own CPU backend runs).  The other configurations are measured
in the same run and reported under ``configs``, each with its own CPU baseline.

Timing: 40 ms of untimed launches of the configuration's own kernel (the GPU's clocks settle to
the load), W untimed launches, then K back-to-back launches in 5 runs, with HIP events on the launch
stream at the run boundaries: the mean over all K is the per-launch time the line reports and the
roofline uses; the median of the 5 runs' per-launch means is reported beside it.  The CPU baseline
is the oracle's restatement of MulImpl<CPU> (src/backend/cpu/mul.cpp:97-145) on the box's host
cores, timed with a steady clock per call as the reference's tests/mul.cpp:17-29 does, on a bounded
sample of each workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,...] [--no-cpu]
                       [--only c2]   (only that config's kernel, e.g. under rocprofv3)
                       [--vendor]    (also time torch's own library GEMM on the same inputs)
       python bench.py --trace-summary kernel_trace.csv --steps K
                       (per-configuration kernel durations of a rocprofv3 trace of this bench)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

# MI355X datasheet peaks (2.4 GHz engine clock, 256 CUs): dense matrix-core rates and HBM3E.
PEAK = {"fp32": 157.3, "bf16": 2516.6, "fp16": 2516.6, "int8": 5033.2}  # TFLOP/s (TOP/s for int8)
PEAK_HBM_GBS = 8000.0

METRIC = "ops::matmul TFLOP/s (% MFMA peak) per dtype; GEMV HBM GB/s (% peak)"

# Kernel trace of `bench.py --steps 20 --warmup 5` under rocprofv3 --kernel-trace --stats on this
# build (profiles/bench_kernel_trace.md): per-kernel average and median durations.
TRACE_FILE = ROOT / "profiles" / "bench_kernel_trace.json"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_inputs(name: str):
    """Seeded host storage arrays for configuration ``name``."""
    from tensorvia_amd import rng
    if name == "c1":
        return dict(a=rng.make("uniform", (2592, 2048), 1, "float32"),
                    b=rng.make("uniform", (2048, 4096), 2, "float32"), dt=6)
    if name == "c2":
        return dict(a=rng.make("uniform", (4096, 4096), 3, "int8", lo=-10, hi=10),
                    b=rng.make("uniform", (4096, 4096), 4, "int8", lo=-10, hi=10), dt=0)
    if name == "c3":
        return dict(a=rng.make("uniform", (16, 2048, 4096), 5, "bfloat16"),
                    b=rng.make("uniform", (4096, 4096), 6, "bfloat16"), dt=4)
    if name == "bf16_4096":
        return dict(a=rng.make("uniform", (4096, 4096), 13, "bfloat16"),
                    b=rng.make("uniform", (4096, 4096), 14, "bfloat16"), dt=4)
    if name == "c4":
        q = rng.normal_f32(7, 32 * 2048 * 128) / np.float32(np.sqrt(128.0))
        k = rng.normal_f32(8, 32 * 2048 * 128) / np.float32(np.sqrt(128.0))
        return dict(a=rng.f32_to_f16_bits(q).reshape(32, 2048, 128), b=rng.f32_to_f16_bits(k).reshape(32, 2048, 128), dt=5)
    if name == "c3_fused":
        d = make_inputs("c3")
        d["bias"] = rng.make("uniform", (4096,), 12, "bfloat16", lo=-1, hi=1)
        return d
    if name in ("c5m1", "c5m8"):
        m = 1 if name == "c5m1" else 8
        return dict(a=rng.make("normal", (m, 4096), 9 if m == 1 else 11, "bfloat16"),
                    b=rng.make("uniform", (4096, 11008), 10, "bfloat16", lo=-0.05, hi=0.05), dt=4)
    raise ValueError(name)


DESC = {
    "c1": "fp32 A[2592,2048] @ B[2048,4096] -> fp32 (README benchmark shape)",
    "c2": "int8 A[4096,4096] @ B[4096,4096] -> int8 (low byte of the int32 sum)",
    "c3": "bf16 A[16,2048,4096] @ B[4096,4096] (B broadcast over batch) -> bf16, fp32 accumulate",
    "c3_fused": "c3 with the fused epilogue: silu(A @ B + bias[4096]) -> bf16 (tv_hip_gemm_ex)",
    "bf16_4096": "bf16 A[4096,4096] @ B[4096,4096] -> bf16, fp32 accumulate (the bf16 4096^3 shape of the targets)",
    "c4": "fp16 Q[32,2048,128] @ K.permute(0,2,1) (strided view, no repack) -> fp16 [32,2048,2048]",
    "c5m1": "bf16 GEMV x[1,4096] @ W[4096,11008] -> bf16, fp32 accumulate (6 W replicas rotated)",
    "c5m8": "bf16 GEMV x[8,4096] @ W[4096,11008] -> bf16, fp32 accumulate (6 W replicas rotated)",
}
DTYPE = {"c1": "fp32", "c2": "int8", "c3": "bf16", "c3_fused": "bf16", "bf16_4096": "bf16", "c4": "fp16", "c5m1": "bf16",
         "c5m8": "bf16"}
# The kernel each configuration's launch runs.
KERNEL = {
    "c1": "gemm_mfma_sk_kernel<GemmCfg<float, 96, 128, 2, 2, 0, 1>, false> (stream-K schedule)",
    "c2": "gemm_dma_kernel<GemmCfg<signed char, 256, 256, 2, 4, 0, 1>, false>",
    "c3": "gemm_dma_chain_kernel<GemmCfg<__bf16, 256, 256, 2, 4, 0, 1>> (chained tiles)",
    "c3_fused": "gemm_dma_kernel<GemmCfg<__bf16, 256, 256, 2, 4, 0, 1>, true>",
    "bf16_4096": "gemm_dma_kernel<GemmCfg<__bf16, 256, 256, 2, 4, 0, 1>, false>",
    "c4": "gemm_smallk_pipe_kernel<GemmCfg<_Float16, 128, 128, 2, 4, 0, 0>, _Float16> (row-synchronous groups)",
    "c5m1": "gemv_mfma_kernel<__bf16, 4, 2, 8>",
    "c5m8": "gemv_mfma_kernel<__bf16, 4, 2, 8>",
}
# The same kernels as they appear in a rocprofv3 kernel trace (demangled, or mangled where the
# profiler's demangler gives up on __bf16 / _Float16 template arguments).
TRACE_KERNEL = {
    "c1": r"gemm_mfma_sk_kernel.*(GemmCfg<float, 96, 128|GemmCfgIfLi96ELi128E)",
    "c2": r"gemm_dma_kernel.*(GemmCfg<signed char, 256, 256|GemmCfgIaLi256ELi256E)",
    "c3": r"gemm_dma_chain_kernel.*(GemmCfg<__bf16|GemmCfgIDF16b)",
    "c3_fused": r"gemm_dma_kernel.*(GemmCfg<__bf16|GemmCfgIDF16b).*(true|Lb1E)",
    "bf16_4096": r"gemm_dma_kernel.*(GemmCfg<__bf16|GemmCfgIDF16b).*(false|Lb0E)",
    "c4": r"gemm_smallk_pipe_kernel.*(GemmCfg<_Float16|GemmCfgIDF16_)",
    "c5m1": r"gemv_mfma_kernel.*(__bf16|DF16b)",
    "c5m8": r"gemv_mfma_kernel.*(__bf16|DF16b)",
    "cast_c3a": r"cast_kernel", "random_c3a": r"random_kernel", "fill_c3a": r"fill_kernel",
    "transpose_c4k": r"repack_transpose16_kernel",
}
# Bound each configuration is judged against (c4's arithmetic intensity, 113.8 FLOP/B, is below
# the fp16 ridge of about 315: HBM-bound).
BOUND = {"c1": "mfma", "c2": "mfma", "c3": "mfma", "c3_fused": "mfma", "bf16_4096": "mfma", "c4": "hbm", "c5m1": "hbm",
         "c5m8": "hbm"}


def work(name: str, inp) -> tuple[float, float]:
    """(algorithmic flops/ops, algorithmic HBM bytes) per call: each operand read once, C written once."""
    a, b = inp["a"], inp["b"]
    es = a.itemsize
    if name == "c4":
        B, M, K = a.shape
        N = b.shape[1]
        return 2.0 * B * M * N * K, (a.size + b.size) * es + B * M * N * es
    if a.ndim == 3:
        B, M, K = a.shape
    else:
        B, (M, K) = 1, a.shape
    N = b.shape[-1]
    return 2.0 * B * M * N * K, (a.size + b.size) * es + B * M * N * es


# Untimed running time of each configuration's own launches before its W warm-up launches.  The
# GPU's clocks follow the load: on MI355X, c1's first blocks of 20 launches ran 428, 386, 366 and
# then 350 us (about 25 ms to settle, fresh or reused buffers alike), and a global warm-up with
# another kernel did not settle them for the next one.
SETTLE_S = 0.04


def timed_launches(launch, steps: int, warmup: int, stream, groups: int = 5):
    """SETTLE_S of untimed launches and W untimed launches, then K back-to-back launches in `groups`
    runs of consecutive launches, with a HIP event on the launch stream at each run boundary.
    Returns the mean per-launch time over the whole timed region, the median over the runs of
    their per-launch means, and the host wall time per step."""
    import torch
    t_settle = time.perf_counter()
    n = 0
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(4):
            launch(n)
            n += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        launch(n + i)
    torch.cuda.synchronize()
    groups = max(1, min(groups, steps))
    bounds = [round(g * steps / groups) for g in range(groups + 1)]
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    t0 = time.perf_counter()
    evs[0].record(stream)
    for g in range(groups):
        for i in range(bounds[g], bounds[g + 1]):
            launch(i)
        evs[g + 1].record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    mean_ms = evs[0].elapsed_time(evs[-1]) / steps
    median_ms = float(np.median([evs[g].elapsed_time(evs[g + 1]) / (bounds[g + 1] - bounds[g]) for g in range(groups)]))
    return mean_ms, median_ms, wall_ms


def rates(res: dict, name: str) -> dict:
    ms = res["kernel_ms_mean"]
    res["tflops"] = res["flops"] / (ms * 1e-3) / 1e12
    res["tflops_frac_peak"] = res["tflops"] / PEAK[DTYPE[name]]
    res["hbm_gbs"] = res["algorithmic_bytes"] / (ms * 1e-3) / 1e9
    res["hbm_frac_peak"] = res["hbm_gbs"] / PEAK_HBM_GBS
    res["roofline_frac"] = res["tflops_frac_peak"] if BOUND[name] == "mfma" else res["hbm_frac_peak"]
    return res


def run_gpu(name: str, steps: int, warmup: int):
    import torch

    import tensorvia_amd as tv
    from tensorvia_amd.matmul import storage_to_torch as to_torch

    inp = make_inputs(name)
    dt = inp["dt"]
    a = to_torch(inp["a"], dt)
    if name == "c4":
        b = to_torch(inp["b"], dt).permute(0, 2, 1)  # strided view
    else:
        b = to_torch(inp["b"], dt)
    reps = [b]
    if name.startswith("c5"):
        # W is 90 MB and the MALL (Infinity Cache) is 256 MB: rotate 6 replicas (540 MB) so every
        # call streams W from HBM.
        reps = [b] + [b.clone() for _ in range(5)]
    out = tv.gemm(a, b)  # allocates the output (and any workspace) outside the timed region
    torch.cuda.synchronize()
    # Descriptors are packed once: a step is one C-ABI call, so the host enqueues launches faster
    # than the GPU retires them and the events bracket back-to-back kernels.
    L = tv.lib()
    descs = [tv.make_args(a, r, out) for r in reps]
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    ep = None
    if "bias" in inp:
        bias = to_torch(inp["bias"], dt)
        ep = tv.TvEpilogue()
        ep.act, ep.bias, ep.sbias_b, ep.sbias_m, ep.sbias_n = tv.ACT_SILU, bias.data_ptr(), 0, 0, 1

    def launch(i):
        if ep is None:
            rc = L.tv_hip_gemm(ctypes.byref(descs[i % len(descs)]), sh)
        else:
            rc = L.tv_hip_gemm_ex(ctypes.byref(descs[i % len(descs)]), ctypes.byref(ep), sh)
        if rc:
            tv.check(rc)

    mean_ms, median_ms, wall_ms = timed_launches(launch, steps, warmup, stream)
    flops, bytes_ = work(name, inp)
    res = {"workload": DESC[name], "dtype": DTYPE[name], "bound": BOUND[name], "kernel": KERNEL[name],
           "kernel_ms_mean": float(mean_ms), "kernel_ms_median_of_runs": median_ms, "ms_per_step": wall_ms,
           "flops": flops, "algorithmic_bytes": bytes_}
    rates(res, name)
    del a, b, reps, out
    torch.cuda.empty_cache()
    return res, inp


def run_vendor(name: str, inp, steps: int, warmup: int) -> dict:
    """The same configuration through torch's own GEMM (hipBLASLt / rocBLAS on ROCm), for comparison.

    Differences from the measured path: c2 uses torch._int_mm (int32 output: the library has no
    int8-output int8 GEMM); c4 multiplies by a materialised K^T (batched half products on a
    transposed right operand are avoided on this platform)."""
    import torch

    from tensorvia_amd.matmul import storage_to_torch as to_torch
    dt = inp["dt"]
    a = to_torch(inp["a"], dt)
    b = to_torch(inp["b"], dt)
    note = "torch.matmul"
    if name == "c2":
        fn = lambda i: torch._int_mm(a, b)  # noqa: E731
        note = "torch._int_mm (int32 output)"
    elif name == "c4":
        bt = b.permute(0, 2, 1).contiguous()
        fn = lambda i: torch.bmm(a, bt)  # noqa: E731
        note = "torch.bmm with K^T materialised"
    elif "bias" in inp:
        bias = to_torch(inp["bias"], dt)
        fn = lambda i: torch.nn.functional.silu(torch.matmul(a, b) + bias)  # noqa: E731
        note = "torch.nn.functional.silu(torch.matmul(a, b) + bias) (three kernels)"
    else:
        reps = [b] + ([b.clone() for _ in range(5)] if name.startswith("c5") else [])
        fn = lambda i: torch.matmul(a, reps[i % len(reps)])  # noqa: E731
        if name.startswith("c5"):
            note = "torch.matmul, 6 W replicas rotated"
    mean_ms, median_ms, _ = timed_launches(fn, steps, warmup, torch.cuda.current_stream())
    flops, bytes_ = work(name, inp)
    res = {"call": note, "ms_mean": mean_ms, "ms_median_of_runs": median_ms, "tflops": flops / (mean_ms * 1e-3) / 1e12,
           "tflops_frac_peak": flops / (mean_ms * 1e-3) / 1e12 / PEAK[DTYPE[name]],
           "hbm_gbs": bytes_ / (mean_ms * 1e-3) / 1e9}
    torch.cuda.empty_cache()
    return res


# Element-wise device ops of the backend, on the c3 A operand's shape (134,217,728 elements).
EW = {
    "cast_c3a": "typecast bf16 -> fp32 of [16,2048,4096] (the CPU backend's widening of c3's A; 2 sources in turn)",
    "random_c3a": "seeded uniform bf16 [16,2048,4096] (ops::Random on the device)",
    "fill_c3a": "fill fp32 [16,2048,4096] with 1.0 (ops::Ones on the device)",
    "transpose_c4k": "ops::Transpose(K, {0,2,1}) materialised: fp16 [32,2048,128] -> [32,128,2048] (tv_hip_repack)",
}


def run_ew(name: str, steps: int, warmup: int) -> dict:
    """HBM-bound element-wise kernels: algorithmic bytes = elements read once + written once."""
    import torch

    import tensorvia_amd as tv
    L = tv.lib()
    n = 16 * 2048 * 4096
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    if name == "cast_c3a":
        # Two sources (2 x 268 MB) taken in turn, so that no call finds its source in the 256 MB
        # MALL (Infinity Cache) from the call before.
        srcs = [torch.empty(n, dtype=torch.int16, device="cuda") for _ in range(2)]  # bf16 storage
        for s_ in srcs:
            tv.check(L.tv_hip_random(ctypes.c_void_p(s_.data_ptr()), tv.BFLOAT16, n, -1.0, 1.0, 5, sh))
        dst = torch.empty(n, dtype=torch.float32, device="cuda")

        def call(i):
            return L.tv_hip_typecast(ctypes.c_void_p(srcs[i & 1].data_ptr()), tv.BFLOAT16,
                                     ctypes.c_void_p(dst.data_ptr()), tv.FLOAT32, n, sh)
        nbytes = n * 2 + n * 4
    elif name == "random_c3a":
        dst = torch.empty(n, dtype=torch.int16, device="cuda")
        call = lambda i: L.tv_hip_random(ctypes.c_void_p(dst.data_ptr()), tv.BFLOAT16, n, -1.0, 1.0, 5, sh)  # noqa: E731
        nbytes = n * 2
    elif name == "transpose_c4k":
        m = 32 * 2048 * 128
        src = torch.empty(m, dtype=torch.int16, device="cuda")  # K, fp16 storage
        tv.check(L.tv_hip_random(ctypes.c_void_p(src.data_ptr()), tv.FLOAT16, m, -1.0, 1.0, 8, sh))
        dst = torch.empty(m, dtype=torch.int16, device="cuda")
        a = tv.TvRepackArgs()
        a.ndim, a.elem_size = 3, 2
        for d, (ext, st) in enumerate(zip((32, 128, 2048), (2048 * 128, 1, 128))):
            a.shape[d], a.strides[d] = ext, st
        a.src, a.dst = src.data_ptr(), dst.data_ptr()
        call = lambda i: L.tv_hip_repack(ctypes.byref(a), sh)  # noqa: E731
        nbytes = m * 2 * 2
    else:
        dst = torch.empty(n, dtype=torch.float32, device="cuda")
        call = lambda i: L.tv_hip_fill(ctypes.c_void_p(dst.data_ptr()), tv.FLOAT32, n, 1.0, sh)  # noqa: E731
        nbytes = n * 4
    tv.check(call(0))

    def launch(i):
        rc = call(i)
        if rc:
            tv.check(rc)

    mean_ms, median_ms, _ = timed_launches(launch, steps, warmup, stream)
    res = {"workload": EW[name], "bound": "hbm", "kernel_ms_mean": mean_ms, "kernel_ms_median_of_runs": median_ms,
           "algorithmic_bytes": nbytes, "hbm_gbs": nbytes / (mean_ms * 1e-3) / 1e9}
    res["hbm_frac_peak"] = res["hbm_gbs"] / PEAK_HBM_GBS
    res["roofline_frac"] = res["hbm_frac_peak"]
    del dst
    torch.cuda.empty_cache()
    return res


def run_copy(steps: int, warmup: int) -> dict:
    """Calibration for the HBM traffic counters: a plain device copy of a known size (512 MiB read,
    512 MiB written per launch; larger than the 256 MB MALL)."""
    import torch
    n = 512 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    mean_ms, median_ms, _ = timed_launches(lambda i: dst.copy_(src), steps, warmup, torch.cuda.current_stream())
    return {"workload": "device copy of 512 MiB (uint8)", "bytes_read": n, "bytes_written": n,
            "kernel_ms_mean": mean_ms, "hbm_gbs": 2 * n / (mean_ms * 1e-3) / 1e9}


# CPU baseline per configuration: calls timed and the sample of the workload they run.  c3 runs
# once, as the equivalent flattened 2-d call [32768,4096] @ [4096,4096] (the reference rejects the
# broadcast form, src/ops.cpp:544-550; about 17 s on 16 threads); c4 multiplies by a
# pre-materialised K^T (the CPU kernel ignores strides), whose transpose is timed apart.
CPU_PLAN = {"c1": (3, None), "c2": (3, None), "c3": (1, None), "bf16_4096": (3, None), "c4": (3, None), "c5m1": (10, None),
            "c5m8": (10, None)}


def cpu_effective_threads(threads: int, batch: int, M: int, N: int) -> int:
    """OpenMP threads with work under the reference's schedule (mul.cpp:87-96): the basic kernel
    (batch*M*N < 2^20) parallelises batch*M rows, the tiled kernel batch x 64-row x 64-column tiles."""
    if batch * M * N < (1 << 20):
        return min(threads, batch * M)
    return min(threads, batch * -(-M // 64) * -(-N // 64))


def run_cpu(name: str, inp) -> dict:
    import oracle
    a, b, dt = inp["a"], inp["b"], inp["dt"]
    iters, _ = CPU_PLAN[name]
    note = "full workload"
    extra = {}
    flops_full, _ = work(name, inp)
    flops = flops_full
    if name == "c3":
        a = a.reshape(-1, a.shape[-1])
        note = f"full workload as the flattened 2-d call [{a.shape[0]},4096]@[4096,4096]"
    if name == "c4":
        t = time.perf_counter()
        b = oracle.transpose_last2(b)  # ops::Transpose(K,{0,2,1})
        extra["transpose_ms"] = (time.perf_counter() - t) * 1e3
        note = f"full workload on a pre-materialised K^T (its transpose {extra['transpose_ms']:.1f} ms, not in the time)"
    oracle.mul(a[..., :8, :], dt, b, dt)  # page in / thread pool warm-up
    times = []
    for _ in range(iters):
        t = time.perf_counter()
        oracle.mul(a, dt, b, dt)
        times.append(time.perf_counter() - t)
    s = float(np.median(times))
    threads = oracle.threads_used()
    batch = a.shape[0] if a.ndim == 3 else 1
    eff = cpu_effective_threads(threads, batch, a.shape[-2], b.shape[-1])
    unit = "TOP/s" if DTYPE[name] == "int8" else "TFLOP/s"
    return {"value": flops / s / 1e12, "unit": unit, "cores": eff, "kind": "port",
            "sample": f"{name}: {note}; {iters} call(s), median; oracle restatement of MulImpl<CPU> "
                      f"(basic/tiled as the reference selects, fp16/bf16 widening included)",
            "seconds_median": s, "iters": iters, "nproc": os.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "openmp_threads": threads,
            "effective_threads": eff, **extra}


OPS_MUL_TIME = ROOT / "tensorvia_amd" / "bin" / "ops_mul_time"


def run_ops_mul(iters: int = 100) -> dict:
    """ops::Mul through libtensorvia.so on c1's shape, as the reference's benchmark runs it
    (tests/mul.cpp:16-31: 100 calls, the result a temporary; published README.md:154-163, CUDA
    19 ms per call on other hardware): per-call wall time split into result allocation + release,
    kernel (HIP events) and launch + synchronisation.  Once with the context's device block cache
    and once without it (TV_HIP_CACHE_LIMIT_MB=0: hipMalloc / hipFree per result, as the
    reference's CUDA backend), each in a child process."""
    import subprocess
    out = {"program": str(OPS_MUL_TIME.relative_to(ROOT)), "iters": iters,
           "reference": "tests/mul.cpp:16-31 loop; README.md:154-163 publishes 19 ms per call (CUDA, other hardware)"}
    if not OPS_MUL_TIME.exists():
        out["error"] = "not built"
        return out
    for key, env_extra in (("cached", {}), ("uncached", {"TV_HIP_CACHE_LIMIT_MB": "0"})):
        env = dict(os.environ, **env_extra)
        r = subprocess.run([str(OPS_MUL_TIME), str(iters)], capture_output=True, text=True, env=env, timeout=300)
        if r.returncode != 0:
            out[key] = {"error": (r.stderr or r.stdout).strip()[-400:]}
            continue
        out[key] = json.loads(r.stdout.strip().splitlines()[-1])
    return out


def _smi_sample():
    """(board power W, mean shader clock MHz) from amd-smi, or None."""
    import subprocess
    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True, text=True, timeout=20)
        d = json.loads(r.stdout)["gpu_data"][0]
        clks = [v["clk"]["value"] for k, v in d["clock"].items() if k.startswith("gfx_") and isinstance(v, dict)]
        return float(d["power"]["socket_power"]["value"]), float(np.mean(clks))
    except Exception:
        return None


def run_power(names, secs: float = 5.0) -> dict:
    """Board power and shader clock (amd-smi, sampled several times a second) while one
    configuration's kernel runs back to back for `secs` seconds, first on the benchmark's seeded
    inputs, then on all-zero operands of the same shapes: the same instructions and memory traffic
    without the data toggling.  A configuration whose time drops on zeros while the clock rises is
    held by the chip's power management, not by its instruction schedule."""
    import subprocess
    import threading

    import torch

    import tensorvia_amd as tv
    from tensorvia_amd.matmul import storage_to_torch as to_torch
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            t = time.time()
            v = _smi_sample()
            if v:
                samples.append((t, *v))
            time.sleep(0.05)

    cap = None
    try:
        m = re.search(r"Max Graphics Package Power \(W\):\s*([\d.]+)",
                      subprocess.run(["rocm-smi", "--showmaxpower"], capture_output=True, text=True, timeout=20).stdout)
        cap = float(m.group(1)) if m else None
    except (OSError, subprocess.SubprocessError):
        pass
    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    L = tv.lib()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    out = {"cap_w": cap, "seconds": secs, "configs": {}}
    for name in names:
        inp = make_inputs(name)
        dt = inp["dt"]
        a = to_torch(inp["a"], dt)
        b = to_torch(inp["b"], dt)
        if name == "c4":
            b = b.permute(0, 2, 1)
        reps = [b] + ([b.clone() for _ in range(5)] if name.startswith("c5") else [])
        c = tv.gemm(a, b)
        flops, bytes_ = work(name, inp)
        res = {}
        for mode in ("random", "zeros"):
            if mode == "zeros":
                a.zero_()
                for r_ in reps:
                    r_.zero_()
            descs = [tv.make_args(a, r_, c) for r_ in reps]
            for i in range(20):
                tv.check(L.tv_hip_gemm(ctypes.byref(descs[i % len(descs)]), sh))
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0, n = time.time(), 0
            e0.record()
            while time.time() - t0 < secs:
                for i in range(50):
                    rc = L.tv_hip_gemm(ctypes.byref(descs[(n + i) % len(descs)]), sh)
                    if rc:
                        tv.check(rc)
                n += 50
                torch.cuda.synchronize()
            e1.record()
            torch.cuda.synchronize()
            t1 = time.time()
            ms = e0.elapsed_time(e1) / n
            w = [(p, f) for (t, p, f) in samples if t0 + 0.7 < t < t1]
            frac = flops / (ms * 1e-3) / 1e12 / PEAK[DTYPE[name]] if BOUND[name] == "mfma" else \
                bytes_ / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS
            res[mode] = {"us_per_launch": ms * 1e3, "roofline_frac": frac, "samples": len(w),
                         "power_w_mean": float(np.mean([p for p, _ in w])) if w else None,
                         "power_w_max": float(np.max([p for p, _ in w])) if w else None,
                         "sclk_mhz_mean": float(np.mean([f for _, f in w])) if w else None}
            log(f"power {name} {mode:6s}: {ms * 1e3:8.2f} us  frac {frac:.3f}  "
                f"{res[mode]['power_w_mean'] or float('nan'):7.1f} W (max {res[mode]['power_w_max'] or float('nan'):.0f})  "
                f"{res[mode]['sclk_mhz_mean'] or float('nan'):6.0f} MHz  ({len(w)} samples)")
            time.sleep(1.0)
        out["configs"][name] = res
        del a, b, reps, c
        torch.cuda.empty_cache()
    stop.set()
    th.join(timeout=30)
    return out


def trace_check(name: str, res: dict) -> dict | None:
    """The committed kernel trace's figures for this config's kernel, beside the live ones."""
    if not TRACE_FILE.exists() or name not in KERNEL:
        return None
    tr = json.loads(TRACE_FILE.read_text())
    k = tr.get("configs", {}).get(name)
    if not k:
        return None
    trace_ms = k["avg_ns"] * 1e-6
    out = {"trace_file": str(TRACE_FILE.relative_to(ROOT)), "trace_avg_ms": trace_ms,
           "trace_median_ms": k.get("median_ns", k["avg_ns"]) * 1e-6,
           "trace_vs_live": trace_ms / res["kernel_ms_mean"],
           "trace_exceeds_ms_per_step": trace_ms > res["ms_per_step"]}
    if BOUND[name] == "mfma":
        out["frac_from_trace"] = res["flops"] / (trace_ms * 1e-3) / 1e12 / PEAK[DTYPE[name]]
    else:
        out["frac_from_trace"] = res["algorithmic_bytes"] / (trace_ms * 1e-3) / 1e9 / PEAK_HBM_GBS
    return out


def trace_summary(csv_path: str, steps: int) -> dict:
    """Per-configuration durations (End - Start) of the last `steps` dispatches of each
    configuration's kernel in a rocprofv3 kernel_trace.csv of `bench.py --steps S --no-cpu`: the
    timed launches close each configuration's run of back-to-back dispatches.  A kernel's dispatches
    are cut into runs at gaps of more than 2 ms, and runs shorter than `steps` dropped; configurations
    that share a kernel (c5 M=1, then M=8) take its runs in order, the others its first run (a
    later run of the same kernel, such as the c2 power sample's zeroed operands at the end of the
    default run, is not the configuration's timing)."""
    import csv
    import re
    import statistics as st
    rows = sorted(csv.DictReader(open(csv_path)), key=lambda r: int(r["Start_Timestamp"]))
    out, used = {}, {}
    for name, pat in TRACE_KERNEL.items():
        rx = re.compile(pat)
        ds = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows if rx.search(r["Kernel_Name"])]
        runs, cur = [], []
        for d in ds:
            if cur and d[0] - cur[-1][1] > 2_000_000:
                runs.append(cur)
                cur = []
            cur.append(d)
        if cur:
            runs.append(cur)
        runs = [r for r in runs if len(r) >= steps]
        if not runs:
            continue
        if pat in used:
            i = used[pat] + 1
        else:
            i = 0
        if i >= len(runs):
            continue
        used[pat] = i
        dur = [e - b for b, e in runs[i][-steps:]]
        out[name] = {"dispatches": len(dur), "avg_ns": st.mean(dur), "median_ns": st.median(dur),
                     "min_ns": min(dur), "max_ns": max(dur), "run_dispatches": len(runs[i])}
    return out


DEFAULT_CONFIGS = "c1,c2,c3,c3_fused,bf16_4096,c4,c5m1,c5m8,cast_c3a,random_c3a,fill_c3a,transpose_c4k"
POWER_CONFIGS = ["c2", "bf16_4096", "c3", "c1", "c4", "c5m1"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default=DEFAULT_CONFIGS)
    ap.add_argument("--only", default=None,
                    help="run only this config's GPU kernel (for profilers); 'copy' runs the traffic calibration copy")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--vendor", action="store_true", help="also time torch's library GEMM on the same inputs")
    ap.add_argument("--no-ops-mul", action="store_true", help="skip timing ops::Mul end to end (c1_ops_mul)")
    ap.add_argument("--no-power", action="store_true",
                    help="skip the short c2 power/clock sample (seeded inputs, then zeros) of the default run")
    ap.add_argument("--power", action="store_true",
                    help="board power and clock (amd-smi) per GEMM config on the seeded inputs and on zeros, then exit")
    ap.add_argument("--trace-summary", metavar="CSV", default=None,
                    help="summarise a rocprofv3 kernel_trace.csv of this bench (with the same --steps) and exit")
    args = ap.parse_args()
    if args.trace_summary:
        print(json.dumps({"steps": args.steps, "configs": trace_summary(args.trace_summary, args.steps)}, indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the matmul path would shard by batch/M or N columns with no exchange, which is not "
              "measured here", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    import tensorvia_amd as tv
    tv.lib()  # fail loudly if the kernel library is not built

    if args.only == "copy":
        print(json.dumps({"only": "copy", **run_copy(args.steps, args.warmup)}))
        return 0
    if args.power:
        names = [n for n in (args.configs.split(",") if args.configs != DEFAULT_CONFIGS else POWER_CONFIGS)
                 if n in DESC and n not in EW and n != "c3_fused"]
        print(json.dumps({"power": run_power(names)}))
        return 0
    names = [args.only] if args.only else args.configs.split(",")
    if "c2" not in names and not args.only:
        names.insert(0, "c2")
    results, inputs = {}, {}
    for n in names:
        if n in EW:
            log(f"gpu {n}: {EW[n]}")
            results[n] = run_ew(n, args.steps, args.warmup)
            log(f"gpu {n}: {results[n]['kernel_ms_mean'] * 1e3:.1f} us  {results[n]['hbm_gbs']:.0f} GB/s")
            continue
        log(f"gpu {n}: {DESC[n]}")
        results[n], inputs[n] = run_gpu(n, args.steps, args.warmup)
        r = results[n]
        log(f"gpu {n}: {r['kernel_ms_mean'] * 1e3:.1f} us mean, {r['kernel_ms_median_of_runs'] * 1e3:.1f} us median "
            f"of 5 runs  {r['tflops']:.1f} T/s  {r['hbm_gbs']:.0f} GB/s  roofline {r['roofline_frac']:.3f}")
        tc = trace_check(n, r)
        if tc:
            r["profile"] = tc
            # The reported fraction is the lower of the live (event) one and the committed trace's.
            r["roofline_frac_events"] = r["roofline_frac"]
            r["roofline_frac"] = min(r["roofline_frac"], tc["frac_from_trace"])
        if args.vendor:
            v = run_vendor(n, inputs[n], args.steps, args.warmup)
            r["torch_library"] = v
            log(f"torch {n}: {v['ms_mean'] * 1e3:.1f} us  {v['tflops']:.1f} T/s  {v['hbm_gbs']:.0f} GB/s  ({v['call']})")
    if args.only:
        print(json.dumps({"only": args.only, **results[args.only]}))
        return 0

    if not args.no_cpu:
        for n in names:
            if n in CPU_PLAN and n in inputs:
                log(f"cpu baseline {n} (oracle)")
                results[n]["cpu_baseline"] = c = run_cpu(n, inputs[n])
                log(f"cpu {n}: {c['seconds_median']:.3f} s per call, {c['value'] * 1e3:.2f} G/s, "
                    f"{c['openmp_threads']} OpenMP threads, {c['effective_threads']} with work")

    if not args.no_ops_mul and "c1" in names:
        log("ops::Mul end to end (tensorvia_amd/bin/ops_mul_time: the reference's tests/mul.cpp loop)")
        results["c1_ops_mul"] = c = run_ops_mul()
        if "cached" in c:
            log(f"ops::Mul c1: {c['cached']['ops_mul_ms']:.3f} ms per call with the block cache, "
                f"{c.get('uncached', {}).get('ops_mul_ms', float('nan')):.3f} ms without")

    power = None
    if not args.no_power:
        log("power and clock during c2 (amd-smi): seeded inputs, then zeroed operands")
        power = run_power(["c2"], secs=2.0)

    head = results["c2"]
    traffic = None
    tf = ROOT / "profiles" / "gemm_int8_c2_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    frac_ev = head["tflops_frac_peak"]
    frac = head["roofline_frac"]  # min(events, committed trace)
    roof = {"bound": "mfma", "achieved": frac * PEAK["int8"], "peak": PEAK["int8"], "unit": "TOP/s",
            "frac": frac, "frac_events": frac_ev, "traffic": traffic,
            "kernel": KERNEL["c2"],
            "per_launch_ms": head["kernel_ms_mean"], "per_launch_ms_median_of_runs": head["kernel_ms_median_of_runs"],
            "achieved_basis": "algorithmic ops / launch duration: the lower of the mean over the timed region (HIP "
                              "events on the launch stream, frac_events) and the committed kernel trace's average "
                              "(profile.frac_from_trace)"}
    if "profile" in head:
        roof["profile"] = head["profile"]
    cpu = head.get("cpu_baseline")
    line = {
        "metric": METRIC,
        "value": head["flops"] / (head["ms_per_step"] * 1e-3) / 1e12,
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded counter-based generator (SplitMix64), uniform ints in [-10,10]",
        "config": {"workload": "c2: " + DESC["c2"], "M": 4096, "N": 4096, "K": 4096, "accumulate": "int32",
                   "why": "BASELINE.json configs[1] (configs[0] is the reference's CPU-runnable README case): "
                          "a full-size config at the reference's own int8 precision and wrap semantics. The "
                          "metric is per dtype, so every config is under configs; the reference's only "
                          "published figure (README.md:154-163, ops::Mul on c1's shape, other hardware) is "
                          "matched by configs.c1_ops_mul"},
        "settle_s_per_config": SETTLE_S,
        "roofline": roof,
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in (
            "value", "unit", "cores", "kind", "sample", "nproc", "omp_num_threads", "openmp_threads", "effective_threads")},
        "configs": results,
    }
    if power is not None:
        line["power"] = {**power, "note": "board power (W) and gfx clock (MHz) sampled while c2 runs back to back; "
                                          "the same kernel on zeroed operands shows what the clock the power cap "
                                          "allows costs (profiles/power_clock_random_vs_zero.md)"}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
