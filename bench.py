#!/usr/bin/env python3
"""Benchmark of the MI355X HIP backend for Tensorvia's ops::Mul (matmul) path.

One "step" is one ops::Mul call (one kernel launch) on device-resident, seeded synthetic inputs.
The JSON line's ``value`` is configuration c2 (int8 A[4096,4096] @ B[4096,4096] -> int8 wrap), the
configuration BASELINE.json's metric is quoted on at N=1; the other four configurations are measured
in the same run and reported under ``configs``.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,...] [--no-cpu]
                       [--only c2]   (only that config's kernel, e.g. under rocprofv3)
                       [--vendor]    (also time torch's own library GEMM on the same inputs)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
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
    "c4": "fp16 Q[32,2048,128] @ K.permute(0,2,1) (strided view, no repack) -> fp16 [32,2048,2048]",
    "c5m1": "bf16 GEMV x[1,4096] @ W[4096,11008] -> bf16, fp32 accumulate (6 W replicas rotated)",
    "c5m8": "bf16 GEMV x[8,4096] @ W[4096,11008] -> bf16, fp32 accumulate (6 W replicas rotated)",
}
DTYPE = {"c1": "fp32", "c2": "int8", "c3": "bf16", "c3_fused": "bf16", "c4": "fp16", "c5m1": "bf16", "c5m8": "bf16"}


def work(name: str, inp) -> tuple[float, float]:
    """(algorithmic flops/ops, algorithmic HBM bytes) per call."""
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
    out_es = es
    return 2.0 * B * M * N * K, (a.size + b.size) * es + B * M * N * out_es


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
    # Descriptors are packed once: the timed loop is one C-ABI call per step, so the host enqueues
    # launches faster than the GPU retires them and the events bracket back-to-back kernels.
    L = tv.lib()
    descs = [tv.make_args(a, r, out) for r in reps]
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    ep = None
    if "bias" in inp:
        bias = to_torch(inp["bias"], dt)
        ep = tv.TvEpilogue()
        ep.act, ep.bias, ep.sbias_b, ep.sbias_m, ep.sbias_n = tv.ACT_SILU, bias.data_ptr(), 0, 0, 1

    def step(i):
        if ep is None:
            rc = L.tv_hip_gemm(ctypes.byref(descs[i % len(descs)]), sh)
        else:
            rc = L.tv_hip_gemm_ex(ctypes.byref(descs[i % len(descs)]), ctypes.byref(ep), sh)
        if rc:
            tv.check(rc)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    per_launch_ms = ev0.elapsed_time(ev1) / steps
    flops, bytes_ = work(name, inp)
    res = {
        "workload": DESC[name],
        "dtype": DTYPE[name],
        "kernel_ms_mean": float(per_launch_ms),
        "ms_per_step": wall_ms,
        "flops": flops,
        "algorithmic_bytes": bytes_,
    }
    res["tflops"] = flops / (res["kernel_ms_mean"] * 1e-3) / 1e12
    res["tflops_frac_peak"] = res["tflops"] / PEAK[DTYPE[name]]
    res["hbm_gbs"] = bytes_ / (res["kernel_ms_mean"] * 1e-3) / 1e9
    res["hbm_frac_peak"] = res["hbm_gbs"] / PEAK_HBM_GBS
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
        fn = lambda i: torch._int_mm(a, b)
        note = "torch._int_mm (int32 output)"
    elif name == "c4":
        bt = b.permute(0, 2, 1).contiguous()
        fn = lambda i: torch.bmm(a, bt)
        note = "torch.bmm with K^T materialised"
    elif "bias" in inp:
        bias = to_torch(inp["bias"], dt)
        fn = lambda i: torch.nn.functional.silu(torch.matmul(a, b) + bias)  # noqa: E731
        note = "torch.nn.functional.silu(torch.matmul(a, b) + bias) (three kernels)"
    else:
        reps = [b] + ([b.clone() for _ in range(5)] if name.startswith("c5") else [])
        fn = lambda i: torch.matmul(a, reps[i % len(reps)])
        if name.startswith("c5"):
            note = "torch.matmul, 6 W replicas rotated"
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        fn(i)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    flops, bytes_ = work(name, inp)
    res = {"call": note, "ms_mean": ms, "tflops": flops / (ms * 1e-3) / 1e12,
           "tflops_frac_peak": flops / (ms * 1e-3) / 1e12 / PEAK[DTYPE[name]], "hbm_gbs": bytes_ / (ms * 1e-3) / 1e9}
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
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if name == "cast_c3a":
        # Two sources (2 x 268 MB) taken in turn, so that no call finds its source in the 256 MB
        # MALL (Infinity Cache) from the call before.
        srcs = [torch.empty(n, dtype=torch.int16, device="cuda") for _ in range(2)]  # bf16 storage
        for s_ in srcs:
            tv.check(L.tv_hip_random(ctypes.c_void_p(s_.data_ptr()), tv.BFLOAT16, n, -1.0, 1.0, 5, sh))
        dst = torch.empty(n, dtype=torch.float32, device="cuda")
        turn = [0]

        def call():
            turn[0] ^= 1
            return L.tv_hip_typecast(ctypes.c_void_p(srcs[turn[0]].data_ptr()), tv.BFLOAT16,
                                     ctypes.c_void_p(dst.data_ptr()), tv.FLOAT32, n, sh)
        nbytes = n * 2 + n * 4
    elif name == "random_c3a":
        dst = torch.empty(n, dtype=torch.int16, device="cuda")
        call = lambda: L.tv_hip_random(ctypes.c_void_p(dst.data_ptr()), tv.BFLOAT16, n, -1.0, 1.0, 5, sh)  # noqa: E731
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
        call = lambda: L.tv_hip_repack(ctypes.byref(a), sh)  # noqa: E731
        nbytes = m * 2 * 2
    else:
        dst = torch.empty(n, dtype=torch.float32, device="cuda")
        call = lambda: L.tv_hip_fill(ctypes.c_void_p(dst.data_ptr()), tv.FLOAT32, n, 1.0, sh)  # noqa: E731
        nbytes = n * 4
    for _ in range(warmup):
        tv.check(call())
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        call()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    res = {"workload": EW[name], "kernel_ms_mean": ms, "algorithmic_bytes": nbytes,
           "hbm_gbs": nbytes / (ms * 1e-3) / 1e9}
    res["hbm_frac_peak"] = res["hbm_gbs"] / PEAK_HBM_GBS
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
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        dst.copy_(src)
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    return {"workload": "device copy of 512 MiB (uint8)", "bytes_read": n, "bytes_written": n,
            "kernel_ms_mean": ms, "hbm_gbs": 2 * n / (ms * 1e-3) / 1e9}


def run_cpu(name: str, inp, iters: int):
    import oracle
    a, b, dt = inp["a"], inp["b"], inp["dt"]
    note = ""
    t_extra = 0.0
    if name == "c3":
        a = a.reshape(-1, a.shape[-1])  # the reference rejects the broadcast form: flattened 2-D call
        note = "flattened [32768,4096]@[4096,4096]"
    if name == "c4":
        t = time.perf_counter()
        b = oracle.transpose_last2(b)  # ops::Transpose(K,{0,2,1}): the CPU matmul ignores strides
        t_extra = time.perf_counter() - t
        note = f"pre-materialised K^T (transpose {t_extra * 1e3:.1f} ms, excluded)"
    oracle.mul(a[:8], dt, b, dt) if a.ndim == 2 else None  # page in / thread pool warm-up
    times = []
    t_start = time.perf_counter()
    # At least `iters` calls, continuing until about 10 s of CPU time has been measured.
    while len(times) < iters or (time.perf_counter() - t_start < 10.0 and len(times) < 50):
        t = time.perf_counter()
        oracle.mul(a, dt, b, dt)
        times.append(time.perf_counter() - t)
    iters = len(times)
    flops, _ = work(name, inp)
    s = float(np.mean(times))
    return {"value": flops / s / 1e12, "unit": "TFLOP/s" if DTYPE[name] != "int8" else "TOP/s",
            "seconds": s, "iters": iters, "cores": oracle.threads_used(), "kind": "port",
            "sample": f"full {name} workload, {iters} iteration(s), oracle restatement of MulImpl<CPU> "
                      f"(tiled/basic as the reference selects, 16-thread cap){'; ' + note if note else ''}",
            "nproc": os.cpu_count(), "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="c1,c2,c3,c3_fused,c4,c5m1,c5m8,cast_c3a,random_c3a,fill_c3a,transpose_c4k")
    ap.add_argument("--only", default=None,
                    help="run only this config's GPU kernel (for profilers); 'copy' runs the traffic calibration copy")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-all", action="store_true", help="CPU baseline for every config, not only c2")
    ap.add_argument("--vendor", action="store_true", help="also time torch's library GEMM on the same inputs")
    args = ap.parse_args()
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
        log(f"gpu {n}: {results[n]['kernel_ms_mean'] * 1e3:.1f} us  {results[n]['tflops']:.1f} T/s  "
            f"{results[n]['hbm_gbs']:.0f} GB/s")
        if args.vendor:
            v = run_vendor(n, inputs[n], args.steps, args.warmup)
            results[n]["torch_library"] = v
            log(f"torch {n}: {v['ms_mean'] * 1e3:.1f} us  {v['tflops']:.1f} T/s  {v['hbm_gbs']:.0f} GB/s  ({v['call']})")
    if args.only:
        print(json.dumps({"only": args.only, **results[args.only]}))
        return 0

    head = results["c2"]
    cpu = None
    if not args.no_cpu:
        log("cpu baseline c2 (oracle)")
        cpu = run_cpu("c2", inputs["c2"], iters=3)
        log(f"cpu c2: {cpu['seconds']:.2f} s, {cpu['value'] * 1e3:.1f} GOP/s on {cpu['cores']} threads")
        if args.cpu_all:
            for n in names:
                if n != "c2" and n not in EW and n != "c3_fused":
                    log(f"cpu baseline {n}")
                    results[n]["cpu_baseline"] = run_cpu(n, inputs[n], iters=1)

    traffic = None
    tf = ROOT / "profiles" / "gemm_int8_c2_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")
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
        "config": {"workload": "c2: " + DESC["c2"], "M": 4096, "N": 4096, "K": 4096, "accumulate": "int32"},
        "roofline": {"bound": "mfma", "achieved": head["tflops"], "peak": PEAK["int8"], "unit": "TOP/s",
                     "frac": head["tflops_frac_peak"], "traffic": traffic,
                     "kernel": "gemm_dma_kernel<int8, 256x256 tile, 2-stage global->LDS DMA, A k-contiguous, B n-contiguous>",
                     "per_launch_ms": head["kernel_ms_mean"]},
        "cpu_baseline": None if cpu is None else {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "configs": results,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
