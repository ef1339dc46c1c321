"""Concurrent C-ABI calls from several host threads, each on its own HIP stream.  The split-K GEMV,
the stream-K GEMMs and the padded operand copies keep their buffers in a workspace per (device,
stream), found through one mutex-guarded table, and the launchers cache per-device values in
atomics; calls on different streams must neither share a buffer nor race on the table.  Each
thread issues every workspace user in turn, without synchronising between calls, so kernels of the
same kind run on several streams at once; every result must then equal the exact sum of its
integer inputs (its low byte for int8 outputs, rounded once for bf16), bit for bit.

The same through the C++ API: tests/cpp/threads_driver.cpp runs ops::Random -> ops::Mul -> to_host()
from four threads that share the HIP context (its stream, block cache and pinned staging).
"""
import subprocess
import threading

import numpy as np
import pytest
import torch

from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT32, INT8, to_storage, to_torch

pytestmark = pytest.mark.gpu

# (name, dtype, M, K, N, value range): each uses the per-stream workspace -- a B copied into padded
# rows (N = 260), an A copied into padded rows (K = 700), a padded W then the split-K GEMV
# (N = 129), the GEMV's split-K slots, the fp32 stream-K slots (64 tiles) and the int8 stream-K
# slots (128 tiles of 128x128).
CASES = [("bf16_padded_b", BFLOAT16, 64, 512, 260, 3), ("bf16_padded_a", BFLOAT16, 300, 700, 1024, 3),
         ("bf16_padded_skinny_w", BFLOAT16, 1, 4096, 129, 2), ("bf16_gemv_split_k", BFLOAT16, 8, 4096, 4096, 2),
         ("fp32_stream_k", FLOAT32, 1024, 1024, 1024, 3), ("int8_stream_k", INT8, 512, 4096, 4096, 127)]
THREADS = 4
ITERS = 6


def _enc(x, dt):
    if dt == INT8:
        return x.astype(np.int8)
    if dt == FLOAT32:
        return x.astype(np.float32)
    return rng.f32_to_bf16_bits(x.astype(np.float32))


def test_threads_on_separate_streams_exact(hip):
    inputs, wants = [], []
    for i, (name, dt, M, K, N, r) in enumerate(CASES):
        x = rng.uniform_int(100 + i, M * K, -r, r).reshape(M, K)
        y = rng.uniform_int(200 + i, K * N, -r, r).reshape(K, N)
        s = np.matmul(x.astype(np.float64), y.astype(np.float64))
        # int8: the low byte of the exact sum; fp32: the exact sum (below 2^24); bf16: the exact sum
        # rounded once.
        wants.append(s.astype(np.int64).astype(np.int8) if dt == INT8 else _enc(s.astype(np.float32), dt))
        inputs.append((to_torch(np.ascontiguousarray(_enc(x, dt)), dt), to_torch(np.ascontiguousarray(_enc(y, dt)), dt)))
    torch.cuda.synchronize()

    results = [[] for _ in range(THREADS)]
    errors = []

    def worker(t):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for it in range(ITERS):
                    for j in range(len(CASES)):
                        k = (j + t + it) % len(CASES)  # threads start on different kinds
                        a, b = inputs[k]
                        results[t].append((k, hip.gemm(a, b, stream=stream)))
            stream.synchronize()
        except Exception as e:  # reported in the main thread
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(THREADS):
        assert len(results[t]) == ITERS * len(CASES)
        for n, (k, c) in enumerate(results[t]):
            np.testing.assert_array_equal(to_storage(c), wants[k], err_msg=f"thread {t} call {n} ({CASES[k][0]})")


def test_cpp_api_from_four_threads(hip):
    """Four threads share the C++ API's HIP context, 12 iterations each (int8, bf16, fp32 GEMV, int8
    GEMV): every iteration's bytes equal the thread's first, and the int8 threads' sampled rows
    equal the low byte of the exact sums (tests/cpp/threads_driver.cpp, in a child process)."""
    from tests.cpp import build as cpp
    r = subprocess.run([str(cpp.binary("threads_driver"))], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    for t in range(4):
        assert f"ok thread {t}: 12 iterations" in r.stdout, r.stdout
