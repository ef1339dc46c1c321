"""GPU: the per-stream workspace under memory pressure, and what tv_hip_gemm_noalloc gives on calls
that tv_hip_gemm serves from the workspace.

* With every workspace allocation failing (tv_hip_inject_alloc_failure, which makes the library ask
  the HIP runtime for more memory than any device has), a call that would split K (stream-K slots,
  GEMV split-K slots) or copy a misaligned operand into padded rows runs on the kernels that need
  no workspace, returns 0 (the failed allocation does not surface as the launch's error) and gives
  the exact result.  Each case runs on a fresh stream, whose workspace is empty.
* A float skinny call on a misaligned W (bf16 N = 129): tv_hip_gemm pads W and runs the matrix-core
  GEMV, tv_hip_gemm_noalloc reads W in place on the GEMM; both meet the bf16 parity bar against
  fp64, and they differ at most in the last bits.
"""
import ctypes

import numpy as np
import pytest
import torch

import tensorvia_amd as tv
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT32, INT8, assert_half_close, to_f32, to_storage, to_torch

pytestmark = pytest.mark.gpu


def _int_operands(dt, shape_a, shape_b, seed, lo, hi):
    a = rng.uniform_int(seed, int(np.prod(shape_a)), lo, hi).reshape(shape_a)
    b = rng.uniform_int(seed + 1, int(np.prod(shape_b)), lo, hi).reshape(shape_b)
    if dt == INT8:
        return a.astype(np.int8), b.astype(np.int8)
    if dt == BFLOAT16:
        return rng.f32_to_bf16_bits(a.astype(np.float32)), rng.f32_to_bf16_bits(b.astype(np.float32))
    return a.astype(np.float32), b.astype(np.float32)


def _exact(dt, a, b):
    """Exact product of integer-valued operands, in the output's storage."""
    if dt == INT8:
        # float64 products and sums of int8 values are exact here (|sum| <= 127^2 K < 2^53); then the
        # low byte (two's complement)
        return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.int64).astype(np.int8)
    fa, fb = to_f32(a, dt).astype(np.float64), to_f32(b, dt).astype(np.float64)
    c = (fa @ fb).astype(np.float32)
    return rng.f32_to_bf16_bits(c) if dt == BFLOAT16 else c


def _gemm_on(stream, fn, ta, tb):
    tc = torch.full(tuple(ta.shape[:-1]) + (tb.shape[-1],), 7, dtype=ta.dtype, device="cuda")
    args = tv.make_args(ta, tb, tc)
    rc = getattr(tv.lib(), fn)(ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream))
    stream.synchronize()
    return rc, to_storage(tc)


# (name, dtype, A shape, B shape, value range): each would use the workspace on a fresh stream.
CASES = [
    ("bf16_padded_b", BFLOAT16, (64, 512), (512, 260), 3),          # N = 260: B copied into padded rows
    ("bf16_padded_skinny_w", BFLOAT16, (1, 4096), (4096, 129), 2),  # W padded, then the split-K GEMV
    ("bf16_gemv_split_k", BFLOAT16, (8, 4096), (4096, 4096), 2),    # GEMV split-K slots
    ("fp32_stream_k", FLOAT32, (1024, 1024), (1024, 1024), 3),      # 64 tiles: stream-K slots
    ("int8_stream_k", INT8, (512, 4096), (4096, 4096), 127),        # 128 tiles of 128x128: split
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_failed_workspace_allocation_falls_back(hip, case):
    name, dt, sa, sb, r = case
    a, b = _int_operands(dt, sa, sb, 900 + len(name), -r, r)
    want = _exact(dt, a, b)
    ta, tb = to_torch(a, dt), to_torch(b, dt)
    L = tv.lib()
    try:
        L.tv_hip_inject_alloc_failure(1000)
        rc, got = _gemm_on(torch.cuda.Stream(), "tv_hip_gemm", ta, tb)
    finally:
        L.tv_hip_inject_alloc_failure(0)
    assert rc == tv.TV_OK, f"{name}: {tv.strerror(rc)}"
    np.testing.assert_array_equal(got, want, err_msg=f"{name}: no-workspace path")
    rc, got = _gemm_on(torch.cuda.Stream(), "tv_hip_gemm", ta, tb)  # the workspace path on a fresh stream
    assert rc == tv.TV_OK
    np.testing.assert_array_equal(got, want, err_msg=f"{name}: workspace path")


def test_earlier_hip_failure_is_not_reported_as_the_call_s(hip):
    """An error that an unrelated HIP call left as the thread's last error (a hipMalloc too large for
    any device, unchecked) is not returned by the next tv_hip_gemm, whose own launch succeeds, and
    the result is exact."""
    hiprt = ctypes.CDLL("libamdhip64.so.7")  # by soname: the runtime already loaded, not a second copy
    hiprt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hiprt.hipMalloc.restype = ctypes.c_int
    hiprt.hipGetLastError.restype = ctypes.c_int
    a, b = _int_operands(INT8, (64, 96), (96, 80), 950, -3, 3)
    ta, tb = to_torch(a, INT8), to_torch(b, INT8)
    tc = torch.zeros((64, 80), dtype=torch.int8, device="cuda")
    args = tv.make_args(ta, tb, tc)
    stream = torch.cuda.current_stream()
    stream.synchronize()
    # No torch call between the planted failure and the library's call: torch reads the last error
    # after its own launches too.
    p = ctypes.c_void_p()
    assert hiprt.hipMalloc(ctypes.byref(p), 1 << 60) != 0  # fails, and stays as the last error
    rc = tv.lib().tv_hip_gemm(ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream))
    last = hiprt.hipGetLastError()
    assert rc == tv.TV_OK, tv.strerror(rc)
    assert last == 0
    stream.synchronize()
    np.testing.assert_array_equal(to_storage(tc), _exact(INT8, a, b))


def test_noalloc_on_padded_skinny_float_call(hip):
    """bf16 x[1,4096] @ W[4096,129], random values: the padded matrix-core GEMV (tv_hip_gemm) and
    the in-place GEMM (tv_hip_gemm_noalloc) sum K in different orders; both are within the bf16 bar
    (1e-2 relative to the fp32-accumulated value), and they differ by at most 2 bf16 ulp."""
    x = rng.make("normal", (1, 4096), 71, "bfloat16")
    w = rng.make("uniform", (4096, 129), 72, "bfloat16", lo=-0.05, hi=0.05)
    tx, tw = to_torch(x, BFLOAT16), to_torch(w, BFLOAT16)
    s = torch.cuda.current_stream()
    rc1, c1 = _gemm_on(s, "tv_hip_gemm", tx, tw)
    rc2, c2 = _gemm_on(s, "tv_hip_gemm_noalloc", tx, tw)
    assert rc1 == tv.TV_OK and rc2 == tv.TV_OK
    fx, fw = to_f32(x, BFLOAT16).astype(np.float64), to_f32(w, BFLOAT16).astype(np.float64)
    ref, bound = fx @ fw, np.abs(fx) @ np.abs(fw)
    f1, f2 = to_f32(c1, BFLOAT16), to_f32(c2, BFLOAT16)
    assert_half_close(f1, ref, bound, 4096)
    assert_half_close(f2, ref, bound, 4096)
    ulp = np.spacing(np.maximum(np.abs(f1), np.abs(f2)).astype(np.float32)) * 65536  # bf16 ulp: 2^16 fp32 ulps
    assert (np.abs(f1 - f2) <= 2 * ulp).all()


def test_workspace_users_captured_after_a_warm_up(hip):
    """tv_hip_gemm under HIP graph capture: once a stream's workspace has grown on an eager call of
    each shape, the same calls on that stream allocate and synchronise nothing, so a graph can
    record them.  The workspace users of CASES are captured on one stream and replayed five times,
    with eager fills of the outputs in between; every replay is exact."""
    L = tv.lib()
    s = torch.cuda.Stream()
    calls = []
    for i, (name, dt, sa, sb, r) in enumerate(CASES):
        a, b = _int_operands(dt, sa, sb, 970 + i, -r, r)
        ta, tb = to_torch(a, dt), to_torch(b, dt)
        tc = torch.zeros(tuple(ta.shape[:-1]) + (tb.shape[-1],), dtype=ta.dtype, device="cuda")
        # the operands stay referenced here: the descriptor holds their raw pointers
        calls.append((name, _exact(dt, a, b), (ta, tb), tc, tv.make_args(ta, tb, tc)))
    torch.cuda.synchronize()
    sh = ctypes.c_void_p(s.cuda_stream)
    for name, want, ops, tc, args in calls:  # the warm-up: grows the stream's workspace
        assert L.tv_hip_gemm(ctypes.byref(args), sh) == tv.TV_OK, name
    s.synchronize()
    for name, want, ops, tc, args in calls:
        np.testing.assert_array_equal(to_storage(tc), want, err_msg=f"{name}: eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for name, want, ops, tc, args in calls:
            tv.check(L.tv_hip_gemm(ctypes.byref(args), sh))
    for rep in range(5):
        for name, want, ops, tc, args in calls:
            tc.fill_(5)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, want, ops, tc, args in calls:
            np.testing.assert_array_equal(to_storage(tc), want, err_msg=f"{name}: replay {rep}")
