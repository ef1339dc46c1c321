"""tv_hip_gemm_noalloc (the entry point that allocates nothing) against tv_hip_gemm, through the C-ABI.

The two share kernels and slice plans, so results must be identical bit for bit; the no-alloc
variant takes the GEMV's split-K partials from the library's static per-GPU array instead of the
per-stream workspace.  Each case runs two calls in a row, the second with a smaller input, so the
second call finds the array holding the first call's partials (its counters must be back at zero).
"""
import ctypes

import numpy as np
import pytest
import torch

import tensorvia_amd as tv
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT32, INT8, INT32, to_storage, to_torch

pytestmark = pytest.mark.gpu


def _operands(dt, shape_a, shape_b, seed):
    if dt == INT8:
        a = rng.uniform_int(seed, int(np.prod(shape_a)), -128, 127).astype(np.int8).reshape(shape_a)
        b = rng.uniform_int(seed + 1, int(np.prod(shape_b)), -128, 127).astype(np.int8).reshape(shape_b)
        return to_torch(a, INT8), to_torch(b, INT8)
    if dt == BFLOAT16:
        a = rng.make("normal", shape_a, seed, "bfloat16")
        b = rng.make("uniform", shape_b, seed + 1, "bfloat16", lo=-0.05, hi=0.05)
        return to_torch(a, BFLOAT16), to_torch(b, BFLOAT16)
    a = rng.uniform_f32(seed, int(np.prod(shape_a)), -1, 1).reshape(shape_a)
    b = rng.uniform_f32(seed + 1, int(np.prod(shape_b)), -1, 1).reshape(shape_b)
    return to_torch(a, FLOAT32), to_torch(b, FLOAT32)


def _call(fn, a, b, out_dtype=None):
    shape = tuple(a.shape[:-1]) + (b.shape[-1],)
    c = torch.zeros(shape, dtype=a.dtype if out_dtype is None else tv.tv_to_torch(out_dtype), device="cuda")
    args = tv.make_args(a, b, c)
    rc = getattr(tv.lib(), fn)(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    tv.check(rc)
    torch.cuda.synchronize()
    return to_storage(c)


# (dtype, out dtype, first (A, B) shapes, second, smaller (A, B) shapes); every first call splits K
# over several workgroups per strip, so it uses the scratch array.
CASES = [
    ("bf16_c5_m8_then_m1", BFLOAT16, None, ((8, 4096), (4096, 11008)), ((1, 1024), (1024, 2048))),
    ("bf16_c5_m1_then_batched", BFLOAT16, None, ((1, 4096), (4096, 11008)), ((2, 3, 512), (512, 640))),
    ("int8_matrix_core_m4_int32", INT8, INT32, ((4, 4096), (4096, 4096)), ((3, 2048), (2048, 1024))),
    ("int8_dot_m2", INT8, None, ((2, 4096), (4096, 4096)), ((1, 1024), (1024, 512))),
    ("fp32_dot_m2", FLOAT32, None, ((2, 2048), (2048, 3000)), ((1, 512), (512, 640))),
    ("gemm_route_m300", BFLOAT16, None, ((300, 512), (512, 640)), ((9, 256), (256, 128))),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_gemm_on_two_calls(hip, case):
    name, dt, out_dt, first, second = case
    for i, (sa, sb) in enumerate((first, second)):
        a, b = _operands(dt, sa, sb, 50 + 7 * i)
        want = _call("tv_hip_gemm", a, b, out_dt)
        got = _call("tv_hip_gemm_noalloc", a, b, out_dt)
        np.testing.assert_array_equal(got, want, err_msg=f"{name} call {i + 1}")
        again = _call("tv_hip_gemm_noalloc", a, b, out_dt)
        np.testing.assert_array_equal(again, want, err_msg=f"{name} call {i + 1} repeated")


def test_noalloc_rejects_a_split_beyond_the_static_scratch(hip):
    """x[8, 32768] @ W[32768, 19200] bf16: 300 strips x 8 K-slices x 2 KiB of partials (4.7 MiB) do
    not fit the 4 MiB array: TV_E_SCRATCH before any launch; tv_hip_gemm serves the same call."""
    a = torch.empty((8, 32768), dtype=torch.bfloat16, device="cuda").normal_()
    b = torch.empty((32768, 19200), dtype=torch.bfloat16, device="cuda").uniform_(-0.05, 0.05)
    c = torch.empty((8, 19200), dtype=torch.bfloat16, device="cuda")
    args = tv.make_args(a, b, c)
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), sh) == tv.TV_E_SCRATCH
    assert "static" in tv.strerror(tv.TV_E_SCRATCH)
    tv.check(tv.lib().tv_hip_gemm(ctypes.byref(args), sh))
    torch.cuda.synchronize()


def test_noalloc_in_a_captured_graph(hip):
    """The callers the entry point is for, under HIP graph capture: a graph records two
    tv_hip_gemm_noalloc calls (bf16 x[8, 4096] @ W[4096, 11008] on the split-K GEMV, whose partials
    and counters live in the static array, then an int8 GEMM) and is replayed five times, with eager
    work in between (fills of the outputs, a smaller eager no-alloc call that reuses the array,
    synchronisations); every replay equals the eager tv_hip_gemm results bit for bit."""
    L = tv.lib()
    a1, b1 = _operands(BFLOAT16, (8, 4096), (4096, 11008), 90)
    a2, b2 = _operands(INT8, (300, 512), (512, 640), 92)
    x3, w3 = _operands(BFLOAT16, (1, 1024), (1024, 2048), 94)
    want1, want2 = _call("tv_hip_gemm", a1, b1), _call("tv_hip_gemm", a2, b2)
    want3 = _call("tv_hip_gemm", x3, w3)
    # Eager first calls: the static array's set-up and the per-shape plans happen outside the capture.
    np.testing.assert_array_equal(_call("tv_hip_gemm_noalloc", a1, b1), want1)
    np.testing.assert_array_equal(_call("tv_hip_gemm_noalloc", a2, b2), want2)
    c1 = torch.zeros((8, 11008), dtype=torch.bfloat16, device="cuda")
    c2 = torch.zeros((300, 640), dtype=torch.int8, device="cuda")
    args1, args2 = tv.make_args(a1, b1, c1), tv.make_args(a2, b2, c2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        tv.check(L.tv_hip_gemm_noalloc(ctypes.byref(args1), sh))
        tv.check(L.tv_hip_gemm_noalloc(ctypes.byref(args2), sh))
    for r in range(5):
        c1.fill_(3.0)
        c2.fill_(3)
        np.testing.assert_array_equal(_call("tv_hip_gemm_noalloc", x3, w3), want3, err_msg=f"eager call before replay {r}")
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_storage(c1), want1, err_msg=f"replay {r}: GEMV")
        np.testing.assert_array_equal(to_storage(c2), want2, err_msg=f"replay {r}: GEMM")
