"""GPU edge cases of the matmul entry points, through the C-ABI:

* K = 0: every output is the empty sum (through the fused epilogue: act(bias)), on the GEMV-shaped
  and GEMM-shaped routes of tv_hip_gemm, tv_hip_gemv and tv_hip_gemm_ex;
* the GEMV kernels at the LDS cap on x's K-slice: shapes whose strip count leaves one K-slice per
  strip, so each slice is as long as x's LDS rows allow (8,192 int8 rows, 4,096 bf16 rows);
* descriptors the C-ABI refuses (zero output strides, negative strides, 2^56-byte spans) on real
  device buffers: refused before any launch, C untouched.

The reference's mul_kernel_basic (src/backend/cpu/mul.cpp:7-25) sums nothing for K = 0 and stores
the zero it started from; for the cap cases the bars are the usual ones (int8 bit-exact against the
exact sums; integer-valued bf16 inputs, whose fp32 sums are exact, bit-exact after rounding).
"""
import ctypes

import numpy as np
import pytest
import torch

import tensorvia_amd as tv
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT32, INT8, INT32, to_storage, to_torch

pytestmark = pytest.mark.gpu


def _k0_operands(dt, batch, M, N):
    tdt = {FLOAT32: torch.float32, BFLOAT16: torch.bfloat16, INT8: torch.int8}[dt]
    lead = (batch,) if batch else ()
    a = torch.empty(lead + (M, 0), dtype=tdt, device="cuda")
    b = torch.empty((0, N), dtype=tdt, device="cuda")
    return a, b


@pytest.mark.parametrize("dt,batch,M,N", [(FLOAT32, 0, 1, 64), (INT8, 0, 2, 96), (BFLOAT16, 0, 1, 32),
                                          (BFLOAT16, 3, 8, 200), (FLOAT32, 0, 300, 130), (INT8, 2, 40, 70)],
                         ids=["f32_m1", "i8_m2", "bf16_n32", "bf16_batched_m8", "f32_m300", "i8_batched_m40"])
@pytest.mark.parametrize("entry", ["gemm", "gemv"])
def test_k0_writes_zeros(hip, dt, batch, M, N, entry):
    if entry == "gemv" and M > 8:
        pytest.skip("tv_hip_gemv serves M <= 8")
    a, b = _k0_operands(dt, batch, M, N)
    out_dtype = INT32 if dt == INT8 else None
    for od in (None, out_dtype) if out_dtype is not None else (None,):
        c = getattr(hip, entry)(a, b, out_dtype=od)  # a rank-3 A takes b broadcast over the batch
        c.fill_(7)  # garbage the kernel must overwrite
        getattr(hip, entry)(a, b, out=c, out_dtype=od)
        torch.cuda.synchronize()
        assert not to_storage(c).any()


@pytest.mark.parametrize("M", [1, 4, 300])
def test_k0_fused_epilogue_is_act_of_bias(hip, M):
    """tv_hip_gemm_ex with K = 0: C = silu(0 + bias) for a per-column bias (fp32 in, fp32 out)."""
    N = 96
    a, b = _k0_operands(FLOAT32, 0, M, N)
    bias = torch.from_numpy(rng.uniform_f32(5, N, -2, 2)).cuda()
    c = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    args = tv.make_args(a, b, c)
    ep = tv.TvEpilogue()
    ep.act, ep.reserved, ep.bias, ep.sbias_b, ep.sbias_m, ep.sbias_n = tv.ACT_SILU, 0, bias.data_ptr(), 0, 0, 1
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep),
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    x = bias.double().cpu().numpy()
    want = np.broadcast_to(x / (1 + np.exp(-x)), (M, N))
    got = c.double().cpu().numpy()
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-30)


def _exact(x, w):
    """Exact integer sums through fp64 (every partial sum is an integer below 2^53)."""
    return np.matmul(x.astype(np.float64), w.astype(np.float64))


def test_gemv_int8_matrix_core_at_lds_cap(hip):
    """x[344,8,16384] @ broadcast W[16384,128] int8: 344 strips, so 2 K-slices of 8,192 rows (64 KB of
    x in LDS beside the matrix-core kernel's static arrays); int8 and int32 outputs bit-exact."""
    Bt, M, K, N = 344, 8, 16384, 128
    x = rng.uniform_int(70, Bt * M * K, -128, 127).astype(np.int8).reshape(Bt, M, K)
    w = rng.uniform_int(71, K * N, -128, 127).astype(np.int8).reshape(K, N)
    exact = _exact(x.reshape(Bt * M, K), w).astype(np.int64).reshape(Bt, M, N)
    tx, tw = to_torch(x, INT8), to_torch(w, INT8)
    c32 = to_storage(hip.gemv(tx, tw, out_dtype=INT32))
    c8 = to_storage(hip.gemv(tx, tw))
    np.testing.assert_array_equal(c32, exact.astype(np.int32))
    np.testing.assert_array_equal(c8, exact.astype(np.int8))


def test_gemv_bf16_matrix_core_at_lds_cap(hip):
    """x[688,8,8192] @ broadcast W[8192,64] bf16, integer values: 688 strips, 2 K-slices of 4,096 rows
    (64 KB of x in LDS); fp32 output exact, bf16 output the RNE rounding of the exact sum."""
    Bt, M, K, N = 688, 8, 8192, 64
    x = rng.uniform_int(72, Bt * M * K, -2, 2).astype(np.float32).reshape(Bt, M, K)
    w = rng.uniform_int(73, K * N, -2, 2).astype(np.float32).reshape(K, N)
    exact = _exact(x.reshape(Bt * M, K), w).astype(np.float32).reshape(Bt, M, N)
    tx, tw = to_torch(rng.f32_to_bf16_bits(x), BFLOAT16), to_torch(rng.f32_to_bf16_bits(w), BFLOAT16)
    c32 = to_storage(hip.gemv(tx, tw, out_dtype=FLOAT32))
    c16 = to_storage(hip.gemv(tx, tw))
    np.testing.assert_array_equal(c32, exact)
    np.testing.assert_array_equal(c16, rng.f32_to_bf16_bits(exact))


def test_gemv_int8_dot_product_at_lds_cap(hip):
    """x[1376,1,16384] @ broadcast W[16384,128] int8 at M = 1 (the dot-product kernel): 1,376 strips,
    2 K-slices of 8,192 rows; int8 and int32 outputs bit-exact."""
    Bt, M, K, N = 1376, 1, 16384, 128
    x = rng.uniform_int(74, Bt * M * K, -128, 127).astype(np.int8).reshape(Bt, M, K)
    w = rng.uniform_int(75, K * N, -128, 127).astype(np.int8).reshape(K, N)
    exact = _exact(x.reshape(Bt * M, K), w).astype(np.int64).reshape(Bt, M, N)
    tx, tw = to_torch(x, INT8), to_torch(w, INT8)
    np.testing.assert_array_equal(to_storage(hip.gemv(tx, tw, out_dtype=INT32)), exact.astype(np.int32))
    np.testing.assert_array_equal(to_storage(hip.gemv(tx, tw)), exact.astype(np.int8))


@pytest.mark.parametrize("entry", ["gemm", "gemv", "noalloc"])
def test_refused_descriptors_leave_c_untouched(hip, entry):
    """Descriptors the C-ABI refuses (a row-expanded output, i.e. two outputs in one element; a
    negative row stride of A; an operand spanning 2^56 bytes) return TV_E_SHAPE before any launch:
    C, filled with a sentinel, is unchanged after the stream has drained.  Real device buffers, so
    a launch that slipped through would write C."""
    M, K, N = 4, 64, 64
    a = to_torch(rng.uniform_int(1, M * K, -3, 3).reshape(M, K).astype(np.float32), FLOAT32)
    b = to_torch(rng.uniform_int(2, K * N, -3, 3).reshape(K, N).astype(np.float32), FLOAT32)
    c = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    fn = {"gemm": tv.lib().tv_hip_gemm, "gemv": tv.lib().tv_hip_gemv, "noalloc": tv.lib().tv_hip_gemm_noalloc}[entry]
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    good = tv.make_args(a, b, c)
    for field, value in (("sc_m", 0), ("sa_m", -K), ("sb_k", 1 << 55)):
        args = tv.make_args(a, b, c)
        setattr(args, field, value)
        if field == "sa_m":
            args.A = a.data_ptr() + (M - 1) * K * 4  # last row first, stepping back: in bounds
        assert fn(ctypes.byref(args), s) == tv.TV_E_SHAPE, field
    torch.cuda.synchronize()
    assert torch.equal(c, torch.full_like(c, 7.0))
    # the unmodified descriptor runs
    assert fn(ctypes.byref(good), s) == tv.TV_OK
    torch.cuda.synchronize()
    want = rng.uniform_int(1, M * K, -3, 3).reshape(M, K).astype(np.float64) @ rng.uniform_int(2, K * N, -3, 3).reshape(K, N)
    np.testing.assert_array_equal(to_storage(c).astype(np.float64), want)
