"""GPU parity of the skinny-M (decode) path: x[M<=8, K] @ W[K, N] through tv_hip_gemv, against the
oracle (mul_kernel_basic restated, which is what the reference runs for these shapes), and
9 <= M <= 32 on the matrix-core GEMV through tv_hip_gemm."""
import numpy as np
import pytest
import torch

import oracle as orc
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT16, FLOAT32, INT8, INT32, assert_fp32_close, assert_half_close, to_f32, to_storage, to_torch

pytestmark = pytest.mark.gpu


def half_bits(x, dt):
    return rng.f32_to_bf16_bits(x) if dt == BFLOAT16 else rng.f32_to_f16_bits(x)


@pytest.mark.parametrize("M", [1, 8])
def test_config5_bf16_full_size(hip, M):
    """c5: x[M,4096] N(0,1) @ W[4096,11008] U[-0.05,0.05], bf16, fp32 accumulate, bf16 out."""
    K, N = 4096, 11008
    x = rng.make("normal", (M, K), 9 if M == 1 else 11, "bfloat16")
    w = rng.make("uniform", (K, N), 10, "bfloat16", lo=-0.05, hi=0.05)
    c = to_f32(to_storage(hip.gemv(to_torch(x, BFLOAT16), to_torch(w, BFLOAT16))), BFLOAT16)
    ref = orc.mul(x, BFLOAT16, w, BFLOAT16)
    assert_half_close(c, ref, orc.abs_bound(to_f32(x, BFLOAT16), to_f32(w, BFLOAT16)), K)
    # deterministic split-K reduction: a second call gives identical bits
    c2 = to_f32(to_storage(hip.gemv(to_torch(x, BFLOAT16), to_torch(w, BFLOAT16))), BFLOAT16)
    np.testing.assert_array_equal(c, c2)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, FLOAT32, INT8])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("KN", [(64, 128), (4096, 1008), (1024, 11008), (16, 32), (208, 144), (4000, 1008)])
def test_gemv_integer_inputs_exact(hip, dt, M, KN):
    K, N = KN
    if dt == INT8:
        x = rng.uniform_int(30, M * K, -128, 127).astype(np.int8).reshape(M, K)
        w = rng.uniform_int(31, K * N, -128, 127).astype(np.int8).reshape(K, N)
        c = hip.gemv(to_torch(x, INT8), to_torch(w, INT8))
        c32 = hip.gemv(to_torch(x, INT8), to_torch(w, INT8), out_dtype=INT32)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_storage(c), orc.mul(x, INT8, w, INT8))
        np.testing.assert_array_equal(to_storage(c32), orc.exact_int(x, w).astype(np.int32))
        return
    x = rng.uniform_int(32, M * K, -2, 2).astype(np.float32).reshape(M, K)
    w = rng.uniform_int(33, K * N, -2, 2).astype(np.float32).reshape(K, N)
    if dt == FLOAT32:
        xs, ws = x, w
    else:
        xs, ws = half_bits(x, dt), half_bits(w, dt)
    ref = orc.mul(xs, dt, ws, dt)  # exact: |sum| <= 4K
    c = to_storage(hip.gemv(to_torch(xs, dt), to_torch(ws, dt)))
    want = ref if dt == FLOAT32 else half_bits(ref, dt)
    np.testing.assert_array_equal(c, want)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, INT8])
@pytest.mark.parametrize("M", [9, 16, 17, 32])
@pytest.mark.parametrize("KN", [(4096, 11008), (4000, 1008), (208, 144)])
def test_skinny_m_matrix_core_exact(hip, dt, M, KN):
    """9 <= M <= 32 through tv_hip_gemm: the matrix-core GEMV with 16 or 32 rows of x staged (16-bit
    up to 32 rows, int8 up to 16; int8 at M = 17 and 32 runs the GEMM instead), split over K
    slices or not, ragged K and N.  Integer-valued inputs: exact sums (half outputs rounded once,
    int8 the low byte, and int32 outputs the sums themselves)."""
    K, N = KN
    if dt == INT8:
        x = rng.uniform_int(34, M * K, -128, 127).astype(np.int8).reshape(M, K)
        w = rng.uniform_int(35, K * N, -128, 127).astype(np.int8).reshape(K, N)
        exact = orc.exact_int(x, w)
        c = to_storage(hip.gemm(to_torch(x, INT8), to_torch(w, INT8)))
        c32 = to_storage(hip.gemm(to_torch(x, INT8), to_torch(w, INT8), out_dtype=INT32))
        np.testing.assert_array_equal(c, exact.astype(np.int8))
        np.testing.assert_array_equal(c32, exact.astype(np.int32))
        return
    x = rng.uniform_int(36, M * K, -2, 2).astype(np.float32).reshape(M, K)
    w = rng.uniform_int(37, K * N, -2, 2).astype(np.float32).reshape(K, N)
    c = to_storage(hip.gemm(to_torch(half_bits(x, dt), dt), to_torch(half_bits(w, dt), dt)))
    np.testing.assert_array_equal(c, half_bits(np.matmul(x, w), dt))


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, INT8, FLOAT32])
@pytest.mark.parametrize("M", [1, 3, 8, 9, 16, 17, 32])
@pytest.mark.parametrize("batch,K,N,bcast", [(0, 4096, 11008, False), (0, 4096, 1000, False), (0, 8200, 130, False),
                                             (0, 8208, 130, False), (0, 136, 4104, False), (0, 144, 4104, False),
                                             (3, 1032, 520, True), (2, 4096, 2000, False)],
                         ids=["K4096-N11008", "K4096-N1000", "K8200-N130", "K8208-N130", "K136-N4104", "K144-N4104",
                              "b3-bcast", "b2"])
def test_k_contiguous_w_matrix_core_exact(hip, dt, M, batch, K, N, bcast):
    """x @ W^T with W stored [N, K] (K-contiguous, the linear-layer layout): M <= 16 on the
    matrix-core GEMV that loads W's fragments directly (gemv_kt_kernel: 64-row strips, K split into
    slices of whole 256-byte chunks or not, K = 8208 and 144 ending in a partial chunk, ragged N, 8
    or 16 staged rows of x, batches with one W or per-batch W; K not a multiple of the 16-byte
    vector, fp32, and M = 17 and 32, on the GEMM).  Integer-valued inputs: exact sums, so the half
    outputs are the exact sums rounded once, int8 the low byte, int32 and fp32 the sums; equal to
    the no-allocation entry point."""
    import ctypes
    import tensorvia_amd as tv
    lead = (batch,) if batch else ()
    wshape = (N, K) if (bcast or not batch) else lead + (N, K)
    lo, hi = (-128, 127) if dt == INT8 else (-2, 2)
    x = rng.uniform_int(50 + M, int(np.prod(lead + (M, K))), lo, hi).astype(np.float32).reshape(lead + (M, K))
    w = rng.uniform_int(51, int(np.prod(wshape)), lo, hi).astype(np.float32).reshape(wshape)
    exact = np.matmul(x.astype(np.int64), np.swapaxes(w, -1, -2).astype(np.int64))
    if dt == INT8:
        tx, tw = to_torch(x.astype(np.int8), INT8), to_torch(w.astype(np.int8), INT8)
        wt = tw.transpose(-1, -2)
        c = to_storage(hip.gemm(tx, wt))
        np.testing.assert_array_equal(c, exact.astype(np.int8))
        np.testing.assert_array_equal(to_storage(hip.gemm(tx, wt, out_dtype=INT32)), exact.astype(np.int32))
    elif dt == FLOAT32:
        tx, tw = to_torch(x, FLOAT32), to_torch(w, FLOAT32)
        wt = tw.transpose(-1, -2)
        c = to_storage(hip.gemm(tx, wt))
        np.testing.assert_array_equal(c, exact.astype(np.float32))
    else:
        tx, tw = to_torch(half_bits(x, dt), dt), to_torch(half_bits(w, dt), dt)
        wt = tw.transpose(-1, -2)
        c = to_storage(hip.gemm(tx, wt))
        np.testing.assert_array_equal(c, half_bits(exact.astype(np.float32), dt))
    plain = torch.zeros(lead + (M, N), dtype=tx.dtype, device="cuda")
    args = tv.make_args(tx, wt, plain)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), c)


@pytest.mark.parametrize("dt,M,K,N", [(BFLOAT16, 1, 4096, 14336), (BFLOAT16, 8, 8192, 28672), (INT8, 8, 8192, 28672),
                                      (BFLOAT16, 1, 2048, 32768)])
def test_gemv_large_w_slice_choice_exact(hip, dt, M, K, N):
    """W shapes whose K-slice count comes from the occupancy rule rather than the 688 / 344
    workgroup target (224, 448 and 512 strips): integer-valued inputs, exact sums, bit-exact
    against exact integer sums (fp32 output for bf16: |sum| <= 4K < 2^24)."""
    if dt == INT8:
        x = rng.uniform_int(40, M * K, -128, 127).astype(np.int8).reshape(M, K)
        w = rng.uniform_int(41, K * N, -128, 127).astype(np.int8).reshape(K, N)
        c32 = hip.gemv(to_torch(x, INT8), to_torch(w, INT8), out_dtype=INT32)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_storage(c32), orc.exact_int(x, w).astype(np.int32))
        return
    x = rng.uniform_int(42, M * K, -2, 2).astype(np.float32).reshape(M, K)
    w = rng.uniform_int(43, K * N, -2, 2).astype(np.float32).reshape(K, N)
    c = to_storage(hip.gemv(to_torch(half_bits(x, dt), dt), to_torch(half_bits(w, dt), dt), out_dtype=FLOAT32))
    np.testing.assert_array_equal(c, (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT32])
def test_gemv_uniform_vs_oracle(hip, dt):
    M, K, N = 4, 2048, 3000
    x = rng.normal_f32(40, M * K).reshape(M, K)
    w = rng.uniform_f32(41, K * N, -0.05, 0.05).reshape(K, N)
    xs, ws = (x, w) if dt == FLOAT32 else (half_bits(x, dt), half_bits(w, dt))
    ref = orc.mul(xs, dt, ws, dt)
    c = to_f32(to_storage(hip.gemv(to_torch(xs, dt), to_torch(ws, dt))), dt)
    bound = orc.abs_bound(to_f32(xs, dt), to_f32(ws, dt))
    (assert_fp32_close if dt == FLOAT32 else assert_half_close)(c, ref, bound, K)


# 16-bit W with N >= 64 runs on the matrix-core kernel, narrower W on the dot-product kernel
@pytest.mark.parametrize("M,N", [(2, 40), (6, 264)], ids=["dot", "mfma"])
def test_gemv_batched_and_broadcast(hip, M, N):
    Bt, K = 3, 520
    x = rng.uniform_int(42, Bt * M * K, -2, 2).astype(np.float32).reshape(Bt, M, K)
    w = rng.uniform_int(43, K * N, -2, 2).astype(np.float32).reshape(K, N)
    xb, wb = rng.f32_to_bf16_bits(x), rng.f32_to_bf16_bits(w)
    c = to_storage(hip.gemv(to_torch(xb, BFLOAT16), to_torch(wb, BFLOAT16)))
    ref = orc.mul(xb.reshape(Bt * M, K), BFLOAT16, wb, BFLOAT16).reshape(Bt, M, N)
    np.testing.assert_array_equal(c, rng.f32_to_bf16_bits(ref))
    w3 = np.stack([w, -w, 2 * w])
    c3 = to_storage(hip.gemv(to_torch(xb, BFLOAT16), to_torch(rng.f32_to_bf16_bits(w3), BFLOAT16)))
    ref3 = orc.mul(xb, BFLOAT16, rng.f32_to_bf16_bits(w3), BFLOAT16)
    np.testing.assert_array_equal(c3, rng.f32_to_bf16_bits(ref3))


def test_gemv_int8_batched_and_broadcast_matrix_core(hip):
    """int8 at M >= 3 with N >= 128 runs on the matrix-core kernel: per-batch and broadcast W,
    int8 (low byte) and int32 outputs, bit-exact."""
    Bt, M, K, N = 3, 4, 1088, 272
    x = rng.uniform_int(46, Bt * M * K, -128, 127).astype(np.int8).reshape(Bt, M, K)
    w3 = rng.uniform_int(47, Bt * K * N, -128, 127).astype(np.int8).reshape(Bt, K, N)
    for w in (w3, w3[1]):
        c = hip.gemv(to_torch(x, INT8), to_torch(np.ascontiguousarray(w), INT8))
        c32 = hip.gemv(to_torch(x, INT8), to_torch(np.ascontiguousarray(w), INT8), out_dtype=INT32)
        torch.cuda.synchronize()
        exact = np.stack([orc.exact_int(x[i], w[i] if w.ndim == 3 else w) for i in range(Bt)])
        np.testing.assert_array_equal(to_storage(c32), exact.astype(np.int32))
        np.testing.assert_array_equal(to_storage(c), exact.astype(np.int8))


def test_gemv_unsupported_layouts_report_and_gemm_serves_them(hip):
    K, N = 256, 64
    x = rng.uniform_int(44, K, -2, 2).astype(np.float32).reshape(1, K)
    w = rng.uniform_int(45, K * N, -2, 2).astype(np.float32).reshape(K, N)
    # K-contiguous W (x @ W^T with W stored [N, K]) is served by tv_hip_gemv itself at 16 bits ...
    wt16 = to_torch(half_bits(np.ascontiguousarray(w.T), BFLOAT16), BFLOAT16).t()
    c16 = hip.gemv(to_torch(half_bits(x, BFLOAT16), BFLOAT16), wt16, out_dtype=FLOAT32)
    np.testing.assert_array_equal(to_storage(c16), orc.mul(x, FLOAT32, w, FLOAT32))
    # ... but not in fp32 (the GEMM serves it), nor W contiguous along neither dimension (every
    # other column of a [K, 2N] array)
    wt = to_torch(np.ascontiguousarray(w.T), FLOAT32).t()
    with pytest.raises(hip.TensorviaHipError) as e:
        hip.gemv(to_torch(x, FLOAT32), wt)
    assert e.value.code == hip.TV_E_UNSUPPORTED
    np.testing.assert_array_equal(to_storage(hip.gemm(to_torch(x, FLOAT32), wt)), orc.mul(x, FLOAT32, w, FLOAT32))
    w2 = np.zeros((K, 2 * N), np.float32)
    w2[:, ::2] = w
    wg = to_torch(w2, FLOAT32)[:, ::2]
    with pytest.raises(hip.TensorviaHipError) as e:
        hip.gemv(to_torch(x, FLOAT32), wg)
    assert e.value.code == hip.TV_E_UNSUPPORTED
    c = to_storage(hip.gemm(to_torch(x, FLOAT32), wg))
    np.testing.assert_array_equal(c, orc.mul(x, FLOAT32, w, FLOAT32))
    with pytest.raises(hip.TensorviaHipError):
        hip.gemv(to_torch(np.zeros((9, K), np.float32), FLOAT32), to_torch(w, FLOAT32))
