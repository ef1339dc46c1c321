"""GPU parity with infinite and NaN operands on every float kernel family.  The reference CPU backend
computes in IEEE arithmetic (src/backend/cpu/mul.cpp:27-85), so an output is NaN when one of its
terms is NaN (a NaN operand, or inf x 0) or when it sums +inf and -inf, +-inf when its infinite
terms share a sign, and otherwise the finite sum; none of these outcomes depends on the summation
order.  The kernels zero-fill what lies outside the matrices (tile edges, k past K, padded rows and
columns, x rows past M): those zeros must never meet an infinite operand in a stored output, which
would turn an expected inf into NaN.

Operands are integers in [-3, 3], with about half of A's rows and of B's columns holding one +inf,
-inf or NaN, so outputs of every kind occur and finite outputs are exact sums (rounded once to a half
output).  The expectation is formed in float64 (_ieee_matmul), compared with NaN equal to NaN.
"""
import ctypes

import numpy as np
import pytest
import torch

import tensorvia_amd as tv
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT16, FLOAT32, FLOAT64, to_f32, to_storage, to_torch

pytestmark = pytest.mark.gpu

# (name, dtype, batch, M, K, N, B stored transposed, output dtype or None, entry)
CASES = [
    ("fp32_tiles", FLOAT32, 0, 300, 256, 200, False, None, "gemm"),
    ("fp32_stream_k", FLOAT32, 0, 64, 16384, 64, False, None, "gemm"),
    ("fp32_gemv_dot", FLOAT32, 0, 2, 4096, 3000, False, None, "gemm"),
    ("bf16_256_tiles", BFLOAT16, 0, 512, 512, 520, False, None, "gemm"),
    ("bf16_128_tiles_bt", BFLOAT16, 0, 300, 1000, 264, True, None, "gemm"),
    ("bf16_chained", BFLOAT16, 8, 2048, 256, 2048, False, None, "gemm"),
    ("fp16_small_k", FLOAT16, 16, 1024, 64, 1024, True, None, "gemm"),
    ("bf16_gemv_m1", BFLOAT16, 0, 1, 4096, 4096, False, FLOAT32, "gemv"),
    ("bf16_gemv_m8", BFLOAT16, 0, 8, 4096, 2048, False, FLOAT32, "gemv"),
    ("bf16_gemv_k_contiguous_w", BFLOAT16, 0, 4, 4096, 3000, True, FLOAT32, "gemv"),
    ("bf16_skinny_m24", BFLOAT16, 0, 24, 2048, 1024, False, FLOAT32, "gemm"),
    ("fp16_padded_rows", FLOAT16, 0, 200, 700, 260, False, FLOAT32, "gemm"),
]


def _operand(shape, seed, specials):
    """Integers in [-3, 3] with `specials` elements replaced by +inf, -inf or NaN."""
    x = rng.uniform_int(seed, int(np.prod(shape)), -3, 3).reshape(shape).astype(np.float64)
    r = np.random.default_rng(seed)
    flat = x.reshape(-1)
    idx = r.choice(flat.size, size=specials, replace=False)
    flat[idx] = r.choice([np.inf, -np.inf, np.nan], size=idx.size)
    return x


def _ieee_matmul(x, y):
    """x @ y in IEEE float64 without trusting a BLAS with special values: the finite terms through a
    matmul of the operands with their specials zeroed (exact integer sums), then each special
    element's terms added one by one with numpy's elementwise IEEE arithmetic (inf x 0 = NaN,
    inf + -inf = NaN)."""
    if x.ndim == 3:
        return np.stack([_ieee_matmul(x[i], y[i]) for i in range(x.shape[0])])
    fx, fy = np.isfinite(x), np.isfinite(y)
    out = np.where(fx, x, 0.0) @ np.where(fy, y, 0.0)
    with np.errstate(invalid="ignore"):
        for m, k in zip(*np.nonzero(~fx)):  # a special in A meets all of B's row k
            out[m, :] += x[m, k] * y[k, :]
        for k, n in zip(*np.nonzero(~fy)):  # a special in B meets A's finite column k
            col = fx[:, k]
            out[col, n] += x[col, k] * y[k, n]
    return out


def _enc(x, dt):
    if dt == FLOAT32:
        return x.astype(np.float32)
    if dt == FLOAT64:
        return x
    f = x.astype(np.float32)
    return rng.f32_to_bf16_bits(f) if dt == BFLOAT16 else f.astype(np.float16).view(np.uint16)


def _dev(x, dt, transposed):
    if transposed:
        return to_torch(np.ascontiguousarray(_enc(np.swapaxes(x, -1, -2), dt)), dt).transpose(-1, -2)
    return to_torch(np.ascontiguousarray(_enc(x, dt)), dt)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_inf_and_nan_operands(hip, case):
    name, dt, batch, M, K, N, bt, out_dt, entry = case
    lead = (batch,) if batch else ()
    # about half of A's rows and of B's columns hold one special value: outputs of every kind (a
    # single row of x keeps none; test_inf_in_a_single_row_of_x covers that)
    x = _operand(lead + (M, K), 7 * M + K, max(batch, 1) * M // 2)
    y = _operand(lead + (K, N), 11 * N + K + 1, max(1, max(batch, 1) * N // 2))
    want = _ieee_matmul(x, y)
    ta, tb = _dev(x, dt, False), _dev(y, dt, bt)
    c = (hip.gemv if entry == "gemv" else hip.gemm)(ta, tb, out_dtype=out_dt)
    torch.cuda.synchronize()
    cdt = dt if out_dt is None else out_dt
    got = to_f32(to_storage(c), cdt).astype(np.float64)
    expect = to_f32(_enc(want, cdt), cdt).astype(np.float64)
    assert np.isnan(expect).any() and np.isinf(expect).any() and np.isfinite(expect).any(), name
    np.testing.assert_array_equal(got, expect, err_msg=name)


@pytest.mark.parametrize("entry", ["gemv", "gemm"])
def test_inf_in_a_single_row_of_x(hip, entry):
    """bf16 x[1, 4096] with x[0, 1000] = +inf, finite W[4096, 4096] whose row 1000 holds positive,
    negative and zero values: the GEMV (split over K) gives +inf, -inf and NaN columns in the same
    pattern; tv_hip_gemm routes the call the same way."""
    x = rng.uniform_int(5, 4096, -3, 3).reshape(1, 4096).astype(np.float64)
    y = rng.uniform_int(6, 4096 * 4096, -3, 3).reshape(4096, 4096).astype(np.float64)
    x[0, 1000] = np.inf
    want = _ieee_matmul(x, y)
    assert np.isnan(want).any() and (want == np.inf).any() and (want == -np.inf).any()
    c = (hip.gemv if entry == "gemv" else hip.gemm)(_dev(x, BFLOAT16, False), _dev(y, BFLOAT16, False), out_dtype=FLOAT32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c).astype(np.float64), want)


def test_inf_and_nan_operands_simt(hip):
    """fp32 x fp64 (the SIMT kernel, fp64 result): the same outcomes."""
    x, y = _operand((37, 300), 3, 18), _operand((300, 53), 4, 26)
    want = _ieee_matmul(x, y)
    ta = to_torch(x.astype(np.float32), FLOAT32)
    tb = to_torch(y, FLOAT64)
    c = hip.gemm(ta, tb)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), want)


# (name, dtype, batch, M, K, N, B stored transposed, output dtype or None, entry, scale exponent)
DENORMAL_CASES = [
    ("fp32_tiles", FLOAT32, 0, 300, 512, 200, False, None, "gemm", -70),
    ("fp32_stream_k", FLOAT32, 0, 64, 8192, 64, False, None, "gemm", -70),
    ("fp32_gemv_dot", FLOAT32, 0, 2, 4096, 3000, False, None, "gemm", -70),
    ("bf16_256_tiles_fp32_out", BFLOAT16, 0, 512, 512, 512, False, FLOAT32, "gemm", -70),
    ("bf16_256_tiles_bf16_out", BFLOAT16, 0, 512, 512, 512, False, None, "gemm", -67),
    ("bf16_gemv_m1", BFLOAT16, 0, 1, 4096, 4096, False, FLOAT32, "gemv", -70),
    ("bf16_gemv_m8_k_contiguous_w", BFLOAT16, 0, 8, 4096, 2048, True, FLOAT32, "gemv", -70),
    ("fp16_small_k_fp16_out", FLOAT16, 16, 1024, 64, 1024, True, None, "gemm", -12),
]


@pytest.mark.parametrize("case", DENORMAL_CASES, ids=[c[0] for c in DENORMAL_CASES])
def test_denormal_products_and_sums_exact(hip, case):
    """Operands are small integers times 2^e, normal numbers whose products and sums lie in the
    output's denormal range (fp32: multiples of 2^-140 against a smallest normal of 2^-126; bf16
    output: multiples of 2^-134, rounded to bf16's denormal step of 2^-133; fp16: multiples of 2^-24
    against 2^-14).  Those sums are exact in fp32, so nothing may flush
    them to zero: fp32 outputs equal the exact sums, half outputs the exact sums rounded once, as
    the reference CPU backend's IEEE arithmetic gives them."""
    name, dt, batch, M, K, N, bt, out_dt, entry, e = case
    lead = (batch,) if batch else ()
    x = rng.uniform_int(3 * M + K, int(np.prod(lead + (M, K))), -3, 3).reshape(lead + (M, K)) * 2.0 ** e
    y = rng.uniform_int(5 * N + K, int(np.prod(lead + (K, N))), -3, 3).reshape(lead + (K, N)) * 2.0 ** e
    want = np.matmul(x, y)
    c = (hip.gemv if entry == "gemv" else hip.gemm)(_dev(x, dt, False), _dev(y, dt, bt), out_dtype=out_dt)
    torch.cuda.synchronize()
    cdt = dt if out_dt is None else out_dt
    expect = to_f32(_enc(want, cdt), cdt)
    tiny = np.finfo(np.float16 if cdt == FLOAT16 else np.float32).tiny
    assert ((expect != 0) & (np.abs(expect) < tiny)).mean() > 0.5, name  # mostly denormal outputs
    np.testing.assert_array_equal(to_f32(to_storage(c), cdt), expect, err_msg=name)
