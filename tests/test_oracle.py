"""Pins the CPU oracle (oracle/mul_oracle.cpp) before it is trusted as the parity checker.

Each check is chosen so a plausible restatement mistake (dropped chunk, transposed operand, wrong
accumulator type, wrong widening) fails it: exact int64 brute force, closed forms, exactly
representable fp32 sums, numpy's independent fp16 conversion and transpose.
"""
import numpy as np
import pytest

import oracle as orc
from oracle import BFLOAT16, FLOAT16, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64
from tensorvia_amd import rng


def _ri(seed, shape, lo, hi, dt):
    return rng.uniform_int(seed, int(np.prod(shape)), lo, hi).astype(dt).reshape(shape)


@pytest.mark.parametrize("variant", [0, 1, 2])
@pytest.mark.parametrize("shape", [(37, 129, 53), (64, 64, 64), (1, 300, 7), (65, 1, 66)])
def test_int8_low_byte_of_exact_sum(shape, variant):
    M, K, N = shape
    a = _ri(1, (M, K), -128, 127, np.int8)
    b = _ri(2, (K, N), -128, 127, np.int8)
    c = orc.mul(a, INT8, b, INT8, variant=variant)
    assert c.dtype == np.int8
    np.testing.assert_array_equal(c, orc.low_byte(orc.exact_int(a, b)))


def test_int8_tiled_is_chosen_at_2pow20_and_matches():
    # batch*M*N = 2^20 selects the tiled kernel (mul.cpp:87-96); K spans 3 chunks of 64 plus a tail.
    a = _ri(3, (1024, 200), -10, 10, np.int8)
    b = _ri(4, (200, 1024), -10, 10, np.int8)
    c = orc.mul(a, INT8, b, INT8)
    np.testing.assert_array_equal(c, orc.low_byte(orc.exact_int(a, b)))


@pytest.mark.parametrize("variant", [1, 2])
def test_int8_known_answers(variant):
    ones = np.ones((8, 4096), np.int8)
    assert not orc.mul(ones, INT8, ones.T.copy(), INT8, variant=variant).any()  # 4096 mod 256 = 0
    k = 3
    a = np.full((5, k), 127, np.int8)
    b = np.full((k, 6), 127, np.int8)
    # 3 * 127 * 127 = 48387 = 189 * 256 + 3
    assert (orc.mul(a, INT8, b, INT8, variant=variant) == 3).all()
    a = np.full((4, 2), -128, np.int8)
    b = np.full((2, 4), -128, np.int8)
    assert (orc.mul(a, INT8, b, INT8, variant=variant) == 0).all()  # 2 * 16384 = 32768 -> low byte 0
    eye = np.eye(70, dtype=np.int8)
    b = _ri(5, (70, 33), -128, 127, np.int8)
    np.testing.assert_array_equal(orc.mul(eye, INT8, b, INT8, variant=variant), b)


@pytest.mark.parametrize("variant", [1, 2])
def test_int8_batched(variant):
    a = _ri(6, (3, 20, 70), -128, 127, np.int8)
    b = _ri(7, (3, 70, 33), -128, 127, np.int8)
    c = orc.mul(a, INT8, b, INT8, variant=variant)
    for i in range(3):
        np.testing.assert_array_equal(c[i], orc.low_byte(orc.exact_int(a[i], b[i])))


@pytest.mark.parametrize("variant", [1, 2])
@pytest.mark.parametrize("shape", [(45, 77, 61), (128, 200, 96)])
def test_fp32_integer_inputs_are_exact(shape, variant):
    # |partial sums| <= 64*K < 2^24: every fp32 operation is exact, whatever the order or FMA use.
    M, K, N = shape
    a = _ri(8, (M, K), -8, 8, np.float32)
    b = _ri(9, (K, N), -8, 8, np.float32)
    c = orc.mul(a, FLOAT32, b, FLOAT32, variant=variant)
    assert c.dtype == np.float32
    np.testing.assert_array_equal(c, orc.f64_matmul(a, b).astype(np.float32))


@pytest.mark.parametrize("variant", [1, 2])
def test_fp32_uniform_within_tolerance(variant):
    M, K, N = 64, 2048, 48
    a = rng.uniform_f32(10, M * K, -1, 1).reshape(M, K)
    b = rng.uniform_f32(11, K * N, -1, 1).reshape(K, N)
    c = orc.mul(a, FLOAT32, b, FLOAT32, variant=variant).astype(np.float64)
    err = np.abs(c - orc.f64_matmul(a, b)) / orc.abs_bound(a, b)
    assert err.max() <= 1e-5 * np.sqrt(K)


def test_fp32_chunks_all_counted():
    # K = 130 = 64 + 64 + 2: a dropped chunk or a chunk counted twice changes the sum.
    a = np.ones((1100, 130), np.float32)
    b = np.ones((130, 1000), np.float32)
    c = orc.mul(a, FLOAT32, b, FLOAT32, variant=2)
    assert (c == 130).all()


def test_bf16_inputs_widen_exactly_and_return_fp32():
    x = _ri(12, (33, 40), -4, 4, np.float32)
    y = _ri(13, (40, 21), -4, 4, np.float32)
    xb, yb = rng.f32_to_bf16_bits(x), rng.f32_to_bf16_bits(y)
    c = orc.mul(xb, BFLOAT16, yb, BFLOAT16)
    assert c.dtype == np.float32  # CPU widens half types (mul.cpp:110-112)
    np.testing.assert_array_equal(c, orc.f64_matmul(x, y).astype(np.float32))


def test_fp16_inputs_widen_exactly():
    x = _ri(14, (17, 50), -6, 6, np.float32)
    y = _ri(15, (50, 9), -6, 6, np.float32)
    c = orc.mul(rng.f32_to_f16_bits(x), FLOAT16, rng.f32_to_f16_bits(y), FLOAT16)
    np.testing.assert_array_equal(c, orc.f64_matmul(x, y).astype(np.float32))


def test_widen_fp16_all_bit_patterns_match_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = orc.widen_f32(bits, FLOAT16)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.isnan(ours[nan]).all()
    np.testing.assert_array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_widen_bf16_known_values():
    bits = np.array([0x3F80, 0xBF80, 0x7F80, 0xFF80, 0x0000, 0x8000, 0x0001, 0x4049], np.uint16)
    expect = np.array([1.0, -1.0, np.inf, -np.inf, 0.0, -0.0, 2.0 ** -133, 3.140625], np.float32)
    np.testing.assert_array_equal(orc.widen_f32(bits, BFLOAT16), expect)


def test_transpose_matches_numpy():
    x = _ri(16, (3, 70, 131), -100, 100, np.int16)
    np.testing.assert_array_equal(orc.transpose_last2(x), x.transpose(0, 2, 1))
    y = rng.uniform_f32(17, 65 * 9, -1, 1).reshape(65, 9)
    np.testing.assert_array_equal(orc.transpose_last2(y), y.T)


def test_result_type_rules():
    # include/core/type_traits.h:270-287 (the code, not the comments above it) after widening.
    assert orc.result_type(INT8, INT8) == INT8
    assert orc.result_type(INT8, INT16) == INT16
    assert orc.result_type(INT64, INT32) == INT64
    assert orc.result_type(BFLOAT16, BFLOAT16) == FLOAT32
    assert orc.result_type(FLOAT16, FLOAT32) == FLOAT32
    assert orc.result_type(INT64, FLOAT32) == FLOAT64
    assert orc.result_type(INT32, FLOAT16) == FLOAT32
    assert orc.result_type(INT8, FLOAT64) == FLOAT64
    assert orc.compute_type(BFLOAT16, BFLOAT16) == BFLOAT16
    assert orc.compute_type(FLOAT16, BFLOAT16) == FLOAT32
    assert orc.compute_type(INT16, BFLOAT16) == FLOAT32


def test_mixed_int_tiled_chunk_wraps_in_a_type():
    # Tiled: each 64-chunk is summed in A's type (int8 here) with B converted to int8, then added
    # into the int16 result (mul.cpp:64-78).  Basic: exact int sum cast to int16 (mul.cpp:13-21).
    a = np.full((1024, 64), 100, np.int8)
    b = np.full((64, 1024), 1, np.int16)
    tiled = orc.mul(a, INT8, b, INT16)  # 2^20 outputs -> tiled
    assert tiled.dtype == np.int16
    assert (tiled == 0).all()  # 6400 mod 256 = 0 inside the int8 chunk sum
    basic = orc.mul(a, INT8, b, INT16, variant=1)
    assert (basic == 6400).all()
    b300 = np.full((64, 1024), 300, np.int16)  # (int8)300 = 44 in the tiled chunk
    t = orc.mul(np.ones((1024, 64), np.int8), INT8, b300, INT16)
    assert (t == ((64 * 44) & 0xFF if (64 * 44) & 0xFF < 128 else ((64 * 44) & 0xFF) - 256)).all()


def test_threads_capped_at_16():
    a = np.ones((4, 4), np.float32)
    orc.mul(a, FLOAT32, a, FLOAT32)
    assert 1 <= orc.threads_used() <= 16


def test_fp64_and_int32_paths():
    a = _ri(18, (20, 30), -1000, 1000, np.int32)
    b = _ri(19, (30, 10), -1000, 1000, np.int32)
    np.testing.assert_array_equal(orc.mul(a, INT32, b, INT32), orc.exact_int(a, b).astype(np.int32))
    x = rng.uniform_f32(20, 600, -1, 1).astype(np.float64).reshape(20, 30)
    y = rng.uniform_f32(21, 300, -1, 1).astype(np.float64).reshape(30, 10)
    np.testing.assert_allclose(orc.mul(x, FLOAT64, y, FLOAT64), x @ y, rtol=0, atol=1e-12)
    z = orc.mul(a, INT32, y.astype(np.float32), FLOAT32, variant=1)
    assert z.dtype == np.float32
