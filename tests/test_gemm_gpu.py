"""GPU parity: the HIP kernels (through the C-ABI) against the CPU oracle and brute force.

Bars: int8 bit-exact (low byte of the exact sum, or the full int32 sum); fp32 within
1e-5*sqrt(K) relative to sum_k |a||b|; bf16/fp16 within 1e-2 of the fp32-accumulated value (plus the
fp32 accumulation allowance); integer-valued float inputs, whose sums every accumulation order
reproduces exactly, bit-exact.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as orc
import tensorvia_amd as tv
from tensorvia_amd import rng
from tests import golden
from tests.util import (BFLOAT16, FLOAT16, FLOAT32, INT8, INT32, assert_fp32_close, assert_half_close,
                        to_f32, to_storage, to_torch)

pytestmark = pytest.mark.gpu


def ints(seed, shape, lo, hi, dt=np.float32):
    return rng.uniform_int(seed, int(np.prod(shape)), lo, hi).astype(dt).reshape(shape)


def half_bits(x, dt):
    return rng.f32_to_bf16_bits(x) if dt == BFLOAT16 else rng.f32_to_f16_bits(x)


# ---- golden vectors -------------------------------------------------------------------------

@pytest.mark.parametrize("name", sorted(golden.load()))
def test_golden_bit_exact(hip, name):
    case = golden.load()[name]
    dta, dtb, dtc, layout = (int(v) for v in case["meta"])
    a = to_torch(case["a"], dta)
    b = to_torch(case["b"], dtb)
    if layout == 1:
        b = b.permute(0, 2, 1)  # strided view, consumed without a repack
    c = hip.gemm(a, b, out_dtype=dtc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), case["c"])


# ---- int8 -----------------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(37, 129, 53), (256, 256, 256), (300, 130, 517), (16, 4096, 16),
                                   (257, 64, 255), (9, 16, 9), (1000, 2000, 300)])
def test_int8_vs_oracle_bit_exact(hip, shape):
    M, K, N = shape
    a = ints(1, (M, K), -128, 127, np.int8)
    b = ints(2, (K, N), -128, 127, np.int8)
    c = hip.gemm(to_torch(a, INT8), to_torch(b, INT8))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), orc.mul(a, INT8, b, INT8))


@pytest.mark.parametrize("batch,M,K,N,pad", [(0, 300, 200, 272, 0), (0, 300, 200, 260, 28), (2, 270, 136, 500, 12)])
def test_int8_tile_store_ragged_and_padded(hip, batch, M, K, N, pad):
    """int8 output with 16-byte aligned rows leaves as whole 256-byte tile rows staged through LDS:
    ragged tiles in M and N, N not a multiple of 16 inside rows padded to a multiple of 16 bytes
    (the last chunk of a row is written byte by byte), batched outputs.  Bit-exact against the
    oracle, and the padding bytes are not written."""
    lead = (batch,) if batch else ()
    a = ints(31, lead + (M, K), -128, 127, np.int8)
    b = ints(32, (K, N), -128, 127, np.int8)
    big = torch.full(lead + (M, N + pad), 77, dtype=torch.int8, device="cuda")
    c = big[..., :N]
    hip.gemm(to_torch(a, INT8), to_torch(b, INT8), out=c)
    torch.cuda.synchronize()
    want = np.stack([orc.mul(a[i], INT8, b, INT8) for i in range(batch)]) if batch else orc.mul(a, INT8, b, INT8)
    np.testing.assert_array_equal(to_storage(c), want)
    if pad:
        assert bool((big[..., N:] == 77).all()), "the tile store wrote past column N"


def test_int8_int32_output(hip):
    a = ints(3, (200, 333), -128, 127, np.int8)
    b = ints(4, (333, 150), -128, 127, np.int8)
    c = hip.gemm(to_torch(a, INT8), to_torch(b, INT8), out_dtype=INT32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), orc.exact_int(a, b).astype(np.int32))


def test_int8_known_answers(hip):
    ones = torch.ones((300, 4096), dtype=torch.int8, device="cuda")
    c = hip.gemm(ones, ones.t())  # K = 4096 -> 4096 mod 256 = 0; B is an N-contiguous... transposed view
    torch.cuda.synchronize()
    assert not c.any().item()
    eye = torch.eye(260, dtype=torch.int8, device="cuda")
    b = to_torch(ints(5, (260, 190), -128, 127, np.int8), INT8)
    c = hip.gemm(eye, b)
    torch.cuda.synchronize()
    assert torch.equal(c, b)


def test_int8_config2_full_size_sampled(hip):
    """c2: int8 [4096,4096] @ [4096,4096], uniform ints in [-10,10]; 128 sampled rows and columns
    against exact int64 sums, plus the full row/column checksum identity mod 256."""
    n = 4096
    a = ints(3, (n, n), -10, 10, np.int8)
    b = ints(4, (n, n), -10, 10, np.int8)
    c = to_storage(hip.gemm(to_torch(a, INT8), to_torch(b, INT8)))
    r = np.random.default_rng(0)
    rows = r.choice(n, 128, replace=False)
    cols = r.choice(n, 128, replace=False)
    np.testing.assert_array_equal(c[rows], orc.low_byte(orc.exact_int(a[rows], b)))
    np.testing.assert_array_equal(c[:, cols], orc.low_byte(orc.exact_int(a, b[:, cols])))
    # checksum of checksums: sum_ij C_ij == (1^T A)(B 1) mod 256 for the exact sums
    lhs = int(c.astype(np.int64).sum()) % 256
    rhs = int((a.astype(np.int64).sum(0) * b.astype(np.int64).sum(1)).sum()) % 256
    assert lhs == rhs


# ---- fp32 -----------------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(45, 77, 61), (128, 128, 128), (2592 // 8, 2048 // 8, 4096 // 8), (129, 257, 65)])
def test_fp32_integer_inputs_bit_exact(hip, shape):
    M, K, N = shape
    a = ints(6, (M, K), -8, 8)
    b = ints(7, (K, N), -8, 8)
    c = hip.gemm(to_torch(a, FLOAT32), to_torch(b, FLOAT32))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), orc.mul(a, FLOAT32, b, FLOAT32))


@pytest.mark.parametrize("shape", [(300, 512, 200), (64, 2048, 96)])
def test_fp32_uniform_vs_oracle(hip, shape):
    M, K, N = shape
    a = rng.uniform_f32(8, M * K, -1, 1).reshape(M, K)
    b = rng.uniform_f32(9, K * N, -1, 1).reshape(K, N)
    c = to_storage(hip.gemm(to_torch(a, FLOAT32), to_torch(b, FLOAT32)))
    assert_fp32_close(c, orc.mul(a, FLOAT32, b, FLOAT32), orc.abs_bound(a, b), K)


@pytest.mark.parametrize("batch,M,K,N", [(0, 2592, 2048, 4096), (0, 1300, 1024, 4100), (2, 1000, 1056, 2100),
                                         (0, 1700, 1056, 2900), (0, 300, 264, 500), (0, 4096, 1024, 4096),
                                         (0, 4400, 1024, 4096)])
def test_fp32_stream_k_bit_exact(hip, batch, M, K, N):
    """fp32 GEMMs on the stream-K schedule, whose tiles are summed in segments by several
    workgroups: c1 (864 tiles of 96x128, 3.375 per CU: one round of whole tiles, then 352 split);
    462 (96x128), 272 (128x128) and 414 (96x128) tiles with ragged M/N tails and a batch (K of 32 and
    33 k-tiles); 12 tiles at K = 9 k-tiles (fewer tiles than CUs); 1024 tiles (two whole rounds,
    nothing split) and 1120 (two rounds, then 96 tiles split over fewer workgroups than are resident).  Integer-valued
    inputs make every order exact: bit-exact against exact sums, equal to the plain kernel
    (tv_hip_gemm_noalloc takes no workspace, hence no stream-K), and equal on a second call."""
    lead = (batch,) if batch else ()
    a = ints(12, lead + (M, K), -3, 3)
    b = ints(13, (K, N), -3, 3)
    ta, tb = to_torch(a, FLOAT32), to_torch(b, FLOAT32)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    c = to_storage(hip.gemm(ta, tb))
    np.testing.assert_array_equal(c, want)
    np.testing.assert_array_equal(to_storage(hip.gemm(ta, tb)), c)
    plain = torch.zeros(lead + (M, N), dtype=torch.float32, device="cuda")
    args = tv.make_args(ta, tb, plain)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), c)


@pytest.mark.parametrize("batch,M,K,N,tile", [
    (0, 2000, 300, 2050, "128x128"), (0, 300, 264, 4096, "64x128"), (0, 4096, 200, 192, "128x64"),
    (8, 1000, 264, 129, "128x64"), (0, 3000, 200, 129, "128x32"), (0, 3000, 4096, 129, "128x32"),
    (0, 8192, 264, 32, "128x32"), (2, 3000, 520, 96, "128x32"), (0, 300, 520, 1000, "32x128"),
    (3, 90, 136, 500, "32x128"), (0, 300, 4096, 1000, "32x128"), (0, 960, 264, 2000, "96x128"),
    (0, 1340, 4096, 2100, "96x128"), (2, 1300, 520, 700, "96x128"), (3, 1700, 136, 600, "96x128")])
def test_fp32_tile_choice_exact(hip, batch, M, K, N, tile):
    """fp32 GEMMs that the tile cost rule (padded work over tile rate and CU fill) sends to each of
    the six fp32 tiles named, with ragged M/N edges, batches, and K = 4096 (the stream-K schedule
    on 120, 80 and 238 tiles).  Integer-valued inputs make every order exact: bit-exact against exact
    sums, and equal to the plain kernel (tv_hip_gemm_noalloc: no workspace, no stream-K)."""
    lead = (batch,) if batch else ()
    a = ints(31, lead + (M, K), -3, 3)
    b = ints(32, lead + (K, N), -3, 3)
    ta, tb = to_torch(a, FLOAT32), to_torch(b, FLOAT32)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    c = to_storage(hip.gemm(ta, tb))
    np.testing.assert_array_equal(c, want)
    plain = torch.zeros(lead + (M, N), dtype=torch.float32, device="cuda")
    args = tv.make_args(ta, tb, plain)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), c)


@pytest.mark.parametrize("M,K,N", [(2592, 520, 1000), (1340, 264, 2100), (960, 4096, 2000)])
def test_fp32_96_row_tile_k_contiguous_b_exact(hip, M, K, N):
    """The 96x128 fp32 tile with B stored [N, K] and used transposed (k-contiguous B), ragged and
    whole row counts, the last on the stream-K schedule (K = 4096): bit-exact on integer-valued
    inputs, equal to the plain kernel (tv_hip_gemm_noalloc)."""
    a = ints(41, (M, K), -3, 3)
    w = ints(42, (N, K), -3, 3)
    ta, tw = to_torch(a, FLOAT32), to_torch(w, FLOAT32)
    want = np.matmul(a.astype(np.float64), w.T.astype(np.float64)).astype(np.float32)
    c = to_storage(hip.gemm(ta, tw.t()))
    np.testing.assert_array_equal(c, want)
    plain = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    args = tv.make_args(ta, tw.t(), plain)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), c)


@pytest.mark.parametrize("batch,M,K,N,a_t,b_t,cpad", [
    (0, 4096, 128, 4096, False, False, 0), (0, 4096, 100, 4096, False, True, 0), (2, 2048, 96, 4096, False, False, 0),
    (0, 4096, 136, 4096, False, False, 3), (0, 8192, 40, 8192, False, True, 0), (0, 4096, 64, 4096, True, False, 0),
    (2, 4096, 72, 2048, True, True, 0)])
def test_fp32_256_tile_whole_rounds_exact(hip, batch, M, K, N, a_t, b_t, cpad):
    """fp32 shapes whose 256x256 tiles fill whole rounds of the CUs (256 or 1,024 tiles) take the
    256x256 tile: row-major and transposed A and B, a ragged K, batches, and C inside wider rows
    (the unstaged stores).  Integer-valued inputs: bit-exact against exact sums, equal to the plain
    kernel (tv_hip_gemm_noalloc), and the fused epilogue (a column bias, then a full [M, N] bias,
    each with relu) equal to the exact composition."""
    lead = (batch,) if batch else ()
    a = ints(51, lead + (M, K), -3, 3)
    b = ints(52, lead + (K, N), -3, 3)
    ta = to_torch(np.ascontiguousarray(np.swapaxes(a, -1, -2)), FLOAT32).transpose(-1, -2) if a_t else to_torch(a, FLOAT32)
    tb = to_torch(np.ascontiguousarray(np.swapaxes(b, -1, -2)), FLOAT32).transpose(-1, -2) if b_t else to_torch(b, FLOAT32)
    want = np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    wide = torch.full(lead + (M, N + cpad), 9.0, dtype=torch.float32, device="cuda")
    c = wide[..., :N]
    hip.gemm(ta, tb, out=c)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c.contiguous()), want)
    if cpad:
        assert bool((wide[..., N:] == 9.0).all())
    plain = torch.zeros(lead + (M, N), dtype=torch.float32, device="cuda")
    args = tv.make_args(ta, tb, plain)
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), sh))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), want)
    bias = ints(53, (N,), -40, 40).astype(np.float32)
    tbias = to_torch(bias, FLOAT32)
    ep = tv.TvEpilogue()
    ep.act, ep.reserved, ep.bias, ep.sbias_b, ep.sbias_m, ep.sbias_n = tv.ACT_RELU, 0, tbias.data_ptr(), 0, 0, 1
    fused = torch.zeros(lead + (M, N), dtype=torch.float32, device="cuda")
    args = tv.make_args(ta, tb, fused)
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), sh))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(fused), np.maximum(want + bias, 0).astype(np.float32))
    # a full [M, N] bias, shared by the batch (batch stride 0)
    full = ints(54, (M, N), -40, 40).astype(np.float32)
    tfull = to_torch(full, FLOAT32)
    ep.bias, ep.sbias_b, ep.sbias_m, ep.sbias_n = tfull.data_ptr(), 0, N, 1
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), sh))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(fused), np.maximum(want + full, 0).astype(np.float32))


@pytest.mark.parametrize("dt", [FLOAT32, BFLOAT16, INT8], ids=["fp32", "bf16", "int8"])
@pytest.mark.parametrize("case", ["n1", "k1", "m1", "b1_k1_bcast", "b1_n1_at"])
def test_unit_extent_strides(hip, dt, case):
    """Operands with a dimension of extent 1 whose stride is smaller than the row it does not step
    over, as torch lays out [K, 1] or [M, 1] (strides (1, 1)): B = W[K, 1] (N = 1), A[M, 1] @ B[1, N]
    (K = 1), A[1, K] as a transposed view of [K, 1] storage (M = 1, on the GEMM: B k-contiguous),
    and the same in 3-d with batch 1.  A loader that sized its buffer range from such a stride cut
    the row short (the elements past the cut read as zeros).  Integer-valued inputs: bit-exact."""
    def enc(x):
        if dt == INT8:
            return x.astype(np.int8)
        return half_bits(x.astype(np.float32), dt) if dt == BFLOAT16 else x.astype(np.float32)

    if case == "n1":
        x, y = ints(51, (300, 708), -3, 3), ints(52, (708, 1), -3, 3)
        ta, tb = to_torch(enc(x), dt), to_torch(enc(y), dt)
    elif case == "k1":
        x, y = ints(53, (256, 1), -3, 3), ints(54, (1, 300), -3, 3)
        ta, tb = to_torch(enc(x), dt), to_torch(enc(y), dt)
    elif case == "m1":
        x, w = ints(55, (708, 1), -3, 3), ints(56, (300, 708), -3, 3)
        ta = to_torch(enc(x), dt).t()          # [1, 708], strides (1, 1)
        tb = to_torch(enc(w), dt).t()          # [708, 300], k-contiguous
        x, y = x.T, w.T
    elif case == "b1_k1_bcast":
        x, y = ints(57, (1, 20, 1), -3, 3), ints(58, (1, 3), -3, 3)
        ta, tb = to_torch(enc(x), dt), to_torch(enc(y), dt)
    else:
        xs, y = ints(59, (1, 708, 17), -3, 3), ints(60, (708, 1), -3, 3)
        ta = to_torch(enc(xs), dt).transpose(-1, -2)  # [1, 17, 708], m-contiguous
        tb = to_torch(enc(y), dt)[None]              # [1, 708, 1]
        x, y = np.swapaxes(xs, -1, -2), y[None]
    s64 = np.matmul(x.astype(np.float64), y.astype(np.float64))
    want = s64.astype(np.int64).astype(np.int8) if dt == INT8 else enc(s64)
    c = hip.gemm(ta, tb)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), want)


def test_fp32_config1_full_size_sampled(hip):
    """c1: fp32 [2592,2048] @ [2048,4096] U[-1,1]: sampled rows/columns against fp64 sums."""
    M, K, N = 2592, 2048, 4096
    a = rng.uniform_f32(1, M * K, -1, 1).reshape(M, K)
    b = rng.uniform_f32(2, K * N, -1, 1).reshape(K, N)
    c = to_storage(hip.gemm(to_torch(a, FLOAT32), to_torch(b, FLOAT32)))
    r = np.random.default_rng(1)
    rows = r.choice(M, 64, replace=False)
    cols = r.choice(N, 64, replace=False)
    assert_fp32_close(c[rows], orc.f64_matmul(a[rows], b), orc.abs_bound(a[rows], b), K)
    assert_fp32_close(c[:, cols], orc.f64_matmul(a, b[:, cols]), orc.abs_bound(a, b[:, cols]), K)


# ---- bf16 / fp16 ----------------------------------------------------------------------------

@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16])
@pytest.mark.parametrize("shape", [(33, 40, 72), (256, 512, 256), (300, 200, 136)])
def test_half_integer_inputs_bit_exact(hip, dt, shape):
    M, K, N = shape
    x = ints(10, (M, K), -3, 3)
    y = ints(11, (K, N), -3, 3)
    ref = orc.mul(half_bits(x, dt), dt, half_bits(y, dt), dt)  # exact fp32 sums
    c = hip.gemm(to_torch(half_bits(x, dt), dt), to_torch(half_bits(y, dt), dt))
    c32 = hip.gemm(to_torch(half_bits(x, dt), dt), to_torch(half_bits(y, dt), dt), out_dtype=FLOAT32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), half_bits(ref, dt))
    np.testing.assert_array_equal(to_storage(c32), ref)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16])
def test_half_uniform_vs_oracle(hip, dt):
    M, K, N = 200, 1024, 328
    x = half_bits(rng.uniform_f32(12, M * K, -1, 1), dt).reshape(M, K)
    y = half_bits(rng.uniform_f32(13, K * N, -1, 1), dt).reshape(K, N)
    ref = orc.mul(x, dt, y, dt)
    c = to_f32(to_storage(hip.gemm(to_torch(x, dt), to_torch(y, dt))), dt)
    assert_half_close(c, ref, orc.abs_bound(to_f32(x, dt), to_f32(y, dt)), K)


def test_bf16_config3_full_size_broadcast_equals_flattened(hip):
    """c3 at its configured size: A[16,2048,4096] @ B[4096,4096] (B broadcast, batch stride 0; 2,048
    output tiles) equals the flattened call [32768,4096] @ [4096,4096] bit for bit (the reference
    rejects the broadcast form, so the flattened 2-d call is what it computes, mul.cpp:97-145), and
    48 sampled rows, 3 in each of the 16 batches, match the oracle under the bf16 bar."""
    Bt, M, K, N = 16, 2048, 4096, 4096
    a = rng.make("uniform", (Bt, M, K), 5, "bfloat16")
    b = rng.make("uniform", (K, N), 6, "bfloat16")
    ta, tb = to_torch(a, BFLOAT16), to_torch(b, BFLOAT16)
    c3 = hip.gemm(ta, tb)
    c2 = hip.gemm(ta.reshape(Bt * M, K), tb)
    torch.cuda.synchronize()
    assert torch.equal(c3.reshape(Bt * M, N), c2)
    r = np.random.default_rng(2)
    rows = np.concatenate([bi * M + r.choice(M, 3, replace=False) for bi in range(Bt)])
    c = to_f32(to_storage(c3.reshape(Bt * M, N)[torch.from_numpy(rows).cuda()]), BFLOAT16)
    del c3, c2, ta
    xa = a.reshape(Bt * M, K)[rows]
    ref = orc.mul(xa, BFLOAT16, b, BFLOAT16)
    assert_half_close(c, ref, orc.abs_bound(to_f32(xa, BFLOAT16), to_f32(b, BFLOAT16)), K)


def test_bf16_4096_full_size_sampled(hip):
    """bf16 [4096,4096] @ [4096,4096] (the bf16 4096^3 throughput shape, bench.py's inputs: seeds 13
    and 14, U[-1,1]; 256 output tiles, one per CU): 48 sampled rows and 48 sampled columns against
    the oracle under the bf16 bar."""
    n = 4096
    a = rng.make("uniform", (n, n), 13, "bfloat16")
    b = rng.make("uniform", (n, n), 14, "bfloat16")
    c = to_f32(to_storage(hip.gemm(to_torch(a, BFLOAT16), to_torch(b, BFLOAT16))), BFLOAT16)
    r = np.random.default_rng(3)
    rows = r.choice(n, 48, replace=False)
    cols = r.choice(n, 48, replace=False)
    fa, fb = to_f32(a, BFLOAT16), to_f32(b, BFLOAT16)
    assert_half_close(c[rows], orc.mul(a[rows], BFLOAT16, b, BFLOAT16), orc.abs_bound(fa[rows], fb), n)
    bc = np.ascontiguousarray(b[:, cols])
    assert_half_close(c[:, cols], orc.mul(a, BFLOAT16, bc, BFLOAT16), orc.abs_bound(fa, fb[:, cols]), n)


def test_fp16_config4_transposed_view(hip):
    """c4 at full size: Q[32,2048,128] @ K.permute(0,2,1) consumed through strides (the persistent
    small-K path), against the oracle on the materialised transpose (ops::Transpose(K,{0,2,1}) on
    the CPU) for every batch."""
    Bt, S, D = 32, 2048, 128
    q = half_bits(rng.normal_f32(7, Bt * S * D) / np.float32(np.sqrt(D)), FLOAT16).reshape(Bt, S, D)
    k = half_bits(rng.normal_f32(8, Bt * S * D) / np.float32(np.sqrt(D)), FLOAT16).reshape(Bt, S, D)
    tq, tk = to_torch(q, FLOAT16), to_torch(k, FLOAT16)
    view = tk.permute(0, 2, 1)
    assert view.stride() == (S * D, 1, D)
    c = to_f32(to_storage(hip.gemm(tq, view)), FLOAT16)
    kt = orc.transpose_last2(k)
    ref = orc.mul(q, FLOAT16, kt, FLOAT16)
    bound = orc.abs_bound(to_f32(q, FLOAT16)[0], to_f32(kt, FLOAT16)[0])
    assert_half_close(c[0], ref[0], bound, D)
    for bi in range(1, Bt):
        assert_half_close(c[bi], ref[bi], orc.abs_bound(to_f32(q, FLOAT16)[bi], to_f32(kt, FLOAT16)[bi]), D)


@pytest.mark.parametrize("dt", [FLOAT16, BFLOAT16, INT8])
@pytest.mark.parametrize("K", [16, 72, 128, 256])
@pytest.mark.parametrize("bt", [False, True])
def test_small_k_persistent_exact(hip, dt, K, bt):
    """The persistent small-K path (K within two 128-byte k-tiles, >= 1024 output tiles): ragged
    256x256 tiles (M=264, N=272), B K-contiguous (transposed view) or N-contiguous, integer-valued
    inputs whose sums every order reproduces: bit-exact against exact fp64 sums."""
    if dt != INT8 and K > 128:
        pytest.skip("16-bit inputs take this path for K <= 128")
    Bt, M, N = 256, 264, 272
    x = ints(60 + K, (Bt, M, K), -2, 2)
    y = ints(61 + K, (Bt, K, N), -2, 2)
    exact = np.matmul(x.astype(np.float64), y.astype(np.float64))
    if dt == INT8:
        xs, ys = x.astype(np.int8), y.astype(np.int8)
        want = orc.low_byte(exact.astype(np.int64))
    else:
        xs, ys = half_bits(x, dt), half_bits(y, dt)
        want = half_bits(exact.astype(np.float32), dt)
    a = to_torch(xs, dt)
    b = to_torch(np.ascontiguousarray(np.swapaxes(ys, 1, 2)), dt).permute(0, 2, 1) if bt else to_torch(ys, dt)
    c = to_storage(hip.gemm(a, b))
    np.testing.assert_array_equal(c, want)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16])
@pytest.mark.parametrize("batch,M,K,N,bt", [(16, 1100, 40, 3832, False), (4, 2048, 32, 9216, True)],
                         ids=["groups-of-30", "72-columns-fallback"])
def test_small_k_row_groups_exact(hip, dt, batch, M, K, N, bt):
    """16-bit small-K GEMMs run 128x128 tiles in groups of as many workgroups as C has column tiles,
    each group walking its own run of row blocks: 30 column tiles make 8 groups of 240 workgroups
    (ragged M, N and K, one B per batch, so B reloads inside a group's run).  With 72 column tiles
    a third of the CUs would idle, so that shape runs the 256x256 small-K kernel instead.
    Integer-valued inputs in [-2, 2]: exact sums, each rounded once."""
    x = ints(24, (batch, M, K), -2, 2)
    y = ints(25, (batch, K, N), -2, 2)
    ta = to_torch(half_bits(x, dt), dt)
    tb = (to_torch(half_bits(np.ascontiguousarray(np.swapaxes(y, 1, 2)), dt), dt).permute(0, 2, 1) if bt
          else to_torch(half_bits(y, dt), dt))
    c = to_storage(hip.gemm(ta, tb))
    np.testing.assert_array_equal(c, half_bits(np.matmul(x, y), dt))


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, INT8])
@pytest.mark.parametrize("batch,M,K,N", [(0, 512, 8192, 1024), (0, 300, 8192, 700), (2, 200, 8192, 520), (0, 1000, 8208, 1000),
                                         (0, 1100, 4104, 2040), (3, 600, 4096, 1280), (0, 1100, 8192, 2040),
                                         (8, 3000, 4096, 64)])
def test_direct_load_stream_k_bit_exact(hip, dt, batch, M, K, N):
    """16-bit and int8 GEMMs with few, long tiles (16-bit: 32, 18, 20, 64, 144, 150, 144 and 192
    tiles of 128x128; int8: 8, 6, 6, 16, 40, 45, 40 and 96 of 256x256; K = 8192, 4096 and the
    ragged 8208 and 4104) run the direct-load kernel's stream-K schedule: tiles summed in segments
    by several workgroups.  16-bit 128x128 tiles split at up to half as many tiles as resident
    workgroups, but above a quarter only into segments of at least 32 k-tiles or on a tile grid of
    one column: 144 tiles at K = 8192 and 8 batches x 24 tiles of one column split, 144 tiles at
    K = 4104 and 150 at K = 4096 stay whole.  int8 splits the 40 and 45 tiles from 33 and 32
    k-tiles (at most a fifth as many tiles as resident workgroups).  Integer-valued inputs: exact fp32 / int32 sums in any order, so the half
    outputs are the exact sums rounded once, int8 the low byte, and everything equals the plain
    kernel's result (tv_hip_gemm_noalloc takes no workspace, hence no stream-K)."""
    lead = (batch,) if batch else ()
    if dt == INT8:
        x = ints(14, lead + (M, K), -128, 127, np.int8)
        y = ints(15, (K, N), -128, 127, np.int8)
        xs, ys = x, y
    else:
        x = ints(14, lead + (M, K), -3, 3)
        y = ints(15, (K, N), -3, 3)
        xs, ys = half_bits(x, dt), half_bits(y, dt)
    ta, tb = to_torch(xs, dt), to_torch(ys, dt)
    exact = np.matmul(x.astype(np.float64), y.astype(np.float64))
    c = to_storage(hip.gemm(ta, tb))
    if dt == INT8:
        np.testing.assert_array_equal(c, orc.low_byte(exact.astype(np.int64)))
        c32 = to_storage(hip.gemm(ta, tb, out_dtype=INT32))
        np.testing.assert_array_equal(c32, exact.astype(np.int32))
    else:
        np.testing.assert_array_equal(c, half_bits(exact.astype(np.float32), dt))
    plain = torch.zeros(lead + (M, N), dtype=ta.dtype, device="cuda")
    args = tv.make_args(ta, tb, plain)
    tv.check(tv.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(plain), c)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, INT8])
@pytest.mark.parametrize("batch,M,K,N,a_t,b_t", [
    (0, 2048, 1000, 4096, False, False),  # 512 tiles of 128x128: two per CU, the most on that size
    (0, 130, 8208, 8000, False, False),   # 126 tiles of 128x128 over 129 k-tiles: split (stream-K)
    (5, 1000, 304, 1096, True, True),     # 360 tiles of 128x128 over a batch, both operands transposed
    (0, 2100, 520, 4104, False, False),   # 561 tiles of 128x128: runs 153 tiles of 256x256 instead
    (0, 2104, 520, 4104, True, False),
    (0, 2100, 520, 4104, False, True)],
    ids=["t128-512", "t128-split", "t128-batch-AtBt", "t256-153", "t256-At", "t256-Bt"])
def test_direct_load_tile_size_exact(hip, dt, batch, M, K, N, a_t, b_t):
    """16-bit and int8 GEMMs on the direct-load kernels run 128x128 tiles while those fit one round
    of resident workgroups (two per CU: at most 512 tiles on 256 CUs) and 256x256 tiles above that.
    Shapes either side of the switch, ragged in M, N and K, with transposed views (int8's 128-row
    M/N-contiguous layout has its own swizzle; int8 rows whose K is not whole 16-byte chunks are
    copied into padded rows first).  Integer-valued inputs: exact sums in any order, half outputs
    each rounded once, int8 the low byte; a second call gives the same bits."""
    lead = (batch,) if batch else ()
    lo, hi = (-8, 8) if dt == INT8 else (-2, 2)
    x = ints(22, lead + (M, K), lo, hi)
    y = ints(23, lead + (K, N), lo, hi)

    def enc(v):
        return v.astype(np.int8) if dt == INT8 else half_bits(v, dt)

    def dev(v, transposed):
        if transposed:
            return to_torch(enc(np.ascontiguousarray(np.swapaxes(v, -1, -2))), dt).transpose(-1, -2)
        return to_torch(enc(v), dt)

    ta, tb = dev(x, a_t), dev(y, b_t)
    c = to_storage(hip.gemm(ta, tb))
    exact = np.matmul(x.astype(np.float64), y.astype(np.float64))
    want = orc.low_byte(exact.astype(np.int64)) if dt == INT8 else half_bits(exact.astype(np.float32), dt)
    np.testing.assert_array_equal(c, want)
    np.testing.assert_array_equal(to_storage(hip.gemm(ta, tb)), c)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16])
@pytest.mark.parametrize("batch,M,K,N", [(0, 4100, 520, 8200), (0, 4100, 100, 8200), (0, 4100, 50, 8200), (3, 2600, 700, 5000)])
def test_direct_load_chain_exact(hip, dt, batch, M, K, N):
    """16-bit GEMMs of at least two 256x256 tiles per CU run the chained persistent kernel (each
    workgroup's k-loop runs on into its next tile, whose first two k-tiles load during the
    previous tile's last steps and store): 561 tiles with ragged M, N and K (9 k-tiles, an odd
    count), K of two and of one k-tile, and 660 tiles over a batch with per-batch B.
    Integer-valued inputs in [-2, 2]: the fp32 sums are exact in any order, so the output is each
    exact sum rounded once; a second call gives the same bits."""
    lead = (batch,) if batch else ()
    x = ints(16, lead + (M, K), -2, 2)
    y = ints(17, lead + (K, N), -2, 2)
    ta, tb = to_torch(half_bits(x, dt), dt), to_torch(half_bits(y, dt), dt)
    exact = np.matmul(x, y)  # fp32 BLAS: integer partial sums below 2^24, exact in any order
    c = to_storage(hip.gemm(ta, tb))
    np.testing.assert_array_equal(c, half_bits(exact, dt))
    np.testing.assert_array_equal(to_storage(hip.gemm(ta, tb)), c)


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16])
@pytest.mark.parametrize("a_t,b_t", [(True, False), (False, True), (True, True)], ids=["At", "Bt", "AtBt"])
def test_direct_load_chain_transposed_views(hip, dt, a_t, b_t):
    """The chained kernel with the other operand layouts, as transposed views consumed through their
    strides (A M-contiguous, B K-contiguous, or both; every pitch a whole number of 16-byte chunks,
    so both stay on the direct-load kernels): 561 tiles, ragged M/N, K = 328 (6 k-tiles).
    Integer-valued inputs, exact sums rounded once."""
    M, K, N = 4104, 328, 8200
    x = ints(18, (M, K), -2, 2)
    y = ints(19, (K, N), -2, 2)
    ta = to_torch(half_bits(np.ascontiguousarray(x.T), dt), dt).t() if a_t else to_torch(half_bits(x, dt), dt)
    tb = to_torch(half_bits(np.ascontiguousarray(y.T), dt), dt).t() if b_t else to_torch(half_bits(y, dt), dt)
    c = to_storage(hip.gemm(ta, tb))
    np.testing.assert_array_equal(c, half_bits(np.matmul(x, y), dt))


@pytest.mark.parametrize("dt", [FLOAT32, BFLOAT16, FLOAT16, INT8])
@pytest.mark.parametrize("batch,M,K,N,a_t,b_t,bcast", [
    (0, 1000, 700, 1030, False, False, False),  # A's rows (K) and B's k rows (N) not whole 16-byte chunks
    (0, 1030, 1002, 700, True, True, False),    # transposed views: A M-contiguous (M = 1030), B K-contiguous (K = 1002)
    (3, 500, 300, 998, False, False, True),     # batched A copied per batch, broadcast B copied once
    (2, 600, 1002, 512, False, True, False),    # per-batch K-contiguous B
    (0, 7, 4096, 129, False, False, False),     # skinny: padded W (N = 129) on the matrix-core GEMV
    (0, 1, 4000, 1001, False, False, False),    # M = 1, ragged N (padded W), K whole chunks
    (0, 20, 1003, 257, False, False, False),    # 9 <= M <= 32 with ragged K (padded x) and N (padded W)
    (4, 5, 4100, 136, False, False, True)],     # batched x with ragged K (padded per batch), broadcast W
    ids=["AK-BN", "AM-BK", "batch-bcastB", "batch-BK", "gemv-N129", "gemv-M1-N1001", "gemv-M20-K1003", "gemv-batch-K4100"])
def test_misaligned_operands_padded_exact(hip, dt, batch, M, K, N, a_t, b_t, bcast):
    """An operand contiguous along one dimension whose rows are not whole 16-byte chunks is copied
    once into zero-padded rows of whole chunks (calls of at least 2^20 multiply-adds, through the
    workspace), and the call runs on the vector loaders: A with K- or M-contiguous rows, B with N-
    or K-contiguous rows, per batch or broadcast; skinny calls (M <= 32) on the matrix-core GEMV
    where it serves the dtype (16-bit; int8 from M = 3; fp32 and int8 M = 1, 2 go to the GEMM),
    reading chunks that straddle N or K from the zero padding.  Integer-valued inputs: exact sums,
    half outputs rounded once, int8 the low byte; fp32 exact."""
    lead = (batch,) if batch else ()
    lo, hi = (-8, 8) if dt == INT8 else (-2, 2)
    x = ints(26, lead + (M, K), lo, hi)
    y = ints(27, (K, N) if bcast else lead + (K, N), lo, hi)

    def enc(v):
        if dt == INT8:
            return v.astype(np.int8)
        return half_bits(v, dt) if dt in (BFLOAT16, FLOAT16) else v.astype(np.float32)

    def dev(v, transposed):
        if transposed:
            return to_torch(np.ascontiguousarray(enc(np.swapaxes(v, -1, -2))), dt).transpose(-1, -2)
        return to_torch(enc(v), dt)

    c = to_storage(hip.gemm(dev(x, a_t), dev(y, b_t)))
    exact = np.matmul(x.astype(np.float64), y.astype(np.float64))
    if dt == INT8:
        np.testing.assert_array_equal(c, orc.low_byte(exact.astype(np.int64)))
    elif dt == FLOAT32:
        np.testing.assert_array_equal(c, exact.astype(np.float32))
    else:
        np.testing.assert_array_equal(c, half_bits(exact.astype(np.float32), dt))


# ---- views, offsets, batches ----------------------------------------------------------------

@pytest.mark.parametrize("dt", [FLOAT32, BFLOAT16, INT8])
def test_views_offsets_and_layouts(hip, dt):
    """Sliced (offset) operands, transposed A and B, non-unit inner strides (gather path) and batched
    B all give the oracle's result on the equivalent dense inputs."""
    lo, hi = (-3, 3)
    M, K, N = 80, 96, 96
    big_a = ints(20, (M + 5, K + 16), lo, hi)
    big_b = ints(21, (K + 8, N + 24), lo, hi)

    def dev(x):
        if dt == INT8:
            return to_torch(x.astype(np.int8), INT8)
        if dt == BFLOAT16:
            return to_torch(rng.f32_to_bf16_bits(x), BFLOAT16)
        return to_torch(x, FLOAT32)

    def ref_of(a, b):
        if dt == INT8:
            return orc.mul(a.astype(np.int8), INT8, b.astype(np.int8), INT8)
        out = orc.mul(a.astype(np.float32), FLOAT32, b.astype(np.float32), FLOAT32)
        return rng.f32_to_bf16_bits(out) if dt == BFLOAT16 else out

    ta, tb = dev(big_a), dev(big_b)
    cases = {
        "offset": (ta[3:3 + M, 8:8 + K], tb[4:4 + K, 16:16 + N], big_a[3:3 + M, 8:8 + K], big_b[4:4 + K, 16:16 + N]),
        "a_transposed": (dev(np.ascontiguousarray(big_a[:M, :K].T)).t(), tb[:K, :N], big_a[:M, :K], big_b[:K, :N]),
        "b_transposed": (ta[:M, :K], dev(np.ascontiguousarray(big_b[:K, :N].T)).t(), big_a[:M, :K], big_b[:K, :N]),
        "gather_a": (ta[:M, 0:2 * (K // 2):2], tb[:K // 2, :N], big_a[:M, 0:2 * (K // 2):2], big_b[:K // 2, :N]),
        "gather_b": (ta[:M, :K // 2], tb[0:K:2, 1:N + 1], big_a[:M, :K // 2], big_b[0:K:2, 1:N + 1]),
        "odd_offset": (ta[1:1 + M, 1:1 + K], tb[1:1 + K, 1:1 + N], big_a[1:1 + M, 1:1 + K], big_b[1:1 + K, 1:1 + N]),
    }
    for name, (x, y, xa, ya) in cases.items():
        c = hip.gemm(x, y)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_storage(c), ref_of(np.ascontiguousarray(xa), np.ascontiguousarray(ya)),
                                      err_msg=name)


@pytest.mark.parametrize("dt", [FLOAT32, FLOAT16, INT8])
def test_batched_equal_batches(hip, dt):
    Bt, M, K, N = 3, 50, 130, 40
    x = ints(22, (Bt, M, K), -3, 3)
    y = ints(23, (Bt, K, N), -3, 3)
    if dt == INT8:
        xs, ys = x.astype(np.int8), y.astype(np.int8)
    elif dt == FLOAT16:
        xs, ys = rng.f32_to_f16_bits(x), rng.f32_to_f16_bits(y)
    else:
        xs, ys = x, y
    c = to_storage(hip.gemm(to_torch(xs, dt), to_torch(ys, dt)))
    ref = orc.mul(xs, dt, ys, dt)
    if dt == FLOAT16:
        ref = rng.f32_to_f16_bits(ref)
    np.testing.assert_array_equal(c, ref)


def test_output_view_with_strides(hip):
    a = ints(24, (40, 64), -3, 3)
    b = ints(25, (64, 48), -3, 3)
    big = torch.zeros((50, 100), dtype=torch.float32, device="cuda")
    out = big[5:45, 10:58]
    hip.gemm(to_torch(a, FLOAT32), to_torch(b, FLOAT32), out=out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(out), orc.mul(a, FLOAT32, b, FLOAT32))
    assert big[:5].abs().sum().item() == 0 and big[:, :10].abs().sum().item() == 0


# ---- SIMT path (dtype pairs without matrix cores) ---------------------------------------------

@pytest.mark.parametrize("pair", [("int32", "int32"), ("int16", "int16"), ("int64", "int64"),
                                  ("int8", "int16"), ("int32", "float32"), ("float64", "float64")])
@pytest.mark.parametrize("shape", [(20, 130, 30), (1024, 70, 1024)])
def test_simt_pairs_vs_oracle(hip, pair, shape):
    import oracle
    names = {"int8": 0, "int16": 1, "int32": 2, "int64": 3, "float32": 6, "float64": 7}
    da, db = names[pair[0]], names[pair[1]]
    M, K, N = shape
    a = ints(26, (M, K), -50, 50, np.dtype(pair[0]))
    b = ints(27, (K, N), -50, 50, np.dtype(pair[1]))
    ref = oracle.mul(a, da, b, db)
    c = hip.gemm(to_torch(a, da), to_torch(b, db), out_dtype=oracle.result_type(da, db))
    torch.cuda.synchronize()
    got = to_storage(c)
    if ref.dtype.kind == "f":
        np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())
    else:
        np.testing.assert_array_equal(got, ref)


def _simt_cases(n=40, seed=20261210):
    """Seeded random calls of the dtype pairs without matrix cores (every pair of the eight dtypes
    but int8, bf16, fp16 and fp32 with themselves): shape up to 200 a side, each operand row-major
    or a transposed view, sometimes batched."""
    r = np.random.default_rng(seed)
    mfma = {(0, 0), (4, 4), (5, 5), (6, 6)}
    pairs = [(a, b) for a in range(8) for b in range(8) if (a, b) not in mfma]
    out = []
    for i in range(n):
        da, db = pairs[int(r.integers(len(pairs)))]
        M, K, N = (int(np.exp(r.uniform(0, np.log(200)))) for _ in range(3))
        out.append((da, db, int(r.choice([0, 0, 2])), M, K, N, bool(r.integers(2)), bool(r.integers(2))))
    return out


SIMT_CASES = _simt_cases()


@pytest.mark.parametrize("case", SIMT_CASES, ids=[f"{c[0]}x{c[1]}-b{c[2]}-{c[3]}x{c[4]}x{c[5]}{'-at' if c[6] else ''}"
                                                  f"{'-bt' if c[7] else ''}" for c in SIMT_CASES])
def test_simt_random_pairs_exact(hip, case):
    """The SIMT kernel on seeded random dtype pairs, shapes, batches and transposed views, with
    integer inputs in [-50, 50] (exact in every dtype, and every sum exact in the accumulator types):
    bit-exact against the oracle's MulImpl<CPU>, in the CPU backend's result dtype."""
    import oracle
    da, db, batch, M, K, N, at, bt = case
    lead = (batch,) if batch else ()
    seed = 3 * M + 5 * K + 7 * N + da * 11 + db
    a = rng.uniform_int(seed, int(np.prod(lead + (M, K))), -50, 50).reshape(lead + (M, K))
    b = rng.uniform_int(seed + 1, int(np.prod(lead + (K, N))), -50, 50).reshape(lead + (K, N))

    def enc(x, dt):
        if dt == BFLOAT16:
            return rng.f32_to_bf16_bits(x.astype(np.float32))
        if dt == FLOAT16:
            return rng.f32_to_f16_bits(x.astype(np.float32))
        return x.astype(orc.NP[dt])

    def dev(x, dt, t):
        if t:
            return to_torch(np.ascontiguousarray(np.swapaxes(enc(x, dt), -1, -2)), dt).transpose(-1, -2)
        return to_torch(np.ascontiguousarray(enc(x, dt)), dt)

    ea, eb = enc(a, da), enc(b, db)
    ref = np.stack([oracle.mul(ea[i], da, eb[i], db) for i in range(batch)]) if batch else oracle.mul(ea, da, eb, db)
    c = hip.gemm(dev(a, da, at), dev(b, db, bt), out_dtype=oracle.result_type(da, db))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), ref)


def test_rejects_bad_output_dtype(hip):
    a = torch.ones((4, 4), dtype=torch.int8, device="cuda")
    with pytest.raises(hip.TensorviaHipError):
        hip.gemm(a, a, out_dtype=FLOAT32)
