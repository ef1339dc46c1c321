"""GPU parity at sizes past 4 GiB: operands, outputs and byte offsets beyond 2^32, element counts
beyond 2^31 (an MI355X holds 288 GB, so such tensors are ordinary there).  Every address the
kernels form is a 64-bit base (per batch, tile, k-tile or K slice) plus a 32-bit offset inside a
range checked on the host; these calls put the bases past 2^32 for each kernel family: the
256x256 direct-load tiles and the chained schedule (bf16, fp16, int8), the fp32 tiles, the
row-synchronous small-K kernel over batches, both GEMV layouts, the SIMT path, the transpose,
the cast and the seeded generator; and through the C++ API, a host round trip and ops::Mul past
4 GiB (tests/cpp/large_driver.cpp).

Checks, all exact:
* sampled rows or columns (always including the first and the last) against numpy's float64 or
  int64 products of the same integer inputs;
* over the whole output, weighted checksums: r^T C 1 = (r^T A)(B 1) and 1^T C w = (1^T A)(B w), with
  row weights r and column weights w, summed in float64 on the device (exact: every term
  is an integer below 2^53), so a dropped, misplaced or duplicated row or column block fails.
Inputs are integers in {-1, 0, 1} (or [-3, 3] for int8), so every sum is exact in the output type
(|sum| <= 256 in bf16, <= 2048 in fp16, below 2^24 in fp32) and every accumulation order agrees.
"""
import ctypes
import subprocess

import numpy as np
import pytest
import torch

import tensorvia_amd as tv
from tensorvia_amd import rng

pytestmark = pytest.mark.gpu

GIB4 = 1 << 32


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _ints(shape, lo, hi, dtype, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    t = torch.randint(lo, hi + 1, shape, dtype=torch.int8, device="cuda", generator=g)
    return t if dtype == torch.int8 else t.to(dtype)


def _rows_sample(n, k=24, seed=0):
    r = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, 1, n // 2, n - 2, n - 1], r.integers(0, n, k)]))


def _f64(t):
    return t.to(torch.float64)


def _weighted_sums(c, wr, wc, chunk):
    """(r^T C 1, 1^T C w) of a [M, N] device tensor, in float64, over row chunks."""
    s_r = torch.zeros((), dtype=torch.float64, device="cuda")
    s_c = torch.zeros((), dtype=torch.float64, device="cuda")
    for i in range(0, c.shape[0], chunk):
        blk = _f64(c[i:i + chunk])
        s_r += (blk.sum(1) * wr[i:i + chunk]).sum()
        s_c += (blk.sum(0) * wc).sum()
    return s_r.item(), s_c.item()


def _expected_sums(a, b, wr, wc, chunk):
    """(r^T A)(B 1) and (1^T A)(B w) for A [M, K], B [K, N] (any layout), in float64."""
    rA = torch.zeros(a.shape[1], dtype=torch.float64, device="cuda")
    oA = torch.zeros(a.shape[1], dtype=torch.float64, device="cuda")
    for i in range(0, a.shape[0], chunk):
        blk = _f64(a[i:i + chunk])
        rA += (blk * wr[i:i + chunk, None]).sum(0)
        oA += blk.sum(0)
    b1 = torch.zeros(b.shape[0], dtype=torch.float64, device="cuda")
    bw = torch.zeros(b.shape[0], dtype=torch.float64, device="cuda")
    for i in range(0, b.shape[0], chunk):
        blk = _f64(b[i:i + chunk])
        b1[i:i + chunk] = blk.sum(1)
        bw[i:i + chunk] = (blk * wc).sum(1)
    return (rA @ b1).item(), (oA @ bw).item()


def _weights(M, N):
    wr = (torch.arange(M, device="cuda", dtype=torch.float64) % 7) + 1
    wc = (torch.arange(N, device="cuda", dtype=torch.float64) % 5) + 1
    return wr, wc


def _check_gemm(a, b, c, round_to, chunk=2048, rows=None):
    """Sampled rows exact against numpy, then both weighted checksums over the whole output."""
    M, N = c.shape
    rows = _rows_sample(M) if rows is None else rows
    idx = torch.from_numpy(rows).cuda()
    want = np.asarray(a.index_select(0, idx).cpu().to(torch.float64).numpy()) @ b.cpu().to(torch.float64).numpy()
    got = c.index_select(0, idx).cpu()
    np.testing.assert_array_equal(round_to(got), round_to(torch.from_numpy(want)), err_msg="sampled rows")
    wr, wc = _weights(M, N)
    assert _weighted_sums(c, wr, wc, chunk) == _expected_sums(a, b, wr, wc, chunk)


def _as_f64(t):
    return t.to(torch.float64).numpy()


@pytest.mark.parametrize("dt,M,N,K", [(torch.bfloat16, 65536, 36864, 256), (torch.float16, 65536, 36864, 64)],
                         ids=["bf16-65536x36864x256", "fp16-65536x36864x64"])
def test_half_output_past_4gib(hip, dt, M, N, K):
    """One [M, N] output of 4.8 GB (2.4e9 elements) in one batch: the 256x256 tiles' stores past
    2^32 bytes.  fp16 with K = 64 is a small-K shape whose single output is too large for the
    row-synchronous kernel's 32-bit store offsets, so the tiled kernel must take it."""
    a = _ints((M, K), -1, 1, dt, 11)
    b = _ints((K, N), -1, 1, dt, 12)
    c = hip.gemm(a, b)
    assert c.numel() * c.element_size() > GIB4
    torch.cuda.synchronize()
    _check_gemm(a, b, c, lambda t: _as_f64(t.to(torch.float32)))


def test_int8_a_past_4gib(hip):
    """int8 A [131072, 40960] (5.4 GB): tile bases of A past 2^32; int8 output (the low byte of the
    exact sum) on sampled rows, int32 output on sampled rows and the whole-output checksums."""
    M, N, K = 131072, 256, 40960
    a = _ints((M, K), -3, 3, torch.int8, 21)
    b = _ints((K, N), -3, 3, torch.int8, 22)
    assert a.numel() > GIB4
    c8 = hip.gemm(a, b)
    c32 = hip.gemm(a, b, out_dtype=tv.INT32)
    torch.cuda.synchronize()
    rows = _rows_sample(M)
    idx = torch.from_numpy(rows).cuda()
    want = a.index_select(0, idx).cpu().to(torch.float64).numpy() @ b.cpu().to(torch.float64).numpy()
    want = want.astype(np.int64)
    np.testing.assert_array_equal(c32.index_select(0, idx).cpu().numpy(), want.astype(np.int32))
    np.testing.assert_array_equal(c8.index_select(0, idx).cpu().numpy(), want.astype(np.int8))
    wr, wc = _weights(M, N)
    assert _weighted_sums(c32, wr, wc, 8192) == _expected_sums(a, b, wr, wc, 1024)


@pytest.mark.parametrize("b_layout", ["n_contiguous", "k_contiguous"])
def test_bf16_b_past_4gib(hip, b_layout):
    """bf16 A [512, 65536] @ B [65536, 36864] (4.8 GB) into fp32: B's k-tile bases (N-contiguous) or
    tile bases (K-contiguous, a transposed view of [36864, 65536]) past 2^32."""
    M, N, K = 512, 36864, 65536
    a = _ints((M, K), -1, 1, torch.bfloat16, 31)
    if b_layout == "n_contiguous":
        b = _ints((K, N), -1, 1, torch.bfloat16, 32)
    else:
        b = _ints((N, K), -1, 1, torch.bfloat16, 33).t()
    c = hip.gemm(a, b, out_dtype=tv.FLOAT32)
    torch.cuda.synchronize()
    cols = _rows_sample(N, 8, seed=5)
    cidx = torch.from_numpy(cols).cuda()
    want = a.cpu().to(torch.float64).numpy() @ b.index_select(1, cidx).cpu().to(torch.float64).numpy()
    np.testing.assert_array_equal(c.index_select(1, cidx).cpu().numpy(), want.astype(np.float32))
    wr, wc = _weights(M, N)
    assert _weighted_sums(c, wr, wc, 512) == _expected_sums(a, b, wr, wc, 2048)


def test_fp32_a_past_4gib(hip):
    """fp32 A [65536, 16640] (4.4 GB) @ B [16640, 256]: the fp32 tiles' A bases past 2^32."""
    M, N, K = 65536, 256, 16640
    a = _ints((M, K), -1, 1, torch.float32, 41)
    b = _ints((K, N), -1, 1, torch.float32, 42)
    assert a.numel() * 4 > GIB4
    c = hip.gemm(a, b)
    torch.cuda.synchronize()
    _check_gemm(a, b, c, _as_f64, chunk=4096)


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("w_layout", ["n_contiguous", "k_contiguous"])
def test_gemv_w_past_4gib(hip, M, w_layout):
    """x[M, 16384] @ W[16384, 139264] bf16 (4.6 GB) on tv_hip_gemv, fp32 output: K-slice bases of W
    (row-major W) or strip bases (x @ W^T, W stored [139264, 16384]) past 2^32."""
    N, K = 139264, 16384
    x = _ints((M, K), -1, 1, torch.bfloat16, 51 + M)
    if w_layout == "n_contiguous":
        w = _ints((K, N), -1, 1, torch.bfloat16, 61)
    else:
        w = _ints((N, K), -1, 1, torch.bfloat16, 62).t()
    c = hip.gemv(x, w, out_dtype=tv.FLOAT32)
    torch.cuda.synchronize()
    cols = _rows_sample(N, 24, seed=7)
    cidx = torch.from_numpy(cols).cuda()
    want = x.cpu().to(torch.float64).numpy() @ w.index_select(1, cidx).cpu().to(torch.float64).numpy()
    np.testing.assert_array_equal(c.index_select(1, cidx).cpu().numpy(), want.astype(np.float32))
    wr, wc = _weights(M, N)
    assert _weighted_sums(c, wr, wc, 8) == _expected_sums(x, w, wr, wc, 1024)


def test_small_k_batched_output_past_4gib(hip):
    """fp16 Q[20, 8192, 128] @ transpose(K[20, 16384, 128]) -> [20, 8192, 16384] (5.4 GB): the
    row-synchronous small-K kernel's per-batch output bases past 2^32."""
    B, M, N, K = 20, 8192, 16384, 128
    q = _ints((B, M, K), -1, 1, torch.float16, 71)
    kk = _ints((B, N, K), -1, 1, torch.float16, 72)
    c = hip.gemm(q, kk.transpose(1, 2))
    assert c.numel() * 2 > GIB4
    torch.cuda.synchronize()
    for bi in (0, 9, B - 1):
        _check_gemm(q[bi], kk[bi].t(), c[bi], lambda t: _as_f64(t.to(torch.float32)), chunk=4096,
                    rows=_rows_sample(M, 8, seed=bi))


def test_simt_output_past_2g_elements(hip):
    """int16 A [65536, 1] @ B [1, 36000] -> int16 [65536, 36000] (2.4e9 elements, 4.7 GB) on the SIMT
    kernel: element offsets past 2^31."""
    M, N = 65536, 36000
    a = _ints((M, 1), -3, 3, torch.int16, 81)
    b = _ints((1, N), -3, 3, torch.int16, 82)
    c = torch.empty((M, N), dtype=torch.int16, device="cuda")
    hip.gemm(a, b, out=c)
    assert c.numel() > (1 << 31)
    torch.cuda.synchronize()
    rows = _rows_sample(M)
    want = a.cpu().numpy().astype(np.int64)[rows] * b.cpu().numpy().astype(np.int64)
    np.testing.assert_array_equal(c[torch.from_numpy(rows).cuda()].cpu().numpy(), want.astype(np.int16))
    wr, wc = _weights(M, N)
    assert _weighted_sums(c, wr, wc, 4096) == _expected_sums(a, b, wr, wc, 4096)


def test_transpose_past_4gib(hip):
    """tv_hip_repack of [2, 32768, 36864] 16-bit elements viewed transposed (4.8 GB): equal to torch's
    own element order of the same view, bit for bit."""
    src = torch.randint(-32768, 32767, (2, 32768, 36864), dtype=torch.int16, device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(91))
    view = src.transpose(1, 2)
    dst = torch.empty(view.shape, dtype=torch.int16, device="cuda")
    a = tv.TvRepackArgs()
    a.ndim, a.elem_size = 3, 2
    for d in range(3):
        a.shape[d] = view.shape[d]
        a.strides[d] = view.stride()[d]
    a.src, a.dst = src.data_ptr(), dst.data_ptr()
    tv.check(tv.lib().tv_hip_repack(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    assert dst.numel() * 2 > GIB4
    for bi in range(2):
        for j in range(0, 36864, 4096):
            assert torch.equal(dst[bi, j:j + 4096], view[bi, j:j + 4096]), (bi, j)


def test_typecast_past_2g_elements(hip):
    """tv_hip_typecast int8 -> fp32 of 2^31 + 4099 elements (8.6 GB out): exact widening everywhere."""
    n = (1 << 31) + 4099
    src = _ints((n,), -128, 127, torch.int8, 101)
    dst = torch.empty(n, dtype=torch.float32, device="cuda")
    tv.check(tv.lib().tv_hip_typecast(ctypes.c_void_p(src.data_ptr()), tv.INT8, ctypes.c_void_p(dst.data_ptr()),
                                      tv.FLOAT32, n, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    torch.cuda.synchronize()
    for i in range(0, n, 1 << 28):
        assert torch.equal(dst[i:i + (1 << 28)], src[i:i + (1 << 28)].to(torch.float32)), i
    np.testing.assert_array_equal(dst[-5000:].cpu().numpy(), src[-5000:].cpu().numpy().astype(np.float32))


def test_random_and_fill_past_2g_elements(hip):
    """tv_hip_random int8 over 2^31 + 1001 elements: windows past 2^31 equal the seeded stream at those
    counters; tv_hip_fill fp32 over 2^30 + 5 elements (4 GiB + 20 bytes) sets every element."""
    n = (1 << 31) + 1001
    buf = torch.empty(n, dtype=torch.int8, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tv.check(tv.lib().tv_hip_random(ctypes.c_void_p(buf.data_ptr()), tv.INT8, n, -100.0, 100.0, 77, s))
    torch.cuda.synchronize()
    for start in (0, (1 << 31) - 500, n - 1000):
        raw = rng.raw_u64(77, 1000, start)
        want = (np.int64(-100) + (((raw >> np.uint64(32)) * np.uint64(201)) >> np.uint64(32)).astype(np.int64))
        np.testing.assert_array_equal(buf[start:start + 1000].cpu().numpy(), want.astype(np.int8), err_msg=str(start))
    del buf
    m = (1 << 30) + 5
    f = torch.zeros(m, dtype=torch.float32, device="cuda")
    tv.check(tv.lib().tv_hip_fill(ctypes.c_void_p(f.data_ptr()), tv.FLOAT32, m, 2.5, s))
    torch.cuda.synchronize()
    assert bool((f == 2.5).all())


def test_cpp_api_past_4gib(hip):
    """The C++ API end to end: a host -> device -> host round trip of 4 GiB + 12,345 bytes through
    the pinned staging chunks, and ops::Mul of a 5.4 GB int8 A made by the device ops::Random,
    sampled rows on either side of A's byte offset 2^32 equal to the low byte of the exact sums
    (tests/cpp/large_driver.cpp, in a child process)."""
    from tests.cpp import build as cpp
    r = subprocess.run([str(cpp.binary("large_driver"))], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "ok round_trip 4294979641 bytes" in r.stdout, r.stdout
    assert "ok mul int8 [131072,40960]@[40960,256]: 12 sampled rows" in r.stdout, r.stdout


@pytest.mark.parametrize("dt,batch,M,K,N,bcast", [
    (torch.bfloat16, 100003, 40, 40, 48, False), (torch.bfloat16, 100003, 3, 64, 64, False),
    (torch.float16, 20003, 128, 32, 128, False), (torch.float32, 100003, 17, 33, 19, False),
    (torch.int8, 100003, 24, 64, 40, True), (torch.int16, 30011, 5, 7, 9, False)],
    ids=["bf16_gemm", "bf16_gemv", "fp16_small_k", "fp32", "int8_bcast_b", "int16_simt"])
def test_many_small_batches(hip, dt, batch, M, K, N, bcast):
    """Tens of thousands of small matrices in one call (the batch folds into the grid's first
    dimension): every route (the direct-load GEMM, the GEMV, the small-K kernel, fp32 tiles, a B
    broadcast over the batch, the SIMT kernel) exact against numpy's sums of the integer inputs."""
    a = _ints((batch, M, K), -3, 3, dt if dt != torch.int16 else torch.int8, 111).to(dt)
    b = _ints((K, N) if bcast else (batch, K, N), -3, 3, dt if dt != torch.int16 else torch.int8, 112).to(dt)
    c = hip.gemm(a, b)
    torch.cuda.synchronize()
    want = np.matmul(a.cpu().to(torch.float64).numpy(), b.cpu().to(torch.float64).numpy())
    got = c.cpu()
    if dt in (torch.int8, torch.int16):
        np.testing.assert_array_equal(got.numpy(), want.astype(np.int64).astype(got.numpy().dtype))
    else:
        np.testing.assert_array_equal(got.to(torch.float64).numpy(), torch.from_numpy(want).to(dt).to(torch.float64).numpy())
