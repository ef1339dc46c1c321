"""GPU parity of the device initialisers and casts (tv_hip_random, tv_hip_fill, tv_hip_typecast).

Expected values come from tensorvia_amd/rng.py (the seeded stream, itself pinned against the C++
host generator in test_cpp_api.py) and from numpy's conversions: integer casts and widenings are
exact, float -> integer truncates toward zero, fp32 -> fp16 / fp64 -> fp32 round to nearest even
(numpy's astype), and bf16 results round to nearest even through rng.f32_to_bf16_bits.  Every
comparison is bit-exact.

Two levels: the C++ API end to end (tests/cpp/init_driver.cpp: ops::Random / Fill / Zeros / Ones /
Typecast of a transposed device view), and the C-ABI on raw device buffers, including misaligned
pointers (the element-loop path), ragged lengths and a large stream checked at sampled offsets.
"""
import ctypes
import re
import subprocess

import numpy as np
import pytest

from tensorvia_amd import rng
from tests.cpp import build as cpp

pytestmark = pytest.mark.gpu

INT8, INT16, INT32, INT64, BFLOAT16, FLOAT16, FLOAT32, FLOAT64 = range(8)
NAMES = ["int8", "int16", "int32", "int64", "bfloat16", "float16", "float32", "float64"]
STORAGE = [np.int8, np.int16, np.int32, np.int64, np.uint16, np.uint16, np.float32, np.float64]
VALID_CASTS = [(INT8, FLOAT32), (INT16, FLOAT32), (INT16, FLOAT64), (INT32, FLOAT32), (INT32, FLOAT64),
               (INT64, FLOAT64), (FLOAT32, FLOAT16), (FLOAT32, INT32), (FLOAT32, INT64), (INT8, INT16),
               (INT8, INT32), (INT8, INT64), (INT16, INT32), (INT32, INT64), (FLOAT16, FLOAT32),
               (FLOAT16, FLOAT64), (FLOAT16, BFLOAT16), (BFLOAT16, FLOAT32), (BFLOAT16, FLOAT64),
               (BFLOAT16, FLOAT16), (FLOAT32, FLOAT64), (FLOAT64, FLOAT32)]


def is_int(dt):
    return dt <= INT64


def lo_hi(dt):
    return (-100, 100) if is_int(dt) else (-300.0, 300.0)


def to_value(bits, dt):
    """Storage array -> numeric array (half types widened exactly to fp32)."""
    if dt == BFLOAT16:
        return rng.bf16_bits_to_f32(bits)
    if dt == FLOAT16:
        return rng.f16_bits_to_f32(bits)
    return bits


def from_value(x, dt):
    """Numeric array -> storage of dtype dt with the device's conversion rules."""
    x = np.asarray(x)
    if dt == BFLOAT16:
        return rng.f32_to_bf16_bits(x.astype(np.float32))
    if dt == FLOAT16:
        return x.astype(np.float32).astype(np.float16).view(np.uint16)
    if is_int(dt) and x.dtype.kind == "f":
        return np.trunc(x).astype(STORAGE[dt])
    return x.astype(STORAGE[dt])


def expected_cast(src_bits, s, d):
    return from_value(to_value(src_bits, s), d)


# ---- C++ API ------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def init_run(tmp_path_factory):
    out = tmp_path_factory.mktemp("cpp_init")
    r = subprocess.run([str(cpp.binary("init_driver")), str(out)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    done = set(re.findall(r"^done (\S+)$", r.stdout, re.M))
    return r, out, done


def _read(out, name, dt, shape):
    return np.fromfile(out / f"{name}.bin", dtype=STORAGE[dt]).reshape(shape)


@pytest.mark.parametrize("dt", range(8), ids=NAMES)
def test_cpp_random_fill_zeros_ones(init_run, dt):
    r, out, done = init_run
    for n in ("rand", "fill", "zeros", "ones"):
        assert f"{n}_{dt}" in done, r.stdout[-2000:]
    lo, hi = lo_hi(dt)
    want = rng.make("uniform", (3, 1001), 40 + dt, NAMES[dt], lo, hi)
    np.testing.assert_array_equal(_read(out, f"rand_{dt}", dt, (3, 1001)), want)
    np.testing.assert_array_equal(_read(out, f"fill_{dt}", dt, (517,)), from_value(np.full(517, 2.75), dt))
    np.testing.assert_array_equal(_read(out, f"zeros_{dt}", dt, (9, 7)), from_value(np.zeros((9, 7)), dt))
    np.testing.assert_array_equal(_read(out, f"ones_{dt}", dt, (9, 7)), from_value(np.ones((9, 7)), dt))


@pytest.mark.parametrize("s,d", VALID_CASTS, ids=[f"{NAMES[s]}->{NAMES[d]}" for s, d in VALID_CASTS])
def test_cpp_typecast_of_transposed_view(init_run, s, d):
    r, out, done = init_run
    name = f"cast_{s}_{d}"
    assert name in done, r.stdout[-2000:]
    lo, hi = lo_hi(s)
    src = rng.make("uniform", (257, 33), 70 + 8 * s + d, NAMES[s], lo, hi)
    want = expected_cast(np.ascontiguousarray(src.T), s, d)
    np.testing.assert_array_equal(_read(out, name, d, (33, 257)), want)


def _fused_ref(a, b, bias, act):
    pre = np.matmul(a, b) + bias
    return {0: pre, 1: np.maximum(pre, 0), 2: pre / (1 + np.exp(-pre)), 3: 1 / (1 + np.exp(-pre)), 4: np.tanh(pre)}[act]


@pytest.mark.parametrize("act", range(5), ids=["none", "relu", "silu", "sigmoid", "tanh"])
def test_cpp_mul_bias_act(init_run, act):
    """ops::MulBiasAct: bf16 [2,64,96] @ broadcast [96,80] + per-column bias, then the activation,
    within the bf16 bar (1e-2 relative plus the matmul bound) of the fp64 composition."""
    r, out, done = init_run
    assert f"fused_{act}" in done, r.stdout[-2000:]
    a = to_value(rng.make("uniform", (2, 64, 96), 90, "bfloat16", -1, 1), BFLOAT16).astype(np.float64)
    b = to_value(rng.make("uniform", (96, 80), 91, "bfloat16", -1, 1), BFLOAT16).astype(np.float64)
    bias = to_value(rng.make("uniform", (80,), 92, "bfloat16", -2, 2), BFLOAT16).astype(np.float64)
    ref = _fused_ref(a, b, bias, act)
    got = to_value(_read(out, f"fused_{act}", BFLOAT16, (2, 64, 80)), BFLOAT16).astype(np.float64)
    tol = 1e-2 * np.abs(ref) + 1e-5 * np.sqrt(96) * np.matmul(np.abs(a), np.abs(b)) + 1e-3
    assert (np.abs(got - ref) <= tol).all()


def test_cpp_mul_bias_act_fp32_full_bias_and_errors(init_run):
    r, out, done = init_run
    assert "fused_f32_full" in done, r.stdout[-2000:]
    a = rng.make("uniform", (64, 96), 93, "float32", -1, 1).astype(np.float64)
    b = rng.make("uniform", (96, 80), 94, "float32", -1, 1).astype(np.float64)
    bias = rng.make("uniform", (64, 80), 95, "float32", -2, 2).astype(np.float64)
    ref = _fused_ref(a, b, bias, 2)
    got = _read(out, "fused_f32_full", FLOAT32, (64, 80)).astype(np.float64)
    tol = 1e-5 * np.sqrt(96) * np.matmul(np.abs(a), np.abs(b)) + 1e-6 * np.abs(ref) + 1e-30
    assert (np.abs(got - ref) <= tol).all()
    for name in ("bias_dtype", "bias_shape", "int8_output"):
        assert re.search(rf"^threw {name}: ", r.stdout, re.M), r.stdout[-2000:]


@pytest.mark.parametrize("i", range(5))
def test_cpp_transpose_into_dst(init_run, i):
    """ops::Transpose(a, dst, axes) (reference src/ops.cpp:1354-1378): dst, a 1-d tensor of the same
    element count, is reshaped to the permuted shape and holds numpy's transpose, bit for bit."""
    r, out, done = init_run
    assert f"tdst_{i}" in done, r.stdout[-2000:]
    src = rng.make("uniform", (4, 6, 10), 100, "int32", -1000, 999)
    if i < 3:
        want = np.transpose(src, [(2, 0, 1), (0, 2, 1), (1, 0, 2)][i])
        dt = INT32
    elif i == 3:
        want = np.transpose(rng.make("uniform", (3, 40, 16), 101, "float16", -1, 1), (0, 2, 1))
        dt = FLOAT16
    else:
        want = np.transpose(src[1:3, 2:6, :], (2, 1, 0))
        dt = INT32
    np.testing.assert_array_equal(_read(out, f"tdst_{i}", dt, want.shape), np.ascontiguousarray(want))


def test_cpp_transpose_into_dst_errors(init_run):
    r, _, _ = init_run
    for name in ("transpose_dst_dtype", "transpose_dst_self"):
        assert re.search(rf"^threw {name}: ", r.stdout, re.M), r.stdout[-2000:]


def test_cpp_failed_allocation_leaves_no_error_behind(init_run):
    """A device tensor too large for the device throws (the reference's CUDA backend throws the
    driver's message, include/backend/cuda/cuda_tensor.cpp:20-23), and the int8 ops::Mul that
    follows succeeds with the exact low-byte result: the failure is not reported again."""
    r, out, done = init_run
    assert re.search(r"^threw alloc_too_large: .*hipMalloc", r.stdout, re.M), r.stdout[-2000:]
    assert "mul_after_oom" in done, r.stdout[-2000:]
    a = rng.make("uniform", (64, 96), 5, "int8", -3, 3)
    b = rng.make("uniform", (96, 80), 6, "int8", -3, 3)
    want = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int8)
    np.testing.assert_array_equal(_read(out, "mul_after_oom", INT8, (64, 80)), want)


def test_cpp_init_driver_exit_status(init_run):
    r, _, _ = init_run
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]


# ---- C-ABI on raw device buffers -------------------------------------------------------------------

@pytest.fixture(scope="module")
def dev():
    import torch

    import tensorvia_amd as tv
    assert torch.cuda.is_available()
    return torch, tv, tv.lib()


def _buf(torch, nbytes):
    return torch.empty(nbytes + 64, dtype=torch.uint8, device="cuda")


def _stream(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _host(torch, buf, off, n, dt):
    torch.cuda.synchronize()
    es = np.dtype(STORAGE[dt]).itemsize
    return buf[off:off + n * es].cpu().numpy().view(STORAGE[dt])


@pytest.mark.parametrize("dt", range(8), ids=NAMES)
@pytest.mark.parametrize("n,misalign", [(1, 0), (7, 0), (8, 0), (4097, 0), (4097, 1), (1000, 3)])
def test_capi_random_ragged_and_misaligned(dev, dt, n, misalign):
    torch, tv, L = dev
    es = np.dtype(STORAGE[dt]).itemsize
    buf = _buf(torch, n * es)
    off = misalign * es
    lo, hi = lo_hi(dt)
    tv.check(L.tv_hip_random(ctypes.c_void_p(buf.data_ptr() + off), dt, n, lo, hi, 1234 + dt, _stream(torch)))
    np.testing.assert_array_equal(_host(torch, buf, off, n, dt), rng.make("uniform", (n,), 1234 + dt, NAMES[dt], lo, hi))


@pytest.mark.parametrize("dt", [INT8, BFLOAT16, FLOAT32, FLOAT64], ids=lambda d: NAMES[d])
def test_capi_random_large_stream_sampled(dev, dt):
    """64 Mi elements (grid-stride loop): windows at sampled offsets equal the stream at those
    counters, and the values cover [lo, hi] with the uniform mean."""
    torch, tv, L = dev
    n = 64 << 20
    es = np.dtype(STORAGE[dt]).itemsize
    buf = torch.empty(n * es, dtype=torch.uint8, device="cuda")
    lo, hi = lo_hi(dt)
    tv.check(L.tv_hip_random(ctypes.c_void_p(buf.data_ptr()), dt, n, lo, hi, 99, _stream(torch)))
    torch.cuda.synchronize()
    for start in (0, 8 * 12345 + 3, n // 2 - 5, n - 1000):
        got = buf[start * es:(start + 1000) * es].cpu().numpy().view(STORAGE[dt])
        raw = rng.raw_u64(99, 1000, start)
        if is_int(dt):
            span = np.uint64(hi - lo + 1)
            want = (np.int64(lo) + (((raw >> np.uint64(32)) * span) >> np.uint64(32)).astype(np.int64)).astype(STORAGE[dt])
        else:
            u = (raw >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
            f = np.float32(lo) + np.float32(hi - lo) * u
            want = from_value(f, dt) if dt != FLOAT64 else f.astype(np.float64)
        np.testing.assert_array_equal(got, want)
    v = to_value(buf[: (1 << 22) * es].cpu().numpy().view(STORAGE[dt]), dt).astype(np.float64)
    assert v.min() >= lo and v.max() <= hi
    assert abs(v.mean() - (lo + hi) / 2) < 0.01 * (hi - lo)


@pytest.mark.parametrize("dt", range(8), ids=NAMES)
@pytest.mark.parametrize("value", [0.0, 1.0, -2.5, 0.1, 65504.0, -3.999])
def test_capi_fill(dev, dt, value):
    torch, tv, L = dev
    if is_int(dt) and not np.iinfo(STORAGE[dt]).min <= np.trunc(value) <= np.iinfo(STORAGE[dt]).max:
        pytest.skip("value outside the integer type: the conversion is undefined")
    n = 1003
    es = np.dtype(STORAGE[dt]).itemsize
    buf = _buf(torch, n * es)
    want = from_value(np.full(n, np.float32(value)), dt)
    for off in (0, es):
        tv.check(L.tv_hip_fill(ctypes.c_void_p(buf.data_ptr() + off), dt, n, value, _stream(torch)))
        np.testing.assert_array_equal(_host(torch, buf, off, n, dt), want)


@pytest.mark.parametrize("s,d", VALID_CASTS, ids=[f"{NAMES[s]}->{NAMES[d]}" for s, d in VALID_CASTS])
@pytest.mark.parametrize("n,soff,doff", [(8 * 1000, 0, 0), (4099, 0, 0), (1001, 1, 0), (1001, 0, 1)])
def test_capi_typecast(dev, s, d, n, soff, doff):
    torch, tv, L = dev
    ess, esd = np.dtype(STORAGE[s]).itemsize, np.dtype(STORAGE[d]).itemsize
    lo, hi = lo_hi(s)
    src = rng.make("uniform", (n,), 500 + s * 8 + d, NAMES[s], lo, hi)
    sbuf = _buf(torch, n * ess)
    sbuf[soff * ess:(soff + n) * ess] = torch.from_numpy(src.view(np.uint8).copy()).cuda()
    dbuf = _buf(torch, n * esd)
    tv.check(L.tv_hip_typecast(ctypes.c_void_p(sbuf.data_ptr() + soff * ess), s,
                               ctypes.c_void_p(dbuf.data_ptr() + doff * esd), d, n, _stream(torch)))
    np.testing.assert_array_equal(_host(torch, dbuf, doff * esd, n, d), expected_cast(src, s, d))


def test_capi_typecast_same_dtype_copies_and_invalid_pair_rejected(dev):
    torch, tv, L = dev
    src = torch.arange(100, dtype=torch.int32, device="cuda")
    dst = torch.zeros(100, dtype=torch.int32, device="cuda")
    tv.check(L.tv_hip_typecast(ctypes.c_void_p(src.data_ptr()), INT32, ctypes.c_void_p(dst.data_ptr()), INT32, 100,
                               _stream(torch)))
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    assert L.tv_hip_typecast(ctypes.c_void_p(src.data_ptr()), INT32, ctypes.c_void_p(dst.data_ptr()), INT8, 100,
                             _stream(torch)) == tv.TV_E_DTYPE
