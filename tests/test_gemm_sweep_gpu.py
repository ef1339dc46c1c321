"""GPU parity sweep over seeded random calls of tv_hip_gemm: dtype (fp32, bf16, fp16, int8), shape
(M, N, K from 1 to a few thousand, log-uniform), batch (none, 1 or 3, B per batch or broadcast)
and the layout of each operand (row-major, or stored transposed and viewed back).  The router
sends such calls to every kernel family: the GEMVs (M <= 32), the small-K kernels, the 128x128 and
256x256 direct-load tiles and their stream-K and chained schedules, the six fp32 tiles, the padded
row copies of misaligned operands and the element-gather loader.

Inputs are integers in [-3, 3], so every accumulation order gives the same fp32 / int32 sum: fp32
outputs must equal the exact sum, half outputs the exact sum rounded once, int8 outputs its low
byte (the reference CPU backend's wrap-around result), bit for bit; every third int8 or half call
asks for the widened int32 / fp32 output, which must hold the exact sum.  The expected values come from
numpy's float64 matmul, exact here (|sum| <= 9 K < 2^24).  Each call also runs through
tv_hip_gemm_noalloc, which must give the same sums without a workspace (or decline with
TV_E_SCRATCH when the GEMV's partials exceed its static scratch).
"""
import ctypes

import numpy as np
import pytest
import torch

from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT16, FLOAT32, INT8, INT32, to_storage, to_torch

pytestmark = pytest.mark.gpu

DTYPES = [FLOAT32, BFLOAT16, FLOAT16, INT8]


def _cases(n, seed, mn, k, max_macs, dtypes=DTYPES):
    """n calls with M, N log-uniform in [mn[0], mn[1]] and K in [k[0], k[1]], at most max_macs
    multiply-adds each (keeps the host-side reference and the sweep to seconds)."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = dtypes[len(out) % len(dtypes)]
        M, N = (int(np.exp(r.uniform(np.log(mn[0]), np.log(mn[1])))) for _ in range(2))
        K = int(np.exp(r.uniform(np.log(k[0]), np.log(k[1]))))
        batch = int(r.choice([0, 0, 1, 3]))
        bcast = batch > 0 and bool(r.integers(2))
        at, bt = bool(r.integers(2)), bool(r.integers(2))
        if max(batch, 1) * M * N * K > max_macs:
            continue
        out.append((dt, batch, M, N, K, bcast, at, bt))
    return out


# Any size from 1 (GEMVs, small K, tiny tiles), then tile-sized shapes (128x128 / 256x256 tiles,
# stream-K and chained schedules, the fp32 tile choice), then shapes of hundreds of tiles (the
# boundaries between one round of tiles, several, and the schedules that split them), then long K
# (the GEMVs' K slices and x staging, the split-K schedules; fp16 is left out there, since sums of
# that many terms leave its range).
CASES = (_cases(48, 20261202, (1, 3000), (1, 3000), 1.5e8) + _cases(24, 20261203, (200, 2600), (16, 2048), 4e8)
         + _cases(16, 20261207, (1000, 4500), (48, 4096), 4e9)
         + _cases(12, 20261209, (1, 600), (4000, 120000), 4e8, [FLOAT32, BFLOAT16, INT8]))


def _enc(x, dt):
    if dt == INT8:
        return x.astype(np.int8)
    if dt == FLOAT32:
        return x.astype(np.float32)
    return rng.f32_to_bf16_bits(x.astype(np.float32)) if dt == BFLOAT16 else rng.f32_to_f16_bits(x.astype(np.float32))


def _dev(x, dt, transposed):
    """Device tensor holding x; transposed: stored as x^T (last two axes) and viewed back."""
    if transposed:
        return to_torch(np.ascontiguousarray(_enc(np.swapaxes(x, -1, -2), dt)), dt).transpose(-1, -2)
    return to_torch(np.ascontiguousarray(_enc(x, dt)), dt)


def _expect(x, y, dt, wide):
    s = np.matmul(x.astype(np.float64), y.astype(np.float64))
    if dt == INT8:
        # the full int32 sum, or its low byte (two's complement)
        return s.astype(np.int32) if wide else s.astype(np.int64).astype(np.int8)
    return s.astype(np.float32) if wide else _enc(s.astype(np.float32), dt)


def _wide(case):
    """Every third int8 / half call asks for the widened output (int32 / fp32) the C-ABI offers."""
    dt, batch, M, N, K = case[:5]
    return dt != FLOAT32 and (M + N + K) % 3 == 0


def _name(c):
    dt, batch, M, N, K, bcast, at, bt = c
    nm = {FLOAT32: "fp32", BFLOAT16: "bf16", FLOAT16: "fp16", INT8: "int8"}[dt]
    lead = f"b{batch}{'bc' if bcast else ''}-" if batch else ""
    return f"{nm}-{lead}{M}x{N}x{K}-{'AT' if at else 'A'}{'BT' if bt else 'B'}" + ("-wide" if _wide(c) else "")


@pytest.mark.parametrize("case", CASES, ids=[_name(c) for c in CASES])
def test_random_call_exact(hip, case):
    dt, batch, M, N, K, bcast, at, bt = case
    seed = 7 * M + 11 * N + 13 * K + 17 * batch + 2 * at + bt
    lead = (batch,) if batch else ()
    x = rng.uniform_int(seed, int(np.prod(lead + (M, K))), -3, 3).reshape(lead + (M, K))
    yshape = (K, N) if bcast or not batch else lead + (K, N)
    y = rng.uniform_int(seed + 1, int(np.prod(yshape)), -3, 3).reshape(yshape)
    ta, tb = _dev(x, dt, at), _dev(y, dt, bt)
    wide = _wide(case)
    c = hip.gemm(ta, tb, out_dtype=(INT32 if dt == INT8 else FLOAT32) if wide else None)
    torch.cuda.synchronize()
    want = _expect(x, y, dt, wide)
    np.testing.assert_array_equal(to_storage(c), want, err_msg=_name(case))
    # tv_hip_gemm_noalloc on the same call: no workspace (no stream-K split, no padded copies, the
    # GEMV's partials in the static scratch), the same exact sums.
    plain = torch.full_like(c, 7)
    args = hip.make_args(ta, tb, plain)
    rc = hip.lib().tv_hip_gemm_noalloc(ctypes.byref(args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc in (hip.TV_OK, hip.TV_E_SCRATCH), hip.strerror(rc)
    torch.cuda.synchronize()
    if rc == hip.TV_OK:
        np.testing.assert_array_equal(to_storage(plain), want, err_msg=_name(case) + " (no-allocation entry)")
