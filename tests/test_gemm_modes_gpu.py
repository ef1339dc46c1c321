"""GPU parity sweep of the direct-load GEMM over its four operand layouts (A K- or M-contiguous, B
N- or K-contiguous, i.e. plain and transposed views) for bf16, fp16 and int8, at seeded ragged
shapes (M, N and K not multiples of the 256 x 256 tile or of the k-tile), plus batched and
B-broadcast calls.  Inputs are small integers, so every accumulation order gives the same fp32 /
int32 sum: the results must equal the oracle bit for bit (half outputs: the exact sum rounded
once; int8: the low byte)."""
import numpy as np
import pytest
import torch

import oracle as orc
from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT16, INT8, to_storage, to_torch

pytestmark = pytest.mark.gpu


def ints(seed, shape, lo=-3, hi=3):
    return rng.uniform_int(seed, int(np.prod(shape)), lo, hi).astype(np.float32).reshape(shape)


def enc(x, dt):
    if dt == INT8:
        return x.astype(np.int8)
    return rng.f32_to_bf16_bits(x) if dt == BFLOAT16 else rng.f32_to_f16_bits(x)


def dev(x, dt, transposed):
    """Device tensor holding x; transposed: stored as x^T and viewed back (the other layout)."""
    if transposed:
        return to_torch(np.ascontiguousarray(enc(np.swapaxes(x, -1, -2), dt)), dt).transpose(-1, -2)
    return to_torch(np.ascontiguousarray(enc(x, dt)), dt)


def expect(x, y, dt):
    ref = orc.mul(enc(x, dt), dt, enc(y, dt), dt)
    return ref if dt == INT8 else enc(ref, dt)


SHAPES = [(1, 1, 1), (257, 255, 129), (300, 520, 65), (511, 97, 700), (64, 300, 256), (600, 17, 384)]


@pytest.mark.parametrize("dt", [BFLOAT16, FLOAT16, INT8], ids=["bf16", "fp16", "int8"])
@pytest.mark.parametrize("at,bt", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["A_rowmajor-B_rowmajor", "A_T-B_rowmajor", "A_rowmajor-B_T", "A_T-B_T"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_layouts_ragged(hip, dt, at, bt, shape):
    M, N, K = shape
    seed = M * 7 + N * 13 + K * 17 + 2 * at + bt
    x, y = ints(seed, (M, K)), ints(seed + 1, (K, N))
    c = hip.gemm(dev(x, dt, at), dev(y, dt, bt))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_storage(c), expect(x, y, dt))


@pytest.mark.parametrize("dt", [BFLOAT16, INT8], ids=["bf16", "int8"])
@pytest.mark.parametrize("bt", [False, True], ids=["B_rowmajor", "B_T"])
def test_batched_and_broadcast(hip, dt, bt):
    Bn, M, N, K = 3, 270, 300, 200
    x = ints(90 + bt, (Bn, M, K))
    yb = ints(91 + bt, (Bn, K, N))
    y1 = ints(92 + bt, (K, N))
    c = hip.gemm(dev(x, dt, False), dev(yb, dt, bt))
    c1 = hip.gemm(dev(x, dt, False), dev(y1, dt, bt))  # B broadcast over the batch
    torch.cuda.synchronize()
    got, got1 = to_storage(c), to_storage(c1)
    for i in range(Bn):
        np.testing.assert_array_equal(got[i], expect(x[i], yb[i], dt))
        np.testing.assert_array_equal(got1[i], expect(x[i], y1, dt))
