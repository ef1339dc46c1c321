"""GPU parity sweep over seeded random views: ops::Mul's operands reach the kernels as strided views
(Metadata: shape, element strides, offset), so each operand is drawn from a row-major tensor, a
transposed view, a sub-block of a larger tensor (offset and row stride), every other column (a
stride of 2 along the contiguous dimension), a row or column expanded with stride 0, and, with a
batch, a batch expanded with stride 0; B may be one matrix broadcast over A's batch.  C is a fresh
tensor or N columns of wider rows, starting at column 0, 1 or 2 (an unaligned start), and the
columns around it must come back untouched.

Integer inputs in [-3, 3] make every accumulation order exact: fp32 outputs equal the exact sum,
half outputs the exact sum rounded once, int8 outputs its low byte, bit for bit.
"""
import numpy as np
import pytest
import torch

from tensorvia_amd import rng
from tests.util import BFLOAT16, FLOAT16, FLOAT32, INT8, to_storage, to_torch

pytestmark = pytest.mark.gpu

DTYPES = [FLOAT32, BFLOAT16, FLOAT16, INT8]
A_LAYOUTS = ["row", "trans", "block", "step", "expand"]
B_LAYOUTS = ["row", "trans", "block", "step", "expand"]
TORCH_DT = {FLOAT32: torch.float32, BFLOAT16: torch.bfloat16, FLOAT16: torch.float16, INT8: torch.int8}


def _cases(n=60, seed=20261204, max_macs=6e7):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = DTYPES[len(out) % 4]
        M, N, K = (int(np.exp(r.uniform(0, np.log(1500)))) for _ in range(3))
        batch = int(r.choice([0, 0, 2, 3]))
        if max(batch, 1) * M * N * K > max_macs:
            continue
        la, lb = str(r.choice(A_LAYOUTS)), str(r.choice(B_LAYOUTS))
        bcast = batch > 0 and bool(r.integers(2))
        a_bexp = batch > 0 and bool(r.integers(3) == 0)  # A's batch expanded (stride 0)
        cpad = int(r.choice([0, 0, 3, 16]))
        out.append((dt, batch, M, N, K, la, lb, bcast, a_bexp, cpad))
    return out


CASES = _cases()


def _name(c):
    dt, batch, M, N, K, la, lb, bcast, a_bexp, cpad = c
    nm = {FLOAT32: "fp32", BFLOAT16: "bf16", FLOAT16: "fp16", INT8: "int8"}[dt]
    lead = f"b{batch}{'bc' if bcast else ''}{'ax' if a_bexp else ''}-" if batch else ""
    return f"{nm}-{lead}{M}x{N}x{K}-A{la}-B{lb}" + (f"-cpad{cpad}" if cpad else "")


def _enc(x, dt):
    if dt == INT8:
        return x.astype(np.int8)
    if dt == FLOAT32:
        return x.astype(np.float32)
    return rng.f32_to_bf16_bits(x.astype(np.float32)) if dt == BFLOAT16 else rng.f32_to_f16_bits(x.astype(np.float32))


def _view(logical, dt, layout, seed):
    """A device view whose values equal `logical` (shape [..., R, C]: R the row dimension, C the
    contiguous one of a row-major matrix), laid out as `layout`.  For "expand" the logical array
    must be constant along the rows (built by the caller)."""
    if layout == "row":
        return to_torch(np.ascontiguousarray(_enc(logical, dt)), dt)
    if layout == "trans":
        return to_torch(np.ascontiguousarray(_enc(np.swapaxes(logical, -1, -2), dt)), dt).transpose(-1, -2)
    if layout == "block":
        *lead, R, C = logical.shape
        r = np.random.default_rng(seed)
        pr, pc = int(r.integers(1, 5)), int(r.integers(1, 9))
        big = rng.uniform_int(seed + 5, int(np.prod(lead + [R + pr, C + pc])), -3, 3).reshape(lead + [R + pr, C + pc])
        big[..., pr:pr + R, pc:pc + C] = logical
        return to_torch(np.ascontiguousarray(_enc(big, dt)), dt)[..., pr:pr + R, pc:pc + C]
    if layout == "step":
        *lead, R, C = logical.shape
        big = np.zeros(lead + [R, 2 * C], dtype=logical.dtype)
        big[..., :, ::2] = logical
        return to_torch(np.ascontiguousarray(_enc(big, dt)), dt)[..., :, ::2]
    if layout == "expand":
        row = logical[..., :1, :]
        return to_torch(np.ascontiguousarray(_enc(row, dt)), dt).expand(*logical.shape)
    raise ValueError(layout)


@pytest.mark.parametrize("case", CASES, ids=[_name(c) for c in CASES])
def test_random_views_exact(hip, case):
    dt, batch, M, N, K, la, lb, bcast, a_bexp, cpad = case
    seed = 3 * M + 5 * N + 7 * K + 11 * batch + 13 * cpad
    lead = (batch,) if batch else ()
    a_lead = (1,) if a_bexp else lead
    x = rng.uniform_int(seed, int(np.prod(a_lead + (M, K))), -3, 3).reshape(a_lead + (M, K))
    if la == "expand":
        x = np.broadcast_to(x[..., :1, :], x.shape).copy()
    b_lead = () if bcast or not batch else lead
    y = rng.uniform_int(seed + 1, int(np.prod(b_lead + (K, N))), -3, 3).reshape(b_lead + (K, N))
    if lb == "expand":  # B's columns expanded: one column, stride 0 along n
        y = np.broadcast_to(y[..., :, :1], y.shape).copy()
        ty = _view(np.swapaxes(y, -1, -2), dt, "expand", seed + 2).transpose(-1, -2)
    else:
        ty = _view(y, dt, lb, seed + 2)
    tx = _view(x, dt, la, seed + 3)
    if a_bexp:
        tx = tx.expand(batch, M, K)
        x = np.broadcast_to(x, lead + (M, K))
    cshape = lead + (M, N)
    coff = (M + N) % 3 if cpad else 0  # C's first column inside the wider rows: an unaligned start
    wide = torch.full(lead + (M, N + cpad), 77, dtype=TORCH_DT[dt], device="cuda")
    c = wide[..., coff:coff + N] if coff + N <= N + cpad else wide[..., :N]
    coff = coff if coff + N <= N + cpad else 0
    hip.gemm(tx, ty, out=c)
    torch.cuda.synchronize()
    s = np.matmul(x.astype(np.float64), y.astype(np.float64))
    want = s.astype(np.int64).astype(np.int8) if dt == INT8 else _enc(s.astype(np.float32), dt)
    np.testing.assert_array_equal(to_storage(c.contiguous()).reshape(cshape), want, err_msg=_name(case))
    if cpad:
        assert bool((wide[..., :coff] == 77).all()), f"{_name(case)}: wrote before C's first column"
        assert bool((wide[..., coff + N:] == 77).all()), f"{_name(case)}: wrote past C's last column"
