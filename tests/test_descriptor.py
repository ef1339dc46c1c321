"""CPU emulation of the C-ABI descriptor (tv_gemm_args) that every GPU test builds with make_args.

include/tensorvia_hip.h states the semantics: element (b, m, k) of A lives at
A + b*sa_b + m*sa_m + k*sa_k (element units, A already including the view's offset), likewise B and
C, and a batch stride of 0 broadcasts an operand.  Here make_args packs CPU torch views (transposes,
sub-blocks with offsets, column steps, expanded rows, columns and batches, a rank-2 B under a
rank-3 A, an output inside wider rows); the emulation reads the operands back from raw memory
through nothing but the descriptor's pointers, extents and strides, multiplies them, and must equal
torch's own product of the views.  This pins the descriptor convention on the host side.
"""
import ctypes

import numpy as np
import pytest
import torch

import tensorvia_amd as tv


def _np_view(ptr, t, shape, strides):
    """numpy view of `shape` with element `strides` starting at address `ptr` inside t's (float64)
    storage."""
    st = t.untyped_storage()
    flat = np.frombuffer((ctypes.c_char * st.nbytes()).from_address(st.data_ptr()), dtype=np.float64)
    assert (ptr - st.data_ptr()) % 8 == 0 and ptr >= st.data_ptr()
    off = (ptr - st.data_ptr()) // 8
    return np.lib.stride_tricks.as_strided(flat[off:], shape=shape, strides=[s * 8 for s in strides], writeable=False)


def _emulate(args, a, b, c):
    """C as the descriptor describes it, from A and B read through the descriptor alone."""
    batch, M, N, K = args.batch, args.M, args.N, args.K
    A = _np_view(args.A, a, (batch, M, K), (args.sa_b, args.sa_m, args.sa_k)).astype(np.float64)
    B = _np_view(args.B, b, (batch, K, N), (args.sb_b, args.sb_k, args.sb_n)).astype(np.float64)
    got_c = _np_view(args.C, c, (batch, M, N), (args.sc_b, args.sc_m, args.sc_n))
    return A @ B, got_c


def _views(seed):
    """A (view), B (view), C (view) for one seeded case; float64 storage, integer values."""
    r = np.random.default_rng(seed)
    batch = int(r.choice([0, 2, 3]))
    M, K, N = (int(r.integers(1, 40)) for _ in range(3))
    lead = (batch,) if batch else ()

    def make(rows, cols, kind, lead_):
        if kind == "row":
            return torch.from_numpy(r.integers(-5, 6, lead_ + (rows, cols)).astype(np.float64))
        if kind == "trans":
            return torch.from_numpy(r.integers(-5, 6, lead_ + (cols, rows)).astype(np.float64)).transpose(-1, -2)
        if kind == "block":
            pr, pc = int(r.integers(1, 4)), int(r.integers(1, 6))
            big = torch.from_numpy(r.integers(-5, 6, lead_ + (rows + pr + 1, cols + pc + 2)).astype(np.float64))
            return big[..., pr:pr + rows, pc:pc + cols]
        if kind == "step":
            big = torch.from_numpy(r.integers(-5, 6, lead_ + (rows, 2 * cols)).astype(np.float64))
            return big[..., :, ::2]
        if kind == "expand_rows":
            row = torch.from_numpy(r.integers(-5, 6, lead_ + (1, cols)).astype(np.float64))
            return row.expand(*lead_, rows, cols)
        if kind == "expand_cols":
            col = torch.from_numpy(r.integers(-5, 6, lead_ + (rows, 1)).astype(np.float64))
            return col.expand(*lead_, rows, cols)
        raise ValueError(kind)

    kinds = ["row", "trans", "block", "step", "expand_rows", "expand_cols"]
    a = make(M, K, str(r.choice(kinds)), lead)
    if batch and r.integers(3) == 0:  # A's batch expanded (stride 0)
        a = a[:1].expand(batch, M, K)
    b_lead = () if (batch and r.integers(2)) or not batch else lead  # a rank-2 B under a rank-3 A
    b = make(K, N, str(r.choice(kinds)), b_lead)
    cpad = int(r.choice([0, 3]))
    wide = torch.full(lead + (M, N + cpad), 77.0, dtype=torch.float64)
    c = wide[..., cpad:cpad + N] if cpad else wide
    return a, b, c


@pytest.mark.parametrize("seed", range(60))
def test_descriptor_describes_the_views(seed):
    a, b, c = _views(seed)
    args = tv.make_args(a, b, c)
    assert (args.dtype_a, args.dtype_b, args.dtype_c) == (tv.FLOAT64,) * 3
    want, cview = _emulate(args, a, b, c)
    ref = torch.matmul(a, b).numpy()
    np.testing.assert_array_equal(want.reshape(ref.shape), ref)
    # C's descriptor addresses exactly the elements of the output view
    c[...] = torch.arange(c.numel(), dtype=torch.float64).reshape(c.shape)
    np.testing.assert_array_equal(cview.reshape(c.shape), c.numpy())
