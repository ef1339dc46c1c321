"""GPU parity of the strided -> contiguous copy (tv_hip_repack: HIPTensor::clone_as_contiguous and the
materialising ops::Transpose; reference RepackImpl<CUDA>, src/backend/cuda/repack.cu:5-54, and
CPUTensor::clone_as_contiguous, include/backend/cpu/cpu_tensor.cpp:32-63).

The expected bytes are the same view gathered on the host from a copy of the source storage
(numpy as_strided over the storage bytes), so the check is bit-exact for every element size.  The
cases cover each kernel the launcher picks: 16-byte rows (contiguous innermost dimension, including
slices and a stride-0 broadcast), the LDS-tiled transpose of the last two dimensions (ragged tiles,
1/2/4/8-byte elements, outer batch dimensions with offsets), and the per-element gather (rows that
are not whole 16-byte chunks, general permutations)."""
import ctypes

import numpy as np
import pytest

import tensorvia_amd as tv

pytestmark = pytest.mark.gpu

DT = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


def run_case(storage_elems, es, shape, strides, offset, seed):
    import torch
    rng = np.random.default_rng(seed)
    host = rng.integers(0, 2**63 - 1, size=storage_elems, dtype=np.uint64).astype(DT[es])
    src = torch.from_numpy(host.view(np.uint8).copy()).cuda()
    numel = int(np.prod(shape)) if shape else 1
    dst = torch.zeros(max(numel * es, 1), dtype=torch.uint8, device="cuda")
    a = tv.TvRepackArgs()
    a.ndim = len(shape)
    a.elem_size = es
    for d, (n, s) in enumerate(zip(shape, strides)):
        a.shape[d] = n
        a.strides[d] = s
    a.src = src.data_ptr() + offset * es
    a.dst = dst.data_ptr()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tv.check(tv.lib().tv_hip_repack(ctypes.byref(a), s))
    torch.cuda.synchronize()
    got = dst.cpu().numpy()[: numel * es].view(DT[es]).reshape(shape)
    view = np.lib.stride_tricks.as_strided(host[offset:], shape=shape, strides=[st * es for st in strides])
    assert np.array_equal(got, view)


@pytest.mark.parametrize("es", [1, 2, 4, 8])
def test_rows_slice(es):
    # base [4, 37, 64 * 16 / es] elements, view [:, 3:20, :]: rows of 1 KB, row stride aligned
    w = 64 * 16 // es
    run_case(4 * 37 * w, es, [4, 17, w], [37 * w, w, 1], 3 * w, seed=es)


def test_rows_broadcast_stride0():
    run_case(256, 4, [5, 3, 64], [0, 64, 1], 0, seed=11)


@pytest.mark.parametrize("es", [1, 2, 4, 8])
@pytest.mark.parametrize("shape_rc", [(64, 64), (130, 70), (1, 200), (7, 1000), (257, 33)])
def test_transpose_last_two(es, shape_rc):
    # K [B, C, R] viewed as K.permute(0, 2, 1): shape [B, R, C], strides [R*C, 1, R]
    R, C = shape_rc
    B = 3
    run_case(B * R * C, es, [B, R, C], [R * C, 1, R], 0, seed=R * 7 + C + es)


def test_transpose_2d_with_offset():
    # a [300, 96] fp16 base, view base[5:, 8:72].t(): shape [64, 295], strides [1, 96], offset 5*96+8
    run_case(300 * 96, 2, [64, 295], [1, 96], 5 * 96 + 8, seed=21)


def test_transpose_c4_shape():
    # config 4's K.permute(0, 2, 1): K fp16 [32, 2048, 128] -> [32, 128, 2048]
    run_case(32 * 2048 * 128, 2, [32, 128, 2048], [2048 * 128, 1, 128], 0, seed=4)


@pytest.mark.parametrize("es", [2, 4])
def test_element_ragged_rows(es):
    # innermost contiguous but 7 elements a row: not whole 16-byte chunks
    run_case(11 * 9, es, [11, 7], [9, 1], 2, seed=31 + es)


def test_element_general_permute():
    # [4, 5, 6] viewed as permute(2, 0, 1): shape [6, 4, 5], strides [1, 30, 6]
    run_case(4 * 5 * 6, 4, [6, 4, 5], [1, 30, 6], 0, seed=41)


def test_misaligned_source_falls_back():
    # a 16-byte-row view whose base is 2 bytes off 16-byte alignment
    run_case(4 * 64 + 1, 2, [4, 64], [64, 1], 1, seed=51)


def _random_views(n=60, seed=20261206):
    """Seeded random views of a random base tensor: rank 1 to 4, a random permutation of the base's
    axes, a random slice (start, stop, step 1 to 3) of each, sometimes one axis broadcast with
    stride 0; element sizes 1, 2, 4 and 8 bytes."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        es = int(r.choice([1, 2, 4, 8]))
        rank = int(r.integers(1, 5))
        base = [int(np.exp(r.uniform(0, np.log(300 if rank <= 2 else 40)))) for _ in range(rank)]
        bstr = [int(np.prod(base[d + 1:])) for d in range(rank)]  # row-major element strides
        shape, strides, offset = [], [], 0
        for d in range(rank):
            step = int(r.choice([1, 1, 1, 2, 3]))
            lo = int(r.integers(0, base[d]))
            hi = int(r.integers(lo + 1, base[d] + 1))
            shape.append(len(range(lo, hi, step)))
            strides.append(bstr[d] * step)
            offset += lo * bstr[d]
        perm = [int(p) for p in r.permutation(rank)]
        shape, strides = [shape[p] for p in perm], [strides[p] for p in perm]
        if rank > 1 and r.integers(4) == 0:
            d = int(r.integers(rank))
            shape[d], strides[d] = int(r.integers(1, 6)), 0
        if int(np.prod(shape)) * es > (64 << 20):
            continue
        out.append((int(np.prod(base)), es, shape, strides, offset))
    return out


RANDOM_VIEWS = _random_views()


@pytest.mark.parametrize("case", RANDOM_VIEWS, ids=[f"es{c[1]}-{'x'.join(map(str, c[2]))}-s{'_'.join(map(str, c[3]))}"
                                                    for c in RANDOM_VIEWS])
def test_random_views(case):
    """clone_as_contiguous of seeded random views (permuted, sliced with steps, broadcast):
    bit-exact against the same view gathered on the host."""
    storage, es, shape, strides, offset = case
    run_case(storage, es, shape, strides, offset, seed=len(shape) * 1000 + offset % 997)
