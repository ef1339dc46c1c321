"""GPU parity of the fused matmul epilogue (tv_hip_gemm_ex): C = act(A @ B + bias) on the fp32
accumulator, rounded once to the output dtype.

The reference composes ops::Mul, ops::Add(C, bias) (same-shape tensors) and ops::Relu / Silu /
Sigmoid / Tanh (src/backend/cpu/activate.cpp:8-40).  The expected value here is that composition in
fp64 on the same inputs (bias materialised to C's shape), and the bar is the matmul's own bound
widened by the activation's slope (at most 1; the float exp/tanh add a few ulp):

  fp32 out:      |c - ref| <= 1e-5 * sqrt(K) * sum_k |a||b| + 1e-6 * |ref| + 1e-30
  bf16/fp16 out: |c - ref| <= 1e-2 * |ref| + 1e-5 * sqrt(K) * sum_k |a||b| + 1e-3 (half ulp near 0)

Every kernel family the router can pick is covered: the fp32 MFMA kernel, the 16-bit direct-load
kernel (bf16, half output and fp32 output; 128x128 and 256x256 tiles), the small-K persistent kernel (fp16, K = 128, >= 1024
tiles) and both GEMV kernels (matrix-core: bf16 at M = 1 and 8; dot-product: fp32, and bf16
narrower than 64 columns), with per-column, full and batch-broadcast bias.
"""
import ctypes

import numpy as np
import pytest

import tensorvia_amd as tv
from tensorvia_amd import rng
from tensorvia_amd.matmul import storage_to_torch, torch_to_storage

pytestmark = pytest.mark.gpu

ACTS = {tv.ACT_NONE: lambda x: x, tv.ACT_RELU: lambda x: np.maximum(x, 0.0),
        tv.ACT_SILU: lambda x: x / (1.0 + np.exp(-x)), tv.ACT_SIGMOID: lambda x: 1.0 / (1.0 + np.exp(-x)),
        tv.ACT_TANH: np.tanh}
ACT_NAMES = {tv.ACT_NONE: "none", tv.ACT_RELU: "relu", tv.ACT_SILU: "silu", tv.ACT_SIGMOID: "sigmoid",
             tv.ACT_TANH: "tanh"}
NAME = {tv.FLOAT32: "float32", tv.BFLOAT16: "bfloat16", tv.FLOAT16: "float16"}


def to_f64(x, dt):
    if dt == tv.BFLOAT16:
        return rng.bf16_bits_to_f32(x).astype(np.float64)
    if dt == tv.FLOAT16:
        return rng.f16_bits_to_f32(x).astype(np.float64)
    return x.astype(np.float64)


def run_case(dt_in, dt_out, batch, M, K, N, bias_kind, act, bt=False, seed=0, check=None, pad=0, reps=1):
    """`check`: the batches compared against the fp64 reference (default: all).  `pad` > 0: C is the
    first N columns of rows N + pad long, and the padding must come back untouched.  `reps`: the
    call is made that many times, each into a freshly filled C, and every result is checked."""
    import torch
    lead = (batch,) if batch else ()
    a = rng.make("uniform", lead + (M, K), 100 + seed, NAME[dt_in], -1, 1)
    b = rng.make("uniform", lead + ((N, K) if bt else (K, N)), 200 + seed, NAME[dt_in], -1, 1)
    bshape = {"col": (N,), "colb": lead + (1, N), "full": lead + (M, N), "bcast": (M, N), "none": None}[bias_kind]
    bias = None if bshape is None else rng.make("uniform", bshape, 300 + seed, NAME[dt_out], -2, 2)

    ta = storage_to_torch(a, dt_in)
    tb = storage_to_torch(b, dt_in)
    if bt:
        tb = tb.transpose(-1, -2)
    out_torch_dtype = {tv.FLOAT32: torch.float32, tv.BFLOAT16: torch.bfloat16, tv.FLOAT16: torch.float16}[dt_out]
    big = torch.full(lead + (M, N + pad), 3.0, dtype=out_torch_dtype, device="cuda")
    tc = big[..., :N]
    args = tv.make_args(ta, tb, tc)
    ep = tv.TvEpilogue()
    ep.act = act
    tbias = None
    if bias is not None:
        tbias = storage_to_torch(bias, dt_out)
        ep.bias = tbias.data_ptr()
        if bias_kind == "col":
            ep.sbias_b, ep.sbias_m, ep.sbias_n = 0, 0, 1
        elif bias_kind == "colb":  # one column bias per batch
            ep.sbias_b, ep.sbias_m, ep.sbias_n = (N if batch else 0), 0, 1
        elif bias_kind == "full":
            ep.sbias_b, ep.sbias_m, ep.sbias_n = (M * N if batch else 0), N, 1
        else:  # one [M, N] bias for every batch
            ep.sbias_b, ep.sbias_m, ep.sbias_n = 0, N, 1
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for _ in range(reps):
        big.fill_(3.0)
        tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), s))
        torch.cuda.synchronize()
        if pad:
            assert bool((big[..., N:] == 3.0).all()), "the fused store wrote past column N"
        outs.append(to_f64(torch_to_storage(tc), dt_out))

    fa, fb = to_f64(a, dt_in), to_f64(b, dt_in)
    if bt:
        fb = np.swapaxes(fb, -1, -2)
    fbias = None if bias is None else np.broadcast_to(to_f64(bias, dt_out), lead + (M, N))
    if batch and check is not None:
        fa, fb = fa[check], fb[check]
        outs = [c[check] for c in outs]
        fbias = None if fbias is None else fbias[check]
    pre = np.matmul(fa, fb)
    if fbias is not None:
        pre = pre + fbias
    ref = ACTS[act](pre)
    bound = np.matmul(np.abs(fa), np.abs(fb))
    if dt_out == tv.FLOAT32:
        tol = 1e-5 * np.sqrt(K) * bound + 1e-6 * np.abs(ref) + 1e-30
    else:
        tol = 1e-2 * np.abs(ref) + 1e-5 * np.sqrt(K) * bound + 1e-3
    for rep, c in enumerate(outs):
        err = np.abs(c - ref)
        bad = err > tol
        assert not bad.any(), (f"call {rep}: {bad.sum()} of {bad.size} outside the bar; worst err {err.max():.3g}, "
                               f"at {np.unravel_index(np.argmax(err - tol), err.shape)}")


@pytest.mark.parametrize("act", list(ACTS), ids=lambda a: ACT_NAMES[a])
@pytest.mark.parametrize("bias_kind", ["col", "full", "none"])
def test_fp32_mfma_kernel(act, bias_kind):
    run_case(tv.FLOAT32, tv.FLOAT32, 0, 200, 96, 130, bias_kind, act)


@pytest.mark.parametrize("act", [tv.ACT_RELU, tv.ACT_SILU, tv.ACT_SIGMOID])
@pytest.mark.parametrize("bias_kind", ["col", "full", "none"])
def test_fp32_96_row_tile(act, bias_kind):
    """fp32 A[1340, 264] @ B[264, 2100]: the tile cost rule picks the 96x128 tile (238 tiles, the
    last row of tiles 92 rows high); the fused epilogue on it."""
    run_case(tv.FLOAT32, tv.FLOAT32, 0, 1340, 264, 2100, bias_kind, act, seed=41)


@pytest.mark.parametrize("act", list(ACTS), ids=lambda a: ACT_NAMES[a])
@pytest.mark.parametrize("bias_kind", ["col", "full", "bcast"])
def test_bf16_direct_load_kernel(act, bias_kind):
    run_case(tv.BFLOAT16, tv.BFLOAT16, 2, 300, 256, 270, bias_kind, act, seed=1)


@pytest.mark.parametrize("dt_in,dt_out", [(tv.BFLOAT16, tv.BFLOAT16), (tv.FLOAT16, tv.FLOAT16),
                                          (tv.BFLOAT16, tv.FLOAT32)], ids=["bf16", "fp16", "bf16-fp32out"])
@pytest.mark.parametrize("act", list(ACTS), ids=lambda a: ACT_NAMES[a])
@pytest.mark.parametrize("bias_kind", ["col", "colb", "none"])
def test_direct_load_column_bias_vector_rows(dt_in, dt_out, act, bias_kind):
    """Rows of C in whole 16-byte chunks (N = 264, a multiple of 8, inside padded rows of 280): the
    direct-load kernel applies a column bias (shared, or one per batch) and the activation while it
    stages the plain output store.  Ragged tiles in M (300) and N (264); the padding stays as it was."""
    run_case(dt_in, dt_out, 2, 300, 256, 264, bias_kind, act, seed=21, pad=16)


@pytest.mark.parametrize("act", [tv.ACT_SILU, tv.ACT_TANH])
@pytest.mark.parametrize("bias_kind", ["col", "full"])
def test_stream_k_fused(act, bias_kind):
    """The fused epilogue on the stream-K schedules: bf16 with 18 tiles of 128x128 (direct-load
    kernel) and fp32 with 12 tiles of 128x128, both over K long enough to split every tile."""
    run_case(tv.BFLOAT16, tv.BFLOAT16, 0, 300, 4096, 700, bias_kind, act, seed=31)
    run_case(tv.FLOAT32, tv.FLOAT32, 0, 300, 2048, 500, bias_kind, act, seed=32)


@pytest.mark.parametrize("act", [tv.ACT_SILU, tv.ACT_TANH])
def test_streaming_store_repeated(act):
    """Regression: the streaming 16-byte store (inline asm) used to be followed, with no wait
    states, by a VALU write of its first data register (the next chunk's LDS address), so that the
    store now and then wrote that value instead of element 0 (fp32 [300,2048] @ [2048,500] with a
    full bias: 4-20 of 150,000 outputs wrong in 1-5 % of calls).  Every one of 100 calls must pass."""
    run_case(tv.FLOAT32, tv.FLOAT32, 0, 300, 2048, 500, "full", act, seed=32, reps=100)


@pytest.mark.parametrize("act", [tv.ACT_RELU, tv.ACT_SILU])
@pytest.mark.parametrize("N,bt", [(4104, False), (4100, True)], ids=["N4104", "N4100-Bt"])
def test_direct_load_256_tiles_fused(act, N, bt):
    """More 128x128 tiles than fit one round of resident workgroups (561 here): the 16-bit GEMM runs
    153 tiles of 256x256, with the fused column bias and activation; rows of C in whole 16-byte
    chunks (N = 4104), or not (N = 4100, B a K-contiguous view so that it still loads directly)."""
    run_case(tv.BFLOAT16, tv.BFLOAT16, 0, 2100, 256, N, "col", act, bt=bt, seed=41)


@pytest.mark.parametrize("act", [tv.ACT_NONE, tv.ACT_RELU, tv.ACT_SILU, tv.ACT_TANH])
@pytest.mark.parametrize("bias_kind,dt", [("col", tv.BFLOAT16), ("colb", tv.BFLOAT16), ("none", tv.FLOAT16)])
def test_two_tiles_per_cu_fused(act, bias_kind, dt):
    """Two or more 256x256 tiles per CU (8 x 8 x 8 = 512 here, the c3 layout at K = 256), where the
    plain GEMM chains tiles: the fused call runs one workgroup per tile, with the per-column (per
    batch) or no bias and the activation applied as the 16-bit output is staged.  Batches 0 and 7
    are checked against the fp64 composition."""
    run_case(dt, dt, 8, 2048, 256, 2048, bias_kind, act, seed=43, check=[0, 7])


@pytest.mark.parametrize("act", [tv.ACT_RELU, tv.ACT_SILU])
def test_bf16_in_fp32_out(act):
    run_case(tv.BFLOAT16, tv.FLOAT32, 0, 260, 320, 300, "col", act, seed=2)


@pytest.mark.parametrize("act,bias_kind", [(tv.ACT_NONE, "col"), (tv.ACT_RELU, "col"), (tv.ACT_SILU, "full"),
                                           (tv.ACT_SIGMOID, "col"), (tv.ACT_TANH, "full")],
                         ids=["none-col", "relu-col", "silu-full", "sigmoid-col", "tanh-full"])
def test_fp16_small_k_persistent(act, bias_kind):
    # The small-K path needs >= 1024 output tiles: 64 batches of 1024 x 1024 at K = 128, B
    # K-contiguous (a transposed view); batches 0, 37 and 63 are checked.
    run_case(tv.FLOAT16, tv.FLOAT16, 64, 1024, 128, 1024, bias_kind, act, bt=True, seed=3, check=[0, 37, 63])


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("act", list(ACTS), ids=lambda a: ACT_NAMES[a])
def test_gemv(M, act):
    run_case(tv.BFLOAT16, tv.BFLOAT16, 0, M, 2048, 1104, "col", act, seed=4 + M)


@pytest.mark.parametrize("act", [tv.ACT_SILU, tv.ACT_SIGMOID])
def test_gemv_narrow_bf16(act):
    """16-bit W narrower than 64 columns runs on the dot-product GEMV kernel (wider W on the
    matrix-core kernel, test_gemv above)."""
    run_case(tv.BFLOAT16, tv.BFLOAT16, 0, 3, 512, 40, "full", act, seed=14)


@pytest.mark.parametrize("act", [tv.ACT_RELU, tv.ACT_TANH])
def test_fp32_gemv(act):
    """M <= 8 with fp32 inputs: the GEMV's fp32 path applies the epilogue per output value."""
    run_case(tv.FLOAT32, tv.FLOAT32, 0, 4, 512, 300, "full", act, seed=12)


def test_column_strided_output_is_rejected():
    """The fused store writes rows of C: a column-strided C (sc_n != 1) on the GEMM path is refused
    before any launch, and C is left untouched."""
    import torch
    a = storage_to_torch(rng.make("uniform", (64, 96), 13, "bfloat16"), tv.BFLOAT16)
    b = storage_to_torch(rng.make("uniform", (96, 80), 14, "bfloat16"), tv.BFLOAT16)
    ct = torch.zeros((80, 64), dtype=torch.bfloat16, device="cuda")
    args = tv.make_args(a, b, ct.t())  # C[m, n] at m + 64 n
    ep = tv.TvEpilogue()
    ep.act = tv.ACT_RELU
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), s) == tv.TV_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert not ct.any()


def test_no_epilogue_equals_plain_gemm():
    """ep = NULL and act = NONE without bias are the plain matmul, bit for bit."""
    import torch
    a = storage_to_torch(rng.make("uniform", (130, 200), 7, "bfloat16"), tv.BFLOAT16)
    b = storage_to_torch(rng.make("uniform", (200, 250), 8, "bfloat16"), tv.BFLOAT16)
    ref = tv.gemm(a, b)
    out = torch.empty_like(ref)
    args = tv.make_args(a, b, out)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), None, s))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    ep = tv.TvEpilogue()
    out.zero_()
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), s))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("act", [tv.ACT_RELU, tv.ACT_SILU, tv.ACT_SIGMOID, tv.ACT_TANH], ids=lambda a: ACT_NAMES[a])
@pytest.mark.parametrize("dt,M,K,N", [(tv.FLOAT32, 64, 96, 80), (tv.BFLOAT16, 300, 256, 272), (tv.BFLOAT16, 1, 512, 128),
                                      (tv.FLOAT32, 3, 512, 96)], ids=["f32_gemm", "bf16_gemm", "bf16_gemv", "f32_gemv"])
def test_infinite_bias_gives_the_activation_limits(act, dt, M, K, N):
    """A per-column bias of +inf / -inf in some columns: the activation's limits, as the reference's
    composition gives them (sigmoid 1 / 0, tanh +1 / -1, relu inf / 0, silu inf / NaN)."""
    import torch
    a = rng.make("uniform", (M, K), 41, NAME[dt], -1, 1)
    b = rng.make("uniform", (K, N), 42, NAME[dt], -1, 1)
    bias = np.zeros(N, dtype=np.float32)
    bias[0::4] = np.inf
    bias[1::4] = -np.inf
    bias_st = rng.f32_to_bf16_bits(bias) if dt == tv.BFLOAT16 else bias
    ta, tb = storage_to_torch(a, dt), storage_to_torch(b, dt)
    tbias = storage_to_torch(bias_st, dt)
    tc = torch.zeros((M, N), dtype=ta.dtype, device="cuda")
    args = tv.make_args(ta, tb, tc)
    ep = tv.TvEpilogue()
    ep.act = act
    ep.bias = tbias.data_ptr()
    ep.sbias_b, ep.sbias_m, ep.sbias_n = 0, 0, 1
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tv.check(tv.lib().tv_hip_gemm_ex(ctypes.byref(args), ctypes.byref(ep), s))
    torch.cuda.synchronize()
    c = to_f64(torch_to_storage(tc), dt)
    with np.errstate(all="ignore"):
        pre = np.matmul(to_f64(a, dt), to_f64(b, dt)) + bias.astype(np.float64)
        ref = ACTS[act](pre)
    inf_cols = np.isinf(bias)
    np.testing.assert_array_equal(c[:, inf_cols], ref[:, inf_cols])  # NaN == NaN here
    assert np.isfinite(c[:, ~inf_cols]).all()


def _random_epilogue_cases(n=40, seed=20261205):
    """Seeded random fused calls: dtype pair, batch, shape (M, N, K log-uniform from 1 to about
    1500), bias layout, activation and B's layout."""
    r = np.random.default_rng(seed)
    pairs = [(tv.FLOAT32, tv.FLOAT32), (tv.BFLOAT16, tv.BFLOAT16), (tv.FLOAT16, tv.FLOAT16), (tv.BFLOAT16, tv.FLOAT32)]
    out = []
    while len(out) < n:
        dt_in, dt_out = pairs[len(out) % 4]
        M, N, K = (int(np.exp(r.uniform(0, np.log(1500)))) for _ in range(3))
        batch = int(r.choice([0, 0, 2]))
        if max(batch, 1) * M * N * K > 4e7:
            continue
        kinds = ["col", "full", "none"] + (["colb", "bcast"] if batch else [])
        out.append((dt_in, dt_out, batch, M, K, N, str(r.choice(kinds)), int(r.choice(list(ACTS))), bool(r.integers(2))))
    return out


RANDOM_EPILOGUE = _random_epilogue_cases()


@pytest.mark.parametrize("case", RANDOM_EPILOGUE, ids=[
    f"{NAME[c[0]]}-{NAME[c[1]]}-b{c[2]}-{c[3]}x{c[5]}x{c[4]}-{c[6]}-{ACT_NAMES[c[7]]}{'-bt' if c[8] else ''}"
    for c in RANDOM_EPILOGUE])
def test_random_fused_calls(case):
    """The fused epilogue on seeded random calls (every kernel family the router picks for them)
    against the fp64 composition act(A @ B + bias), within the matmul's own bound."""
    dt_in, dt_out, batch, M, K, N, bias_kind, act, bt = case
    run_case(dt_in, dt_out, batch, M, K, N, bias_kind, act, bt=bt, seed=7 * M + 11 * N + 13 * K)
