"""GPU parity of the C++ API end to end: seeded ops::Random on the HIP device, views (transposes,
slices with offsets, batch broadcast), ops::Mul through MulImpl<Device::HIP>, to_host().

One driver process runs every case (tests/cpp/mul_driver.cpp); each test then checks one case:
the device-generated operands equal tensorvia_amd/rng.py's bit for bit, and C meets the bar of
its dtype against the CPU oracle / fp64 on the same views: integers bit-exact, fp32 within
1e-5*sqrt(K) of sum_k |a||b|, bf16/fp16 within 1e-2 relative of the fp32-accumulated value.
"""
import re
import subprocess

import numpy as np
import pytest

import oracle as orc
from tensorvia_amd import rng
from tests.cpp import build as cpp
from tests.util import (BFLOAT16, FLOAT16, FLOAT32, INT8, INT32, assert_fp32_close, assert_half_close, to_f32)

pytestmark = pytest.mark.gpu

NAMES = {INT8: "int8", INT32: "int32", BFLOAT16: "bfloat16", FLOAT16: "float16", FLOAT32: "float32"}
STORAGE = {INT8: np.int8, INT32: np.int32, BFLOAT16: np.uint16, FLOAT16: np.uint16, FLOAT32: np.float32}

# name, dtype_a, dtype_b, layout, batch, M, K, N, lo, hi, seed_a, seed_b
CASES = [
    ("i8_contig", INT8, INT8, "contig", 0, 300, 520, 270, -128, 127, 1, 2),
    ("i8_range10_bt", INT8, INT8, "bt", 0, 512, 512, 512, -10, 10, 3, 4),
    ("i8_batched_slice", INT8, INT8, "slice", 3, 77, 200, 130, -128, 127, 5, 6),
    ("f32_contig", FLOAT32, FLOAT32, "contig", 0, 259, 300, 515, -1, 1, 7, 8),
    ("f32_a_transposed", FLOAT32, FLOAT32, "at", 0, 192, 256, 320, -1, 1, 9, 10),
    ("f32_batched_slice", FLOAT32, FLOAT32, "slice", 2, 100, 130, 70, -1, 1, 11, 12),
    ("bf16_broadcast_b", BFLOAT16, BFLOAT16, "bcast", 3, 130, 256, 200, -1, 1, 13, 14),
    ("f16_permuted_b", FLOAT16, FLOAT16, "bt", 4, 128, 128, 256, -1, 1, 15, 16),
    ("bf16_gemv_m1", BFLOAT16, BFLOAT16, "contig", 0, 1, 4096, 1104, -1, 1, 17, 18),
    ("bf16_gemv_m8", BFLOAT16, BFLOAT16, "contig", 0, 8, 1024, 2048, -1, 1, 19, 20),
    ("f16_b_transposed_2d", FLOAT16, FLOAT16, "bt", 0, 96, 160, 72, -1, 1, 21, 22),
    ("i32_simt", INT32, INT32, "contig", 0, 50, 70, 40, -50, 50, 23, 24),
    ("i32_f32_mixed", INT32, FLOAT32, "contig", 0, 33, 65, 17, -50, 50, 25, 26),
]


def _random_cases(n=24, seed=20261208):
    """Seeded random ops::Mul calls through the C++ API: dtype, layout (contiguous, B broadcast,
    B or A transposed, sliced views with offsets), batch and shape (M, N, K log-uniform)."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = [INT8, FLOAT32, BFLOAT16, FLOAT16][len(out) % 4]
        layout = str(r.choice(["contig", "bcast", "bt", "at", "slice"]))
        batch = int(r.choice([1, 2, 3])) if layout == "bcast" else int(r.choice([0, 0, 2]))
        M, K, N = (int(np.exp(r.uniform(0, np.log(1200)))) for _ in range(3))
        if max(batch, 1) * M * N * K > 5e7:
            continue
        lo, hi = (-128, 127) if dt == INT8 else (-1, 1)
        i = len(out)
        out.append((f"rand{i}_{NAMES[dt]}_{layout}", dt, dt, layout, batch, M, K, N, lo, hi, 100 + 2 * i, 101 + 2 * i))
    return out


CASES += _random_cases()
# K = 0 cannot reach ops::Mul: a tensor with a zero-sized dimension is rejected when it is built
# (calc_numel, reference include/core/type_traits.h:296; tests/cpp/host_api_test.cpp checks it).
# The C-ABI serves K = 0 (tests/test_edge_gpu.py).


def _base_shapes(layout, batch, M, K, N):
    lead = (batch,) if batch else ()
    if layout == "contig":
        return lead + (M, K), lead + (K, N)
    if layout == "bcast":
        return lead + (M, K), (K, N)
    if layout == "bt":
        return lead + (M, K), lead + (N, K)
    if layout == "at":
        return lead + (K, M), lead + (K, N)
    if layout == "slice":
        return lead + (M + 3, K + 5), lead + (K + 2, N + 4)
    raise ValueError(layout)


def _views(layout, a, b, M, K, N):
    """numpy views matching the driver's, as dense arrays [b?, M, K] and [b?, K, N]."""
    sw = lambda x: np.swapaxes(x, -1, -2)  # noqa: E731
    if layout == "bt":
        b = sw(b)
    elif layout == "at":
        a = sw(a)
    elif layout == "slice":
        a, b = a[..., 1:M + 1, 2:K + 2], b[..., 1:K + 1, 3:N + 3]
    if layout == "bcast":
        b = np.broadcast_to(b, (a.shape[0],) + b.shape)
    return np.ascontiguousarray(a), np.ascontiguousarray(b)


@pytest.fixture(scope="module")
def driver_run(tmp_path_factory):
    out = tmp_path_factory.mktemp("cpp_mul")
    casefile = out / "cases.txt"
    casefile.write_text("".join(" ".join(str(v) for v in c) + "\n" for c in CASES))
    r = subprocess.run([str(cpp.binary("mul_driver")), str(casefile), str(out)], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-4000:], r.stderr[-4000:], flush=True)
    done = {m.group(1): int(m.group(2)) for m in re.finditer(r"^done (\S+) dtype (\d+)$", r.stdout, re.M)}
    return r, out, done


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_cpp_mul_case(driver_run, case):
    r, out, done = driver_run
    name, dta, dtb, layout, batch, M, K, N, lo, hi, sa, sb = case
    assert name in done, f"driver did not finish {name}:\n{r.stdout[-3000:]}"
    dtc = done[name]
    assert dtc == orc.compute_type(dta, dtb)

    sha, shb = _base_shapes(layout, batch, M, K, N)
    a = rng.make("uniform", sha, sa, NAMES[dta], lo, hi)
    b = rng.make("uniform", shb, sb, NAMES[dtb], lo, hi)
    got_a = np.fromfile(out / f"{name}_a.bin", dtype=STORAGE[dta]).reshape(sha)
    got_b = np.fromfile(out / f"{name}_b.bin", dtype=STORAGE[dtb]).reshape(shb)
    np.testing.assert_array_equal(got_a, a, err_msg="device Random differs from the host generator")
    np.testing.assert_array_equal(got_b, b, err_msg="device Random differs from the host generator")

    va, vb = _views(layout, a, b, M, K, N)
    out_shape = ((batch,) if batch else ()) + (M, N)
    c = np.fromfile(out / f"{name}_c.bin", dtype=STORAGE[dtc]).reshape(out_shape)
    if dtc in (INT8, INT32):
        np.testing.assert_array_equal(c, orc.mul(va, dta, vb, dtb))
        return
    fa = to_f32(va, dta).astype(np.float64)
    fb = to_f32(vb, dtb).astype(np.float64)
    ref = np.matmul(fa, fb)
    bound = np.matmul(np.abs(fa), np.abs(fb))
    if dtc == FLOAT32:
        assert_fp32_close(c, ref, bound, K)
    else:
        assert_half_close(to_f32(c, dtc), ref, bound, K)


def test_cpp_driver_exit_status(driver_run):
    r, _, _ = driver_run
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
