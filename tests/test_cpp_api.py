"""The C++ API's host side (no GPU): views, offsets, ops::Mul validation, Typecast, and the seeded
generator, whose streams must equal tensorvia_amd/rng.py's bit for bit."""
import subprocess

import numpy as np
import pytest

from tensorvia_amd import rng
from tests.cpp import build as cpp


@pytest.fixture(scope="module")
def host_run(tmp_path_factory):
    out = tmp_path_factory.mktemp("host_api")
    r = subprocess.run([str(cpp.binary("host_api_test")), str(out)], capture_output=True, text=True, timeout=120)
    return r, out


@pytest.mark.parametrize("check", ["transpose_view_strides", "slice_offset_and_gather", "permute_021_like_config4",
                                   "copy_of_view_is_contiguous", "mul_validation_messages", "parallel_memcpy",
                                   "typecast_widening_exact", "random_streams_dumped"])
def test_host_api_check(host_run, check):
    r, _ = host_run
    assert f"ok {check}" in r.stdout.splitlines(), r.stdout + r.stderr


def test_host_api_exit_status(host_run):
    r, _ = host_run
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("tag,dtype,lo,hi,seed", [("f32", "float32", -1, 1, 1), ("bf16", "bfloat16", -1, 1, 5),
                                                  ("f16", "float16", -0.05, 0.05, 10), ("i8", "int8", -10, 10, 3),
                                                  ("i8full", "int8", -128, 127, 77), ("i32", "int32", -1000, 999, 42)])
def test_cpp_random_matches_python_generator(host_run, tag, dtype, lo, hi, seed):
    _, out = host_run
    n = 4099
    storage = {"float32": np.float32, "bfloat16": np.uint16, "float16": np.uint16, "int8": np.int8,
               "int32": np.int32}[dtype]
    got = np.fromfile(out / f"random_{tag}.bin", dtype=storage)
    # The C++ side takes float bounds: pass the same fp32-rounded values here.
    want = rng.make("uniform", (n,), seed, dtype, float(np.float32(lo)), float(np.float32(hi)))
    np.testing.assert_array_equal(got, want)
    if dtype.startswith("int"):
        assert got.min() == lo and got.max() == hi  # inclusive bounds are reached


def test_libtensorvia_exports_the_plugin_api():
    """libtensorvia.so loads without a GPU and exports the operator and backend entry points."""
    import ctypes

    from tensorvia_amd import build_ext
    ctypes.CDLL(str(build_ext.HOST_LIB))
    names = subprocess.run(["nm", "-D", "-C", "--defined-only", str(build_ext.HOST_LIB)], capture_output=True,
                           text=True, check=True).stdout
    for sym in ["ops::MulImpl<(via::Device)4>::execute(Tensor const&, Tensor const&)",
                "ops::Mul(Tensor const&, Tensor const&)", "ops::matmul(Tensor const&, Tensor const&)",
                "HIPContext::get()", "HIPTensor::clone_as_contiguous(Metadata const&) const",
                "register_tensor_impl(", "copy_device_to_host(", "copy_host_to_device(",
                "ops::Transpose(Tensor const&, std::initializer_list<long>)",
                "ops::Transpose(Tensor const&, Tensor&, std::initializer_list<long>)",
                "ops::TransposeImpl<(via::Device)4>::execute(Tensor const&, Tensor&, std::initializer_list<long>)",
                "ops::Typecast(Tensor const&, via::DataType)"]:
        assert sym in names, sym


@pytest.mark.parametrize("exe,env", [("host_api_test_asan", {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                                                             "UBSAN_OPTIONS": "print_stacktrace=1"}),
                                     ("host_api_test_tsan", {"TSAN_OPTIONS": "halt_on_error=1"})])
def test_host_api_under_sanitizers(tmp_path, exe, env):
    """The same host checks built with the host sources of libtensorvia.so under AddressSanitizer +
    UndefinedBehaviorSanitizer (leak detection on) and under ThreadSanitizer: every check passes and
    no sanitizer reports (tests/cpp/build.py --sanitize builds them; CPU only)."""
    import os
    r = subprocess.run([str(cpp.binary(exe)), str(tmp_path)], capture_output=True, text=True, timeout=300,
                       env={**os.environ, **env})
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "FAIL" not in r.stdout and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
