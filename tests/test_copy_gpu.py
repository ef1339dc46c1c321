"""GPU test of the host <-> device boundary of the C++ API (reference copy_host_to_device /
copy_device_to_host, include/backend/cuda/cuda_copy.cpp:9-26, and the factory's host -> device deep
copy, cuda_tensor.cpp:14-33): tests/cpp/copy_driver.cpp round-trips host bytes through a HIP tensor
at sizes below, at and across the 4 MiB direct-copy threshold and the 16 MiB pinned staging chunk
(ragged last chunks included); every byte must come back unchanged."""
import subprocess

import pytest

from tests.cpp import build as cpp

pytestmark = pytest.mark.gpu

SIZES = [1, 1000, 4 * 2**20 - 1, 4 * 2**20, 16 * 2**20, 16 * 2**20 + 3, 32 * 2**20 + 17, 40 * 2**20 + 12345,
         24 * 2**20 + 5, 17 * 2**20 + 4]


@pytest.fixture(scope="module")
def copy_run():
    r = subprocess.run([str(cpp.binary("copy_driver"))], capture_output=True, text=True, timeout=300)
    return r


def test_exit_status(copy_run):
    assert copy_run.returncode == 0, copy_run.stdout + copy_run.stderr


@pytest.mark.parametrize("nbytes", SIZES)
def test_round_trip(copy_run, nbytes):
    assert f"ok {nbytes}" in copy_run.stdout.splitlines(), copy_run.stdout + copy_run.stderr
