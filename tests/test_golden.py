"""The oracle reproduces every committed golden vector (CPU)."""
import numpy as np
import pytest

import oracle as orc
from tests import golden
from tests.util import BFLOAT16, FLOAT16, FLOAT32, INT8, INT32

CASES = golden.load()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_golden(name):
    case = CASES[name]
    dta, dtb, dtc, layout = (int(v) for v in case["meta"])
    a, b, c = case["a"], case["b"], case["c"]
    if layout == 1:  # B given as K[b, n, k]; the CPU path needs the materialised transpose
        b = orc.transpose_last2(b)
    got = orc.mul(a, dta, b, dtb)
    if dtc in (INT8, FLOAT32) and got.dtype == c.dtype:
        np.testing.assert_array_equal(got, c)
    elif dtc == INT32:
        # CPU result dtype is int8 for int8 inputs; its value is the low byte of the int32 sum
        np.testing.assert_array_equal(got, orc.low_byte(c))
    else:
        # half outputs: the CPU returns fp32; the golden is that fp32 value rounded once
        from tensorvia_amd import rng
        rounded = rng.f32_to_bf16_bits(got) if dtc == BFLOAT16 else rng.f32_to_f16_bits(got)
        np.testing.assert_array_equal(rounded, c)
        assert dtc in (BFLOAT16, FLOAT16)
