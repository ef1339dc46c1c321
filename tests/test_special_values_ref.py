"""CPU check of the expectation the special-value GPU tests use (_ieee_matmul in
test_special_values_gpu.py): on small operands with +inf, -inf and NaN entries it must equal a
plain triple loop of IEEE float64 multiply-adds, NaN equal to NaN."""
import numpy as np

from tests.test_special_values_gpu import _ieee_matmul, _operand


def test_ieee_matmul_equals_the_triple_loop():
    for seed in range(40):
        x, y = _operand((5, 7), seed, 3), _operand((7, 6), seed + 100, 3)
        want = np.zeros((5, 6))
        with np.errstate(invalid="ignore"):
            for m in range(5):
                for n in range(6):
                    t = 0.0
                    for k in range(7):
                        t = t + x[m, k] * y[k, n]
                    want[m, n] = t
        np.testing.assert_array_equal(_ieee_matmul(x, y), want, err_msg=str(seed))
    xb, yb = _operand((2, 4, 9), 1, 3), _operand((2, 9, 3), 2, 3)
    got = _ieee_matmul(xb, yb)
    for i in range(2):
        np.testing.assert_array_equal(got[i], _ieee_matmul(xb[i], yb[i]))
