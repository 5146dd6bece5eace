"""CPU: the float64 convolution references of the whole-tensor GPU checks
(fp64_reference.py) against the oracle's restatements of the reference's
conv2d_cpu and conv backward, on small shapes of every stride/padding kind,
and against a planted mistake (a kernel flipped in space), which must fail."""
import numpy as np
import pytest

import fp64_reference as f64
import oracle
from util_parity import amax, assert_close

CASES = [  # n, c, h, w, co, k, stride, pad
    (2, 3, 7, 7, 4, 3, 1, 1), (2, 5, 9, 8, 3, 3, 2, 1), (1, 4, 11, 11, 2, 5, 3, 2),
    (3, 2, 6, 6, 5, 1, 2, 0), (2, 3, 8, 8, 4, 7, 2, 3), (1, 6, 5, 7, 3, 2, 1, 0),
]


@pytest.mark.parametrize("case", CASES)
def test_fp64_conv_matches_oracle(case):
    n, c, h, w, co, k, s, p = case
    x = oracle.normal((n, c, h, w), 1)
    wt = oracle.normal((co, c, k, k), 2)
    b = oracle.normal((co,), 3)
    want = oracle.conv2d(x, wt, b, s, p)
    got = f64.conv2d(x, wt, b, s, p)
    assert_close(got, want, c * k * k, amax(x), amax(wt), "fp64 conv", extra=1e-5)
    ho, wo = want.shape[2:]
    dy = oracle.normal((n, co, ho, wo), 4)
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, s, p)
    dx, dw, db = f64.conv2d_backward(x, wt, dy, s, p)
    assert_close(dx, wdx, co * k * k, amax(dy), amax(wt), "fp64 dX")
    assert_close(dw, wdw, n * ho * wo, amax(dy), amax(x), "fp64 dW")
    assert_close(db, wdb, n * ho * wo, amax(dy), 1.0, "fp64 db")


def test_fp64_conv_planted_flip_fails():
    x = oracle.normal((2, 3, 7, 7), 1)
    wt = oracle.normal((4, 3, 3, 3), 2)
    want = oracle.conv2d(x, wt, None, 1, 1)
    got = f64.conv2d(x, np.ascontiguousarray(wt[:, :, ::-1, ::-1]), None, 1, 1)
    with pytest.raises(AssertionError):
        assert_close(got, want, 27, amax(x), amax(wt), "flipped kernel")


def test_fp64_matmul_is_numpy_exact_product():
    # the whole-matrix GEMM checks use a64 @ b64; pin that form against the
    # oracle's matmul on a ragged shape (transposed operand included)
    a = oracle.uniform((37, 53), 5)
    b = oracle.uniform((41, 53), 6)
    assert_close(a.astype(np.float64) @ b.astype(np.float64).T, oracle.matmul(a, b.T.copy()),
                 53, 1.0, 1.0, "fp64 matmul")
