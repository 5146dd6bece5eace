"""Degenerate shapes on the GPU: empty outputs and empty batches.

The reference sizes a convolution's output with safe_out_size
(include/TensorOps.hpp:17-20), which gives 0 when the kernel is larger than
the padded input; its CPU backward then leaves dX and dW at zero and db at
zero (include/TensorOps.hpp:318-415, restated in oracle/oracle.c).  A batch
of zero matrices is an empty bmm.  None of these may launch a kernel over an
empty grid or touch memory outside the (empty) outputs.
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("h,w,k,pad", [(2, 2, 5, 0), (3, 7, 4, 0), (1, 1, 4, 1)])
def test_conv_with_empty_output(dev, h, w, k, pad):
    n, c, co = 2, 3, 4
    ho, wo = oracle.conv_out(h, pad, k, 1), oracle.conv_out(w, pad, k, 1)
    assert ho == 0 or wo == 0
    x = oracle.normal((n, c, h, w), 1)
    wt = oracle.normal((co, c, k, k), 2)
    b = oracle.normal((co,), 3)
    X, W = torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev)
    y = mt.conv2d(X, W, torch.from_numpy(b).to(dev), 1, pad)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (n, co, ho, wo)
    dy = torch.empty((n, co, ho, wo), device=dev)
    dx, dw, db = mt.conv2d_backward(X, W, dy, 1, pad)
    torch.cuda.synchronize()
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, np.zeros((n, co, ho, wo), np.float32), 1, pad)
    np.testing.assert_array_equal(dx.cpu().numpy(), wdx)
    np.testing.assert_array_equal(dw.cpu().numpy(), wdw)
    np.testing.assert_array_equal(db.cpu().numpy(), wdb)
    assert not dx.cpu().numpy().any() and not dw.cpu().numpy().any() and not db.cpu().numpy().any()


def test_bmm_with_empty_batch(dev):
    A = torch.empty((0, 5, 7), device=dev)
    B = torch.empty((0, 7, 3), device=dev)
    C = mt.bmm(A, B)
    torch.cuda.synchronize()
    assert tuple(C.shape) == (0, 5, 3)


def test_one_by_one_by_one(dev):
    a = np.array([[1.5]], np.float32)
    b = np.array([[-2.0]], np.float32)
    c = mt.matmul(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(c, oracle.matmul(a, b))


def test_linear_over_zero_rows(dev):
    # Linear over an empty batch of samples: Y is [0, out]; dX is [0, in],
    # dW = dYᵀ·X sums over no rows (zeros, plus beta·dW) and so does db.
    x = torch.empty((0, 6), device=dev)
    w = torch.from_numpy(oracle.normal((5, 6), 1)).to(dev)
    b = torch.from_numpy(oracle.normal((5,), 2)).to(dev)
    y = mt.linear(x, w, b)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, 5)
    dy = torch.empty((0, 5), device=dev)
    dx, dw, db = mt.linear_backward(dy, x, w)
    torch.cuda.synchronize()
    assert tuple(dx.shape) == (0, 6)
    np.testing.assert_array_equal(dw.cpu().numpy(), np.zeros((5, 6), np.float32))
    np.testing.assert_array_equal(db.cpu().numpy(), np.zeros((5,), np.float32))


def test_conv_over_zero_images(dev):
    x = np.zeros((0, 16, 6, 6), np.float32)
    wt = oracle.normal((16, 16, 3, 3), 1)
    X, W = torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev)
    y = mt.conv2d(X, W, torch.zeros(16, device=dev), 1, 1)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (0, 16, 6, 6)
    dx, dw, db = mt.conv2d_backward(X, W, torch.empty((0, 16, 6, 6), device=dev), 1, 1)
    torch.cuda.synchronize()
    assert tuple(dx.shape) == (0, 16, 6, 6)
    np.testing.assert_array_equal(dw.cpu().numpy(), np.zeros_like(wt))
    np.testing.assert_array_equal(db.cpu().numpy(), np.zeros((16,), np.float32))
