"""GPU: benchmark configurations 2, 3 and 5a and the 63-row skinny product
checked element-wise over the whole output (forward, and 5a's dX, dW and db)
against float64 products of the same seeded inputs (numpy BLAS;
fp64_reference.py for the convolution, pinned to the CPU oracle in
test_fp64_reference.py).  The oracle itself takes minutes
per full tensor at these sizes; the other tests check them on sampled rows,
channels and images plus size-independent identities.  Bound: the fp32 parity
bound 1e-5 * sqrt(K) * max|a| * max|b| against the exact sum."""
import numpy as np
import pytest
import torch

import fp64_reference as f64
import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_config2_4096_every_element(dev):
    a = oracle.uniform((4096, 4096), 42)
    b = oracle.uniform((4096, 4096), 43)
    c = host(mt.gemm(g(a, dev), g(b, dev)))
    print(f"[config] C2 {mt.last_config()}", flush=True)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert_close(c, want, 4096, amax(a), amax(b), "C2 every element")


def test_config3_views_every_element(dev):
    a = oracle.normal((2048, 1024), 42)
    b = oracle.normal((2048, 1024), 43)
    A, B = g(a, dev), g(b, dev)
    want = a.astype(np.float64) @ b.astype(np.float64).T
    c = host(mt.gemm(A, B.t()))
    print(f"[config] C3a {mt.last_config()}", flush=True)
    assert_close(c, want, 1024, amax(a), amax(b), "C3a every element")
    c = host(mt.gemm(A[128:], B.t()))
    print(f"[config] C3b {mt.last_config()}", flush=True)
    assert_close(c, want[128:], 1024, amax(a), amax(b), "C3b every element")


def test_config5a_forward_and_backward_every_element(dev):
    x = oracle.normal((32, 256, 14, 14), 42)
    w = oracle.normal((256, 256, 3, 3), 43, std=(2.0 / 2304) ** 0.5)
    b = oracle.normal((256,), 45, std=0.1)
    dy = oracle.normal((32, 256, 14, 14), 44, std=0.01)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    y = host(mt.conv2d(X, W, g(b, dev), 1, 1))
    print(f"[config] C5a forward {mt.last_config()}", flush=True)
    assert_close(y, f64.conv2d(x, w, b, 1, 1), 2304, amax(x), amax(w), "C5a forward",
                 extra=1e-6)
    dx, dw, db = (host(t) for t in mt.conv2d_backward(X, W, dY, 1, 1))
    wdx, wdw, wdb = f64.conv2d_backward(x, w, dy, 1, 1)
    assert_close(dx, wdx, 2304, amax(dy), amax(w), "C5a dX every element")
    assert_close(dw, wdw, 32 * 196, amax(dy), amax(x), "C5a dW every element")
    assert_close(db, wdb, 32 * 196, amax(dy), 1.0, "C5a db")


@pytest.mark.parametrize("c_in,c_out,k,pad", [(128, 128, 3, 1), (256, 512, 1, 0)])
def test_resnet_downsampling_layer_every_element(dev, c_in, c_out, k, pad):
    # stride-2 layers at batch 32 on 56x56 (the 3x3 and the 1x1 shortcut of a
    # ResNet stage change): forward, dX (phased), dW + db, every element
    x = oracle.normal((32, c_in, 56, 56), 52)
    w = oracle.normal((c_out, c_in, k, k), 53, std=(2.0 / (c_in * k * k)) ** 0.5)
    X, W = g(x, dev), g(w, dev)
    y = host(mt.conv2d(X, W, None, 2, pad))
    print(f"[config] s2 forward {mt.last_config()}", flush=True)
    assert_close(y, f64.conv2d(x, w, None, 2, pad), c_in * k * k, amax(x), amax(w),
                 "stride-2 forward")
    dy = oracle.normal(y.shape, 54, std=0.01)
    dx, dw, db = (host(t) for t in mt.conv2d_backward(X, W, g(dy, dev), 2, pad))
    wdx, wdw, wdb = f64.conv2d_backward(x, w, dy, 2, pad)
    npix = 32 * y.shape[2] * y.shape[3]
    assert_close(dx, wdx, c_out * k * k, amax(dy), amax(w), "stride-2 dX every element")
    assert_close(dw, wdw, npix, amax(dy), amax(x), "stride-2 dW every element")
    assert_close(db, wdb, npix, amax(dy), 1.0, "stride-2 db")


def test_skinny_63_rows_every_element(dev):
    # the reference benchmark's 63x4096·4096x4096 row (test/benchmark.cpp:738):
    # 64x64 MFMA tiles with split-K over a 63-row ragged tile
    a = oracle.uniform((63, 4096), 46)
    b = oracle.uniform((4096, 4096), 47)
    c = host(mt.gemm(g(a, dev), g(b, dev)))
    print(f"[config] 63 rows {mt.last_config()}", flush=True)
    assert_close(c, a.astype(np.float64) @ b.astype(np.float64), 4096, amax(a), amax(b),
                 "63x4096x4096 every element")


def test_resnet_stem_every_element(dev):
    # the 7x7 stride-2 RGB stem at batch 32 (c_in = 3: forward and dW + db on
    # the input padded with a zero channel, dX phased): every element
    x = oracle.normal((32, 3, 224, 224), 55)
    w = oracle.normal((64, 3, 7, 7), 56, std=(2.0 / 147) ** 0.5)
    b = oracle.normal((64,), 57, std=0.1)
    X, W = g(x, dev), g(w, dev)
    y = host(mt.conv2d(X, W, g(b, dev), 2, 3))
    print(f"[config] stem forward {mt.last_config()}", flush=True)
    assert_close(y, f64.conv2d(x, w, b, 2, 3), 147, amax(x), amax(w), "stem forward",
                 extra=1e-6)
    dy = oracle.normal(y.shape, 58, std=0.01)
    dx, dw, db = (host(t) for t in mt.conv2d_backward(X, W, g(dy, dev), 2, 3))
    wdx, wdw, wdb = f64.conv2d_backward(x, w, dy, 2, 3)
    npix = 32 * y.shape[2] * y.shape[3]
    assert_close(dx, wdx, 64 * 49, amax(dy), amax(w), "stem dX every element")
    assert_close(dw, wdw, npix, amax(dy), amax(x), "stem dW every element")
    assert_close(db, wdb, npix, amax(dy), 1.0, "stem db")
