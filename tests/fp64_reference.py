"""Float64 references of the convolution for whole-tensor checks at the
benchmark sizes (test infrastructure).

The CPU oracle restates the reference's loops one output at a time and takes
minutes on a whole 32 x 256 x 14 x 14 layer; these compute the same sums in
float64 through numpy's BLAS (a column matrix of the input windows, then one
product), in about a second.  They are exact sums up to float64 rounding, so
they stand in for the oracle where the parity bound (1e-5 * sqrt(K) * max|a| *
max|b|, fp32 against exact) is the test; test_oracle.py pins each against the
oracle's conv2d_cpu / conv2d_backward_*_cpu restatements
(include/TensorOps.hpp:235-273, src/gpu_ops.cpp conv backward) on small
shapes of every stride and padding kind.
"""
from __future__ import annotations

from typing import Optional

import numpy as np


def _windows(x: np.ndarray, kh: int, kw: int, stride: int, pad: int) -> np.ndarray:
    """[n*ho*wo, c*kh*kw] float64 columns: row (img, oh, ow), column (c, r, s)."""
    n, c = x.shape[:2]
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    win = np.lib.stride_tricks.sliding_window_view(xp, (kh, kw), axis=(2, 3))
    win = win[:, :, ::stride, ::stride]          # [n, c, ho, wo, kh, kw]
    ho, wo = win.shape[2], win.shape[3]
    return win.transpose(0, 2, 3, 1, 4, 5).reshape(n * ho * wo, c * kh * kw), ho, wo


def conv2d(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray], stride: int,
           pad: int) -> np.ndarray:
    """out[img][co][oh][ow] = b[co] + sum_{c,r,s} x_pad[img][c][oh*s+r][ow*s+s'] * w[co][c][r][s']."""
    n = x.shape[0]
    co, _, kh, kw = w.shape
    cols, ho, wo = _windows(x, kh, kw, stride, pad)
    out = cols @ w.astype(np.float64).reshape(co, -1).T           # [n*ho*wo, co]
    out = out.reshape(n, ho, wo, co).transpose(0, 3, 1, 2)
    if b is not None:
        out = out + b.astype(np.float64)[None, :, None, None]
    return out


def conv2d_backward(x: np.ndarray, w: np.ndarray, dy: np.ndarray, stride: int, pad: int):
    """(dX, dW, db) of conv2d for the output gradient dy, in float64."""
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    cols, ho, wo = _windows(x, kh, kw, stride, pad)
    assert dy.shape == (n, co, ho, wo), (dy.shape, (n, co, ho, wo))
    dyr = dy.astype(np.float64).transpose(0, 2, 3, 1).reshape(-1, co)   # [n*ho*wo, co]
    dw = (dyr.T @ cols).reshape(w.shape)
    db = dyr.sum(axis=0)
    dcols = (dyr @ w.astype(np.float64).reshape(co, -1)).reshape(n, ho, wo, c, kh, kw)
    dxp = np.zeros((n, c, h + 2 * pad, wd + 2 * pad), np.float64)
    for r in range(kh):
        for s in range(kw):
            dxp[:, :, r:r + stride * (ho - 1) + 1:stride, s:s + stride * (wo - 1) + 1:stride] += \
                dcols[:, :, :, :, r, s].transpose(0, 3, 1, 2)
    return dxp[:, :, pad:pad + h, pad:pad + wd], dw, db
