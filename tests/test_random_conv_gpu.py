"""Randomised Conv2D forward and backward through the cost model's own plans.

The conv tests in test_linear_conv_gpu.py pin chosen geometries and paths.
Here 40 seeded draws mix what a caller can hand over at once: batch 1-4,
channel counts that are multiples of 16 (implicit forward GEMM), of 4
(implicit weight gradient) or neither (im2col + GEMM), square and non-square
kernels from 1x1 to 5x5, strides 1-3, padding 0-2 (so dX goes through the
flipped-weight forward convolution or through col2im), inputs that are dense
or NCHW views (a channel slice, channels-last storage, every second image),
a bias or none, and dW accumulated into an existing gradient or not.

Each result must meet the GEMM parity bound 1e-5*sqrt(K)*max|A|*max|B|
against the reference's conv2d_cpu / conv2d_backward_{input,weight,bias}_cpu
restated in oracle/oracle.c (include/TensorOps.hpp:235-415), with K the
reduction length of that output.  A second forward call on the same inputs
must return the same bits (split-K partials are summed in a fixed order).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

N_CASES = 40


def _channels(rng) -> int:
    r = rng.random()
    if r < 0.35:
        return 16 * int(rng.integers(1, 5))
    if r < 0.65:
        return 4 * int(rng.integers(1, 11))
    return int(rng.integers(1, 21))


def _case(rng, i: int) -> dict:
    while True:
        kh = int(rng.integers(1, 6))
        kw = kh if rng.random() < 0.4 else int(rng.integers(1, 6))
        d = dict(n=int(rng.integers(1, 5)), c=_channels(rng), co=_channels(rng),
                 h=int(rng.integers(1, 25)), w=int(rng.integers(1, 25)), kh=kh, kw=kw,
                 stride=int(rng.integers(1, 4)), pad=int(rng.integers(0, 3)))
        if i % 4 == 0:
            # the geometry whose dX is the forward convolution of dY with the
            # flipped weights: stride 1, square kernel, pad <= k-1, c_out % 16 == 0
            d.update(kw=kh, stride=1, pad=min(d["pad"], kh - 1), co=16 * int(rng.integers(1, 4)))
        if (oracle.conv_out(d["h"], d["pad"], d["kh"], d["stride"]) > 0
                and oracle.conv_out(d["w"], d["pad"], d["kw"], d["stride"]) > 0):
            break
    d.update(view=str(rng.choice(["dense", "dense", "channel_slice", "nhwc", "batch_step"])),
             bias=bool(rng.random() < 0.6), beta_w=float(rng.choice([0.0, 0.0, 1.0, 0.5])),
             seed=5000 + 10 * i)
    return d


_rng = np.random.default_rng(20261202)
CASES = [_case(_rng, i) for i in range(N_CASES)]


def _input_view(x: np.ndarray, view: str, seed: int, dev) -> torch.Tensor:
    """x (dense NCHW) on the GPU as the NCHW view `view`."""
    n, c, h, w = x.shape
    if view == "channel_slice":
        big = np.zeros((n, c + 3, h, w), np.float32)
        big[:, 1:1 + c] = x
        return torch.from_numpy(big).to(dev)[:, 1:1 + c]
    if view == "nhwc":
        return torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 3, 1))).to(dev).permute(0, 3, 1, 2)
    if view == "batch_step":
        big = np.zeros((2 * n, c, h, w), np.float32)
        big[::2] = x
        return torch.from_numpy(big).to(dev)[::2]
    return torch.from_numpy(x).to(dev)


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(N_CASES)])
def test_random_conv_auto_plan(dev, case):
    n, c, h, wd, co = case["n"], case["c"], case["h"], case["w"], case["co"]
    kh, kw, stride, pad, seed = case["kh"], case["kw"], case["stride"], case["pad"], case["seed"]
    ho, wo = oracle.conv_out(h, pad, kh, stride), oracle.conv_out(wd, pad, kw, stride)
    x = oracle.normal((n, c, h, wd), seed)
    w = oracle.normal((co, c, kh, kw), seed + 1)
    b = oracle.normal((co,), seed + 2) if case["bias"] else None
    dy = oracle.normal((n, co, ho, wo), seed + 3)
    X = _input_view(x, case["view"], seed, dev)
    W = torch.from_numpy(w).to(dev)
    Bt = torch.from_numpy(b).to(dev) if b is not None else None

    y = mt.conv2d(X, W, Bt, stride, pad)
    cfg = mt.last_config()
    y2 = mt.conv2d(X, W, Bt, stride, pad)
    torch.cuda.synchronize()
    print(f"[case] {case} -> forward {cfg}", flush=True)
    y, y2 = y.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "forward not deterministic"
    extra = 2e-6 * (1.0 + amax(b)) if b is not None else 0.0
    assert_close(y, oracle.conv2d(x, w, b, stride, pad), c * kh * kw, amax(x), amax(w),
                 f"random conv fwd {case}", extra=extra)

    beta_w = case["beta_w"]
    dw_prev = oracle.uniform((co, c, kh, kw), seed + 4)
    dw_in = torch.from_numpy(dw_prev).to(dev) if beta_w != 0.0 else None
    dX, dW, db = mt.conv2d_backward(torch.from_numpy(x).to(dev), W, torch.from_numpy(dy).to(dev),
                                    stride, pad, dw=dw_in, beta_w=beta_w)
    torch.cuda.synchronize()
    dX, dW, db = dX.cpu().numpy(), dW.cpu().numpy(), db.cpu().numpy()
    wdx, wdw, wdb = oracle.conv2d_backward(x, w, dy, stride, pad)
    if beta_w != 0.0:
        wdw = wdw.astype(np.float64) + beta_w * dw_prev
    assert_close(dX, wdx, co * kh * kw, amax(dy), amax(w), f"random conv dX {case}")
    assert_close(dW, wdw, n * ho * wo, amax(dy), amax(x), f"random conv dW {case}",
                 extra=2e-6 * (1.0 + beta_w) if beta_w != 0.0 else 0.0)
    assert_close(db, wdb, n * ho * wo, amax(dy), 1.0, f"random conv db {case}")


# The halo-patch kernel under forced tile configurations and split factors
# (a forced configuration takes it wherever its patches fit): NCHW-view
# geometries with c_in not a multiple of 16 (the channels-last kernel takes
# those) and c_in*kh*kw % 4 == 0, at least two taps, strides 1-3, padding
# 0-2, dense or channel-slice inputs, and the dX of the stride-1 square
# cases through the same kernel.
def _halo_case(rng, i: int) -> dict:
    while True:
        kh = int(rng.integers(1, 6))
        kw = kh if rng.random() < 0.5 else int(rng.integers(1, 6))
        c = int(rng.integers(1, 41))
        if c % 16 == 0 or (c * kh * kw) % 4 or kh * kw < 2:
            continue
        d = dict(n=int(rng.integers(1, 5)), c=c, co=int(rng.integers(1, 49)),
                 h=int(rng.integers(2, 20)), w=int(rng.integers(2, 30)), kh=kh, kw=kw,
                 stride=int(rng.integers(1, 4)), pad=int(rng.integers(0, 3)),
                 cfg=int(rng.integers(0, 4)), split=int(rng.choice([1, 2, 3, 5])),
                 view=str(rng.choice(["dense", "channel_slice"])), seed=7000 + 10 * i)
        if (oracle.conv_out(d["h"], d["pad"], kh, d["stride"]) > 0
                and oracle.conv_out(d["w"], d["pad"], kw, d["stride"]) > 0):
            return d


N_HALO = 30
_hrng = np.random.default_rng(20261203)
HALO_CASES = [_halo_case(_hrng, i) for i in range(N_HALO)]


@pytest.mark.parametrize("case", HALO_CASES, ids=[f"h{i}" for i in range(N_HALO)])
def test_random_conv_halo_forced(dev, case):
    n, c, h, wd, co = case["n"], case["c"], case["h"], case["w"], case["co"]
    kh, kw, stride, pad, seed = case["kh"], case["kw"], case["stride"], case["pad"], case["seed"]
    x = oracle.normal((n, c, h, wd), seed)
    w = oracle.normal((co, c, kh, kw), seed + 1)
    b = oracle.normal((co,), seed + 2)
    X = _input_view(x, case["view"], seed, dev)
    W, Bt = torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev)
    with mt.forced_config(mt.FAMILY_DL, case["cfg"], case["split"]):
        y = mt.conv2d(X, W, Bt, stride, pad)
        cfg = mt.last_config()
        y2 = mt.conv2d(X, W, Bt, stride, pad)
    torch.cuda.synchronize()
    print(f"[case] {case} -> forward {cfg}", flush=True)
    y, y2 = y.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "forward not deterministic"
    assert_close(y, oracle.conv2d(x, w, b, stride, pad), c * kh * kw, amax(x), amax(w),
                 f"forced halo conv {case}", extra=2e-6 * (1.0 + amax(b)))
    if stride == 1 and kh == kw and pad <= kh - 1 and (co * kh * kw) % 4 == 0 and co % 16:
        ho, wo = oracle.conv_out(h, pad, kh, 1), oracle.conv_out(wd, pad, kw, 1)
        dy = oracle.normal((n, co, ho, wo), seed + 3)
        with mt.forced_config(mt.FAMILY_DL, case["cfg"], case["split"]):
            dX, _, _ = mt.conv2d_backward(torch.from_numpy(x).to(dev), W,
                                          torch.from_numpy(dy).to(dev), 1, pad,
                                          need_dw=False, need_db=False)
            print(f"[case] dX {mt.last_config()}", flush=True)
        wdx, _, _ = oracle.conv2d_backward(x, w, dy, 1, pad)
        assert_close(dX.cpu().numpy(), wdx, co * kh * kw, amax(dy), amax(w),
                     f"forced halo dX {case}")


def test_random_conv_halo_forced_coverage(dev):
    """Most of the forced draws above run the halo kernel (the rest have bands
    too large for their tile): each case's forward is run here again, under
    its forced configuration, so the check holds whatever subset of the
    parametrized tests ran in this process."""
    seen = []
    for case in HALO_CASES:
        x = oracle.normal((case["n"], case["c"], case["h"], case["w"]), case["seed"])
        w = oracle.normal((case["co"], case["c"], case["kh"], case["kw"]), case["seed"] + 1)
        X = _input_view(x, case["view"], case["seed"], dev)
        with mt.forced_config(mt.FAMILY_DL, case["cfg"], case["split"]):
            mt.conv2d(X, torch.from_numpy(w).to(dev), None, case["stride"], case["pad"])
            seen.append("b=im2col_halo" in mt.last_config())
    torch.cuda.synchronize()
    assert sum(seen) >= N_HALO // 2, seen
