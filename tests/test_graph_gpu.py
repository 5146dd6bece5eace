"""HIP-graph capture of the GEMM entry points (graph-capture integration of the
reference's GraphExecutor, include/GraphExecutor.hpp:142-203).

Every entry point only enqueues kernels on the given stream (no host sync, no
allocation, no hipMemsetAsync), so a captured sequence replays the same
kernels.  Each replay is checked bit-for-bit against the eager result on the
same inputs, with eager work (new inputs written in place) between replays.
"""
import ctypes

import numpy as np
import pytest
import torch

import minitensor_amd as mt

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_graph_linear_fwd_bwd_replays(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    X = torch.randn(256, 2048, device=dev, generator=gen)
    W = torch.randn(1000, 2048, device=dev, generator=gen) * (2.0 / 2048) ** 0.5
    b = torch.randn(1000, device=dev, generator=gen)
    dY = torch.randn(256, 1000, device=dev, generator=gen) * 0.01
    Y = torch.empty(256, 1000, device=dev)
    dX = torch.empty(256, 2048, device=dev)
    dW = torch.empty(1000, 2048, device=dev)
    db = torch.empty(1000, device=dev)
    ws = mt.workspace(mt.lib().mt_linear_workspace_f32(256, 2048, 1000), dev)

    def step():
        mt.linear(X, W, b, out=Y, ws=ws)
        mt.linear_backward(dY, X, W, dx=dX, dw=dW, db=db, ws=ws)

    g = _capture(step)
    for rep in range(4):
        # eager work between replays: new inputs, in place
        X.copy_(torch.randn(256, 2048, device=dev, generator=gen))
        dY.copy_(torch.randn(256, 1000, device=dev, generator=gen) * 0.01)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (Y, dX, dW, db)]
        step()                                   # eager on the same inputs
        torch.cuda.synchronize()
        for name, a, e in zip(("Y", "dX", "dW", "db"), got, (Y, dX, dW, db)):
            assert torch.equal(a, e), f"replay {rep}: {name} differs from eager"
        print(f"[graph] replay {rep} == eager", flush=True)


def test_graph_split_k_and_batched_replays(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    A = torch.rand(64, 8192, device=dev, generator=gen)
    B = torch.rand(8192, 64, device=dev, generator=gen)
    C = torch.empty(64, 64, device=dev)
    ws = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)), dev)
    Ab = torch.rand(8, 96, 40, device=dev, generator=gen)
    Bb = torch.rand(8, 40, 72, device=dev, generator=gen)
    Cb = torch.empty(8, 96, 72, device=dev)

    def step():
        mt.gemm(A, B, out=C, ws=ws)
        mt.gemm(Ab, Bb, out=Cb)

    mt.gemm(A, B, out=C, ws=ws)
    torch.cuda.synchronize()
    assert "split=1 " not in mt.last_config() + " "     # the split-K pair is captured
    g = _capture(step)
    for rep in range(3):
        A.mul_(0.5).add_(0.25)
        Bb.add_(1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        c1, c2 = C.clone(), Cb.clone()
        step()
        torch.cuda.synchronize()
        assert torch.equal(c1, C) and torch.equal(c2, Cb), f"replay {rep} differs"
        ref = (A.double() @ B.double()).float()
        assert torch.allclose(C, ref, rtol=1e-4, atol=1e-3)


def test_graph_conv_replays(dev):
    """Conv2D forward and backward captured: the channels-last path (the fused
    layout launch, split-K GEMM and reduction), the halo-patch kernel over an
    NCHW input (its offset table is a kernel argument, its LDS dynamic), and
    dX, dW + db (dY read in NCHW, db summed by the dW reduction)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    x = torch.randn(8, 32, 14, 14, device=dev, generator=gen)
    w = torch.randn(64, 32, 3, 3, device=dev, generator=gen) * 0.1
    b = torch.randn(64, device=dev, generator=gen)
    dy = torch.randn(8, 64, 14, 14, device=dev, generator=gen) * 0.01
    xh = torch.randn(32, 24, 28, 28, device=dev, generator=gen)
    wh = torch.randn(128, 24, 3, 3, device=dev, generator=gen) * 0.1
    d = mt.Conv2dDesc(8, 32, 14, 14, 64, 3, 3, 1, 1)
    dh = mt.Conv2dDesc(32, 24, 28, 28, 128, 3, 3, 1, 1)
    ws = mt.workspace(max(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(d)),
                          mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d))), dev)
    wsh = mt.workspace(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(dh)), dev)
    y = torch.empty(8, 64, 14, 14, device=dev)
    yh = torch.empty(32, 128, 28, 28, device=dev)
    dx = torch.empty_like(x)
    dw = torch.empty_like(w)
    db = torch.empty_like(b)
    outs = (y, yh, dx, dw, db)

    def step():
        y.copy_(mt.conv2d(x, w, b, 1, 1, ws=ws))
        yh.copy_(mt.conv2d(xh, wh, None, 1, 1, ws=wsh))
        gx, gw, gb = mt.conv2d_backward(x, w, dy, 1, 1, ws=ws)
        dx.copy_(gx); dw.copy_(gw); db.copy_(gb)

    mt.conv2d(xh, wh, None, 1, 1, ws=wsh)
    torch.cuda.synchronize()
    print(f"[config] halo layer: {mt.last_config()}", flush=True)
    g = _capture(step)
    for rep in range(3):
        x.mul_(0.5).add_(0.1)
        xh.add_(0.25)
        dy.mul_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        step()
        torch.cuda.synchronize()
        for name, a, e in zip(("y", "yh", "dx", "dw", "db"), got, outs):
            assert torch.equal(a, e), f"replay {rep}: {name} differs from eager"
        print(f"[graph] conv replay {rep} == eager", flush=True)


def test_graph_skinny_and_phased_dx_replays(dev):
    """The vector-ALU kernels (a split GEMV with its reduction launch, a
    transposed GEMV, a rank-k product), a strided convolution's dX by stride
    phase (dY copy, phase weights, one GEMM per phase into compact outputs,
    the interleave) and a strided 1x1 layer's dX (the per-image product, the
    interleave) captured together; every replay equals the eager calls bit
    for bit."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(8)
    a = torch.rand(1, 4096, device=dev, generator=gen)
    B = torch.rand(4096, 2048, device=dev, generator=gen)
    c = torch.empty(1, 2048, device=dev)
    ws_g = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(a), mt.mat(B), mt.mat(c)), dev)
    At = torch.rand(1000, 512, device=dev, generator=gen)
    v = torch.rand(512, 3, device=dev, generator=gen)
    cv = torch.empty(1000, 3, device=dev)
    ws_t = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(At), mt.mat(v), mt.mat(cv)), dev)
    u = torch.rand(2048, 2, device=dev, generator=gen)
    w2 = torch.rand(2, 2048, device=dev, generator=gen)
    r = torch.empty(2048, 2048, device=dev)
    x = torch.randn(4, 32, 26, 26, device=dev, generator=gen)
    wc = torch.randn(64, 32, 1, 1, device=dev, generator=gen) * 0.1
    dy = torch.randn(4, 64, 13, 13, device=dev, generator=gen)
    d = mt.Conv2dDesc(4, 32, 26, 26, 64, 1, 1, 2, 0)
    dx = torch.empty_like(x)
    # 28x28 -> 14x14 (196 positions, a multiple of 4): the per-image product
    dy2 = torch.randn(4, 64, 14, 14, device=dev, generator=gen)
    d2 = mt.Conv2dDesc(4, 32, 28, 28, 64, 1, 1, 2, 0)
    dx2 = torch.empty(4, 32, 28, 28, device=dev)
    ws_c2 = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d2)), dev)

    with mt.forced_config(mt.FAMILY_DL, 1, 1):   # the phased dX on this small layer
        ws_c = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
    cfgs = []

    def step():
        mt.gemm(a, B, out=c, ws=ws_g)
        cfgs.append(mt.last_config())
        mt.gemm(At, v, out=cv, ws=ws_t)
        cfgs.append(mt.last_config())
        mt.gemm(u, w2, out=r)
        cfgs.append(mt.last_config())
        with mt.forced_config(mt.FAMILY_DL, 1, 1):
            rc = mt.lib().mt_conv2d_bwd_input_f32(
                ctypes.byref(d), dy.data_ptr(), wc.data_ptr(), dx.data_ptr(), ws_c.data_ptr(),
                ws_c.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            cfgs.append(mt.last_config())
        assert rc == mt.MT_OK
        rc = mt.lib().mt_conv2d_bwd_input_f32(
            ctypes.byref(d2), dy2.data_ptr(), wc.data_ptr(), dx2.data_ptr(),
            mt._ptr(ws_c2), 0 if ws_c2 is None else ws_c2.numel(),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        cfgs.append(mt.last_config())
        assert rc == mt.MT_OK

    step()
    torch.cuda.synchronize()
    print(f"[graph] {cfgs}", flush=True)
    assert cfgs[0].startswith("sk gemv_mv ") and "split=1 " not in cfgs[0] + " ", cfgs
    assert cfgs[1].startswith("sk gemv_kv_t ") and cfgs[2].startswith("sk rankk "), cfgs
    assert "b=im2col " in cfgs[3] + " ", cfgs
    assert "a=mv b=mv" in cfgs[4] and "im2col" not in cfgs[4], cfgs
    g = _capture(step)
    for rep in range(3):
        a.copy_(torch.rand(1, 4096, device=dev, generator=gen))
        dy.copy_(torch.randn(4, 64, 13, 13, device=dev, generator=gen))
        dy2.copy_(torch.randn(4, 64, 14, 14, device=dev, generator=gen))
        dx.fill_(7.0)
        dx2.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (c, cv, r, dx, dx2)]
        dx.fill_(-7.0)
        dx2.fill_(-7.0)
        step()
        torch.cuda.synchronize()
        for name, x1, e in zip(("gemv", "gemv_t", "rank-k", "dX", "dX 1x1 s2"), got,
                               (c, cv, r, dx, dx2)):
            assert torch.equal(x1, e), f"replay {rep}: {name} differs from eager"
        print(f"[graph] skinny + phased dX replay {rep} == eager", flush=True)
