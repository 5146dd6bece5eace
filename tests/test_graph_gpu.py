"""HIP-graph capture of the GEMM entry points (graph-capture integration of the
reference's GraphExecutor, include/GraphExecutor.hpp:142-203).

Every entry point only enqueues kernels on the given stream (no host sync, no
allocation, no hipMemsetAsync), so a captured sequence replays the same
kernels.  Each replay is checked bit-for-bit against the eager result on the
same inputs, with eager work (new inputs written in place) between replays.
"""
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
