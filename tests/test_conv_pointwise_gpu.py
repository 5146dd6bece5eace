"""1x1 convolutions (stride 1, no padding, c_in and positions per image
multiples of 4) as one product per image over the NCHW tensors:
Y_b = W·X_b, dX_b = Wᵀ·dY_b, and dW = Σ_b dY_b·X_bᵀ written as per-image
partials (GemmParams::part) that the split-K reduction sums together with
beta·dW and the bias gradient.

Cases: bias, ragged channel counts, one image, input views whose (h, w) fold
into one position index (NHWC storage, a channel slice) and one that does not
(a spatial crop, which takes the NCHW-view kernel), every kernel family and
split forced on the batch-summed dW (each family's partial-store path),
unaligned operands (the register-staged kernels), gradient accumulation,
exactly the queried workspace, determinism and graph replay.  Oracle: the
reference's conv2d_cpu and conv2d_backward_{input,weight,bias}_cpu restated
in oracle/oracle.c (include/TensorOps.hpp:235-273, 276-345); bound
1e-5*sqrt(K)*max|a|*max|b| (tests/util_parity.py).
"""
import ctypes

import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

# n, c_in, h, w, c_out
SHAPES = [
    (4, 16, 8, 8, 24),
    (3, 64, 14, 14, 32),
    (1, 36, 6, 10, 20),     # one image, 60 positions
    (2, 12, 4, 4, 100),     # 16 positions: one K chunk
]


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def sync_np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _desc(n, c, h, w, co):
    return mt.Conv2dDesc(n, c, h, w, co, 1, 1, 1, 0)


@pytest.mark.parametrize("shape", SHAPES)
def test_pointwise_forward(dev, shape):
    n, c, h, w, co = shape
    x = oracle.normal((n, c, h, w), 1)
    wt = oracle.normal((co, c, 1, 1), 2)
    b = oracle.normal((co,), 3)
    y = mt.conv2d(g(x, dev), g(wt, dev), g(b, dev), 1, 0)
    cfg = mt.last_config()
    print(f"[config] {cfg}", flush=True)
    assert "im2col" not in cfg, cfg
    assert_close(sync_np(y), oracle.conv2d(x, wt, b, 1, 0), c, amax(x), amax(wt), "1x1 forward")


def test_pointwise_forward_views(dev):
    """NHWC storage and a channel slice fold (h, w) into one index and are read
    in place by the batched product; a spatial crop does not and takes the
    NCHW-view kernel.  All three against the oracle on the dense copy."""
    n, c, h, w, co = 2, 32, 12, 12, 40
    wt = oracle.normal((co, c, 1, 1), 5)
    W = g(wt, dev)
    nhwc = g(oracle.normal((n, h, w, c), 6), dev)
    wide = g(oracle.normal((n, c + 8, h, w), 7), dev)
    big = g(oracle.normal((n, c, h + 4, w + 4), 8), dev)
    cases = [("nhwc", nhwc.permute(0, 3, 1, 2), False),
             ("channel slice", wide[:, 4:4 + c], False),
             ("spatial crop", big[:, :, 2:2 + h, 2:2 + w], True)]
    for name, xv, crop in cases:
        y = mt.conv2d(xv, W, None, 1, 0)
        cfg = mt.last_config()
        print(f"[config] {name}: {cfg}", flush=True)
        assert ("im2col" in cfg) == crop, (name, cfg)
        xd = sync_np(xv.contiguous())
        assert_close(sync_np(y), oracle.conv2d(xd, wt, None, 1, 0), c, amax(xd), amax(wt), name)


@pytest.mark.parametrize("shape", SHAPES)
def test_pointwise_backward(dev, shape):
    """dX, and dW + db accumulated into existing gradients (beta_w = 0.5,
    beta_b = 2) in one call, bit-identical on a repeat."""
    n, c, h, w, co = shape
    x = oracle.normal((n, c, h, w), 11)
    wt = oracle.normal((co, c, 1, 1), 12)
    dy = oracle.normal((n, co, h, w), 13)
    dw0 = oracle.normal((co, c, 1, 1), 14)
    db0 = oracle.normal((co,), 15)
    X, Wt, dY = g(x, dev), g(wt, dev), g(dy, dev)
    dX, _, _ = mt.conv2d_backward(X, Wt, dY, 1, 0, need_dw=False, need_db=False)
    print(f"[config] dX {mt.last_config()}", flush=True)
    assert "im2col" not in mt.last_config()
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, 1, 0)
    assert_close(sync_np(dX), wdx, co, amax(dy), amax(wt), "1x1 dX")
    d = _desc(n, c, h, w, co)
    ws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
    outs = []
    for _ in range(2):
        dW, dB = g(dw0, dev), g(db0, dev)
        rc = mt.lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                                    dW.data_ptr(), 0.5, dB.data_ptr(), 2.0,
                                                    ws.data_ptr(), ws.numel(), None)
        assert rc == 0, mt.lib().mt_strerror(rc).decode()
        outs.append((sync_np(dW), sync_np(dB)))
    cfg = mt.last_config()
    print(f"[config] dW {cfg}", flush=True)
    assert "batch-summed" in cfg, cfg
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    K = n * h * w
    assert_close(outs[0][0], 0.5 * dw0.astype(np.float64) + wdw, K, amax(dy), amax(x),
                 "1x1 dW + 0.5 dW0", extra=1e-5)
    assert_close(outs[0][1], 2.0 * db0.astype(np.float64) + wdb, K, amax(dy), 1.0,
                 "1x1 db + 2 db0", extra=1e-5)


def _forced_cases():
    out = []
    for fam, name in ((mt.FAMILY_DL, "dl"), (mt.FAMILY_RS, "rs"), (mt.FAMILY_KSW, "ksw")):
        for cfg in range(mt.config_count(fam)):
            if fam == mt.FAMILY_DL and cfg >= 7:     # the implicit-im2col convolution tile
                continue
            for splits in (1, 3):
                out.append((fam, name, cfg, splits))
    return out


@pytest.mark.parametrize("fam,name,cfg,splits", _forced_cases())
def test_pointwise_dw_every_family(dev, fam, name, cfg, splits):
    """The batch-summed dW through every tile configuration at one and three
    splits: each family's epilogue writes per-image partials, and the
    reduction sums splits x images of them.  db: the direct-to-LDS kernels
    fuse it as row sums of dY per (split, image) that the reduction sums
    ("rows"); the other families leave it to the reduction's pass over dY."""
    n, c, h, w, co = 3, 24, 12, 12, 40
    x = oracle.normal((n, c, h, w), 21)
    wt = oracle.normal((co, c, 1, 1), 22)
    dy = oracle.normal((n, co, h, w), 23)
    X, dY = g(x, dev), g(dy, dev)
    d = _desc(n, c, h, w, co)
    with mt.forced_config(fam, cfg, splits):
        ws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
        dW = torch.empty(co, c, 1, 1, device=dev)
        dB = torch.empty(co, device=dev)
        rc = mt.lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                                    dW.data_ptr(), 0.0, dB.data_ptr(), 0.0,
                                                    ws.data_ptr(), ws.numel(), None)
        assert rc == 0, mt.lib().mt_strerror(rc).decode()
        cfg_s = mt.last_config()
    print(f"[config] {cfg_s}", flush=True)
    assert cfg_s.startswith(name) and "batch-summed" in cfg_s, cfg_s
    assert cfg_s.endswith(" rows") == (fam == mt.FAMILY_DL), cfg_s
    _, wdw, wdb = oracle.conv2d_backward(x, wt, dy, 1, 0)
    K = n * h * w
    assert_close(sync_np(dW), wdw, K, amax(dy), amax(x), f"dW {cfg_s}")
    assert_close(sync_np(dB), wdb, K, amax(dy), 1.0, f"db {cfg_s}")


def test_pointwise_unaligned_operands(dev):
    """x, dY and the outputs one float off 16-byte alignment: the products
    take the register-staged kernels (scalar gathers), results unchanged."""
    n, c, h, w, co = 2, 16, 6, 6, 12
    x = oracle.normal((n, c, h, w), 31)
    wt = oracle.normal((co, c, 1, 1), 32)
    dy = oracle.normal((n, co, h, w), 33)
    d = _desc(n, c, h, w, co)

    def off(a):
        buf = torch.zeros(a.size + 1, device=dev)
        buf[1:] = g(a.reshape(-1), dev)
        return buf[1:]

    X, Wt, dY = off(x), off(wt), off(dy)
    ws = mt.workspace(max(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(d)),
                          mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d))), dev)
    Y, dX, dW, dB = (off(np.zeros(s, np.float32)) for s in
                     ((n, co, h, w), (n, c, h, w), (co, c, 1, 1), (co,)))
    lib = mt.lib()
    assert lib.mt_conv2d_fwd_f32(ctypes.byref(d), X.data_ptr(), Wt.data_ptr(), None, Y.data_ptr(),
                                 ws.data_ptr(), ws.numel(), None) == 0
    print(f"[config] fwd {mt.last_config()}", flush=True)
    assert lib.mt_conv2d_bwd_input_f32(ctypes.byref(d), dY.data_ptr(), Wt.data_ptr(),
                                       dX.data_ptr(), ws.data_ptr(), ws.numel(), None) == 0
    assert lib.mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                             dW.data_ptr(), 0.0, dB.data_ptr(), 0.0,
                                             ws.data_ptr(), ws.numel(), None) == 0
    print(f"[config] dW {mt.last_config()}", flush=True)
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, 1, 0)
    K = n * h * w
    assert_close(sync_np(Y).reshape(n, co, h, w), oracle.conv2d(x, wt, None, 1, 0), c, amax(x),
                 amax(wt), "fwd")
    assert_close(sync_np(dX).reshape(n, c, h, w), wdx, co, amax(dy), amax(wt), "dX")
    assert_close(sync_np(dW).reshape(co, c, 1, 1), wdw, K, amax(dy), amax(x), "dW")
    assert_close(sync_np(dB), wdb, K, amax(dy), 1.0, "db")


def test_pointwise_workspace_is_exact_and_graph_replays(dev):
    """The ResNet 56x56 256->64 1x1 layer at batch 8: forward, dX and dW + db
    run in exactly the queried workspaces, and a captured graph of the three
    replays bit-identically to the eager calls."""
    n, c, h, w, co = 8, 256, 56, 56, 64
    x = oracle.normal((n, c, h, w), 41)
    wt = oracle.normal((co, c, 1, 1), 42, std=0.06)
    dy = oracle.normal((n, co, h, w), 43)
    X, Wt, dY = g(x, dev), g(wt, dev), g(dy, dev)
    d = _desc(n, c, h, w, co)
    lib = mt.lib()
    fws = mt.workspace(lib.mt_conv2d_workspace_f32(ctypes.byref(d)), dev)
    bws = mt.workspace(lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
    Y = torch.empty(n, co, h, w, device=dev)
    dX = torch.empty(n, c, h, w, device=dev)
    dW = torch.empty(co, c, 1, 1, device=dev)
    dB = torch.empty(co, device=dev)

    def step():
        for rc in (lib.mt_conv2d_fwd_f32(ctypes.byref(d), X.data_ptr(), Wt.data_ptr(), None,
                                         Y.data_ptr(), mt._ptr(fws), fws.numel() if fws is not None
                                         else 0, mt._stream(None)),
                   lib.mt_conv2d_bwd_input_f32(ctypes.byref(d), dY.data_ptr(), Wt.data_ptr(),
                                               dX.data_ptr(), mt._ptr(bws), 0 if bws is None else bws.numel(),
                                               mt._stream(None)),
                   lib.mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(),
                                                     dY.data_ptr(), dW.data_ptr(), 0.0,
                                                     dB.data_ptr(), 0.0, mt._ptr(bws),
                                                     0 if bws is None else bws.numel(),
                                                     mt._stream(None))):
            assert rc == 0, mt.lib().mt_strerror(rc).decode()

    step()
    eager = [sync_np(t).copy() for t in (Y, dX, dW, dB)]
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, 1, 0)
    K = n * h * w
    assert_close(eager[0], oracle.conv2d(x, wt, None, 1, 0), c, amax(x), amax(wt), "fwd")
    assert_close(eager[1], wdx, co, amax(dy), amax(wt), "dX")
    assert_close(eager[2], wdw, K, amax(dy), amax(x), "dW")
    assert_close(eager[3], wdb, K, amax(dy), 1.0, "db")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        for t in (Y, dX, dW, dB):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        for got, want in zip((Y, dX, dW, dB), eager):
            assert np.array_equal(sync_np(got), want)


@pytest.mark.parametrize("n,c,h,w,co,stride", [
    (2, 16, 8, 8, 24, 2),      # 4x4 output
    (3, 32, 11, 7, 20, 3),     # ragged: 4x3 output, rows and columns past the last phase
    (1, 12, 13, 13, 40, 4),    # 4x4 output, 13 = 3*4 + 1
    (4, 64, 28, 28, 128, 2),   # a ResNet downsampling shortcut, batch 4
])
def test_pointwise_strided_dx(dev, n, c, h, w, co, stride):
    """dX of a strided 1x1 layer without padding: the product Wᵀ·dY_b per
    image into the phase-(0, 0) buffer, then the interleave writes dX with
    zeros on every pixel no tap reaches; dW + db: x's output positions copied
    out, then the batch-summed 1x1 product.  Against the oracle, bit-identical
    on a repeat."""
    x = oracle.normal((n, c, h, w), 51)
    wt = oracle.normal((co, c, 1, 1), 52)
    ho, wo = oracle.conv_out(h, 0, 1, stride), oracle.conv_out(w, 0, 1, stride)
    dy = oracle.normal((n, co, ho, wo), 53)
    X, Wt, dY = g(x, dev), g(wt, dev), g(dy, dev)
    outs = []
    for _ in range(2):
        dX, _, _ = mt.conv2d_backward(X, Wt, dY, stride, 0, need_dw=False, need_db=False)
        outs.append(sync_np(dX))
    cfg = mt.last_config()
    print(f"[config] {cfg}", flush=True)
    assert "im2col" not in cfg and "a=mv b=mv" in cfg, cfg
    assert np.array_equal(outs[0], outs[1])
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, stride, 0)
    assert_close(outs[0], wdx, co, amax(dy), amax(wt), f"1x1 stride {stride} dX")
    _, dW, dB = mt.conv2d_backward(X, Wt, dY, stride, 0, need_dx=False)
    cfg = mt.last_config()
    print(f"[config] dW {cfg}", flush=True)
    assert "batch-summed" in cfg, cfg
    K = n * ho * wo
    assert_close(sync_np(dW), wdw, K, amax(dy), amax(x), f"1x1 stride {stride} dW")
    assert_close(sync_np(dB), wdb, K, amax(dy), 1.0, f"1x1 stride {stride} db")


def _random_cases(seed=20261202, count=24):
    """Seeded 1x1 layers that take the per-image paths: c_in a multiple of 4,
    positions per image (of the output) a multiple of 4, stride 1-4."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        s = int(rng.choice([1, 1, 2, 3, 4]))
        n = int(rng.integers(1, 5))
        c = 4 * int(rng.integers(1, 33))
        co = int(rng.integers(1, 97))
        h, w = int(rng.integers(1, 30)), int(rng.integers(1, 30))
        ho, wo = (h - 1) // s + 1, (w - 1) // s + 1
        if (ho * wo) % 4:
            continue
        out.append((n, c, h, w, co, s, float(rng.choice([0.0, 1.0, 0.5]))))
    return out


@pytest.mark.parametrize("case", _random_cases(), ids=lambda c: "n{}c{}h{}w{}o{}s{}b{}".format(*c))
def test_pointwise_random(dev, case):
    """Forward (stride 1) with bias, dX, and dW + db accumulated with beta
    into existing gradients, against the oracle."""
    n, c, h, w, co, s, beta = case
    ho, wo = (h - 1) // s + 1, (w - 1) // s + 1
    seed = n * 1000 + c * 10 + co
    x = oracle.normal((n, c, h, w), seed)
    wt = oracle.normal((co, c, 1, 1), seed + 1)
    b = oracle.normal((co,), seed + 2)
    dy = oracle.normal((n, co, ho, wo), seed + 3)
    dw0 = oracle.normal((co, c, 1, 1), seed + 4)
    db0 = oracle.normal((co,), seed + 5)
    X, Wt, dY = g(x, dev), g(wt, dev), g(dy, dev)
    if s == 1:
        y = mt.conv2d(X, Wt, g(b, dev), 1, 0)
        print(f"[config] fwd {mt.last_config()}", flush=True)
        assert_close(sync_np(y), oracle.conv2d(x, wt, b, 1, 0), c, amax(x), amax(wt), "fwd",
                     extra=2e-6 * (1.0 + amax(b)))
    dX, _, _ = mt.conv2d_backward(X, Wt, dY, s, 0, need_dw=False, need_db=False)
    print(f"[config] dX {mt.last_config()}", flush=True)
    d = mt.Conv2dDesc(n, c, h, w, co, 1, 1, s, 0)
    ws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
    dW, dB = g(dw0, dev), g(db0, dev)
    rc = mt.lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                                dW.data_ptr(), beta, dB.data_ptr(), beta,
                                                mt._ptr(ws), 0 if ws is None else ws.numel(),
                                                None)
    assert rc == 0, mt.lib().mt_strerror(rc).decode()
    print(f"[config] dW {mt.last_config()}", flush=True)
    wdx, wdw, wdb = oracle.conv2d_backward(x, wt, dy, s, 0)
    K = n * ho * wo
    assert_close(sync_np(dX), wdx, co, amax(dy), amax(wt), "dX")
    assert_close(sync_np(dW), beta * dw0.astype(np.float64) + wdw, K, amax(dy), amax(x), "dW",
                 extra=1e-5)
    assert_close(sync_np(dB), beta * db0.astype(np.float64) + wdb, K, amax(dy), 1.0, "db",
                 extra=1e-5)
