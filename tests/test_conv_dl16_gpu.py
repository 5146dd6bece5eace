"""The convolution kernel on 16x16 MFMA blocks (gemm_f32_dl16, direct-to-LDS
configuration 7: 64x112 tiles, K-chunks split over two groups of waves)
against the CPU oracle, forced through mt_gemm_force_config on the
channels-last implicit-im2col operand, and taken by the cost model.

Cases: ragged output channels and pixels (tiles past M and N), K ranges of
one chunk (empty wave groups), odd chunk counts (groups with one chunk less),
1x1 to 5x5 kernels, strides 1-2, padding, bias, split-K on top, the input
gradient through the flipped-weight forward convolution, determinism, and
the 5a layer at full size against the cost model's own plan.  Oracle: the
reference's conv2d_cpu / conv2d_backward_input_cpu restated in
oracle/oracle.c (include/TensorOps.hpp:235-273, 276-310); bound
1e-5*sqrt(K)*max|x|*max|w| (tests/util_parity.py).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

DL16 = [7]
TILE = {7: "64x112"}

# n, c_in, h, w, c_out, k, stride, pad
SHAPES = [
    (2, 32, 14, 14, 64, 3, 1, 1),     # 392 pixels: 3.5 tiles of 112
    (1, 16, 17, 17, 48, 5, 2, 2),     # 48 output channels: a partial tile row
    (3, 64, 7, 7, 80, 1, 1, 0),       # 1x1, 147 pixels
    (2, 16, 9, 11, 40, 3, 1, 1),      # K = 144: 9 chunks (odd)
    (4, 16, 5, 5, 64, 1, 1, 0),       # K = 16: one chunk, other groups idle
    (1, 128, 8, 8, 96, 3, 2, 1),      # K = 1152, stride 2
]


def _run(dev, cfg, shape, splits=1, bias=True):
    n, c, h, w, co, k, stride, pad = shape
    seed = 900 + 7 * cfg + sum(shape)
    x = oracle.normal((n, c, h, w), seed)
    wt = oracle.normal((co, c, k, k), seed + 1)
    b = oracle.normal((co,), seed + 2) if bias else None
    X, W = torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev)
    Bt = torch.from_numpy(b).to(dev) if bias else None
    with mt.forced_config(mt.FAMILY_DL, cfg, splits):
        y = mt.conv2d(X, W, Bt, stride, pad)
        name = mt.last_config()
        y2 = mt.conv2d(X, W, Bt, stride, pad)
    print(f"[config] {shape} split={splits} -> {name}", flush=True)
    torch.cuda.synchronize()
    assert name.startswith(f"dl {TILE[cfg]} ") and "b=im2col " in name and name.endswith(
        f" cfg={cfg}"), name
    y, y2 = y.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "not deterministic"
    extra = 2e-6 * (1.0 + amax(b)) if bias else 0.0
    assert_close(y, oracle.conv2d(x, wt, b, stride, pad), c * k * k, amax(x), amax(wt),
                 f"dl16 cfg {cfg} {shape} split {splits}", extra=extra)
    return name


@pytest.mark.parametrize("cfg", DL16)
@pytest.mark.parametrize("shape", SHAPES, ids=[f"s{i}" for i in range(len(SHAPES))])
def test_forced_forward(dev, cfg, shape):
    _run(dev, cfg, shape, bias=shape[1] != 64)


@pytest.mark.parametrize("cfg", DL16)
@pytest.mark.parametrize("splits", [2, 3])
def test_forced_split_k(dev, cfg, splits):
    name = _run(dev, cfg, (1, 256, 7, 7, 64, 3, 1, 1), splits=splits)
    assert f"split={splits} " in name


@pytest.mark.parametrize("cfg", DL16)
def test_forced_input_gradient(dev, cfg):
    """Stride 1, square kernel: dX is the forward convolution of dY with the
    flipped weights, through the same kernel."""
    n, c, h, w, co, k, pad = 2, 24, 10, 13, 32, 3, 1
    seed = 1300 + cfg
    x = oracle.normal((n, c, h, w), seed)
    wt = oracle.normal((co, c, k, k), seed + 1)
    dy = oracle.normal((n, co, h, w), seed + 2)
    with mt.forced_config(mt.FAMILY_DL, cfg, 1):
        dX, _, _ = mt.conv2d_backward(torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev),
                                      torch.from_numpy(dy).to(dev), 1, pad, need_dw=False,
                                      need_db=False)
        name = mt.last_config()
    print(f"[config] dX -> {name}", flush=True)
    torch.cuda.synchronize()
    assert name.endswith(f" cfg={cfg}"), name
    wdx, _, _ = oracle.conv2d_backward(x, wt, dy, 1, pad)
    assert_close(dX.cpu().numpy(), wdx, co * k * k, amax(dy), amax(wt), f"dl16 cfg {cfg} dX")


@pytest.mark.parametrize("cfg", DL16)
def test_full_size_5a_layer(dev, cfg):
    """n 32, 256 -> 256 channels, 14x14, 3x3: each forced configuration against
    the cost model's plan, and both against the oracle on sampled outputs."""
    x = oracle.normal((32, 256, 14, 14), 71)
    wt = (oracle.normal((256, 256, 3, 3), 72) * np.float32(np.sqrt(2.0 / 2304))).astype(np.float32)
    X, W = torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev)
    auto = mt.conv2d(X, W, None, 1, 1)
    with mt.forced_config(mt.FAMILY_DL, cfg, 1):
        y = mt.conv2d(X, W, None, 1, 1)
        name = mt.last_config()
    print(f"[config] 5a -> {name}", flush=True)
    torch.cuda.synchronize()
    assert name.endswith(f" cfg={cfg}") and "split=1 " in name, name
    y, auto = y.cpu().numpy(), auto.cpu().numpy()
    bound = 1e-5 * np.sqrt(2304) * amax(x) * amax(wt)
    assert np.max(np.abs(y - auto)) <= 2 * bound
    # exact sums of two images against the oracle (the whole batch is slow on the CPU)
    for img in (0, 31):
        want = oracle.conv2d(x[img:img + 1], wt, None, 1, 1)
        assert_close(y[img:img + 1], want, 2304, amax(x), amax(wt), f"dl16 cfg {cfg} 5a img {img}")


def test_cost_model_takes_it_for_a_28x28_layer(dev):
    """n 32, 128 -> 128 channels, 28x28, 3x3: 448 tiles of 64x112, two per CU
    (the plan measured 88.9 us against 96.3 for the 128x128 tile)."""
    x = oracle.normal((32, 128, 28, 28), 81)
    wt = (oracle.normal((128, 128, 3, 3), 82) * np.float32(np.sqrt(2.0 / 1152))).astype(np.float32)
    b = oracle.normal((128,), 83)
    y = mt.conv2d(torch.from_numpy(x).to(dev), torch.from_numpy(wt).to(dev),
                  torch.from_numpy(b).to(dev), 1, 1)
    name = mt.last_config()
    print(f"[config] 28x28 -> {name}", flush=True)
    torch.cuda.synchronize()
    assert name == "dl 64x112 a=kv b=im2col split=1 wgs=448 cfg=7", name
    y = y.cpu().numpy()
    for img in (0, 17):
        want = oracle.conv2d(x[img:img + 1], wt, b, 1, 1)
        assert_close(y[img:img + 1], want, 1152, amax(x), amax(wt), f"28x28 img {img}",
                     extra=2e-6 * (1.0 + amax(b)))


def test_cost_model_keeps_the_5a_layer_off_it(dev):
    """224 tiles of 64x112 would run one workgroup per CU: the 5a layer keeps
    the 256x128 tile with split-K."""
    x = torch.zeros(32, 256, 14, 14, device=dev)
    w = torch.zeros(256, 256, 3, 3, device=dev)
    mt.conv2d(x, w, None, 1, 1)
    assert mt.last_config().startswith("dl 256x128 "), mt.last_config()


def test_graph_replays_match_eager(dev):
    """The 28x28 layer's forward and input gradient (both on this kernel)
    captured in a HIP graph: every replay, with the inputs changed in place
    between them, gives the eager result bit for bit."""
    import ctypes
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    x = torch.randn(32, 128, 28, 28, device=dev, generator=gen)
    w = torch.randn(128, 128, 3, 3, device=dev, generator=gen) * 0.03
    b = torch.randn(128, device=dev, generator=gen)
    dy = torch.randn(32, 128, 28, 28, device=dev, generator=gen) * 0.01
    d = mt.Conv2dDesc(32, 128, 28, 28, 128, 3, 3, 1, 1)
    ws = mt.workspace(max(mt.lib().mt_conv2d_workspace_f32(ctypes.byref(d)),
                          mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d))), dev)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    names = []

    def step():
        y.copy_(mt.conv2d(x, w, b, 1, 1, ws=ws))
        names.append(mt.last_config())
        gx, _, _ = mt.conv2d_backward(x, w, dy, 1, 1, need_dw=False, need_db=False, ws=ws)
        names.append(mt.last_config())
        dx.copy_(gx)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert all(n.endswith(" cfg=7") for n in names[:2]), names[:2]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for rep in range(3):
        x.mul_(0.5).add_(0.1)
        dy.mul_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = (y.clone(), dx.clone())
        step()
        torch.cuda.synchronize()
        assert torch.equal(got[0], y) and torch.equal(got[1], dx), f"replay {rep} differs"
        print(f"[graph] dl16 replay {rep} == eager", flush=True)


def _random_case(rng, i):
    while True:
        kh = int(rng.integers(1, 6))
        kw = kh if rng.random() < 0.5 else int(rng.integers(1, 6))
        d = dict(n=int(rng.integers(1, 5)), c=16 * int(rng.integers(1, 6)),
                 co=int(rng.integers(1, 150)), h=int(rng.integers(1, 24)),
                 w=int(rng.integers(1, 24)), kh=kh, kw=kw, stride=int(rng.integers(1, 4)),
                 pad=int(rng.integers(0, 3)), split=int(rng.choice([1, 1, 2, 3])),
                 view=str(rng.choice(["dense", "dense", "channel_slice", "nhwc"])),
                 bias=bool(rng.random() < 0.6), seed=9100 + 10 * i)
        if (oracle.conv_out(d["h"], d["pad"], kh, d["stride"]) > 0
                and oracle.conv_out(d["w"], d["pad"], kw, d["stride"]) > 0):
            return d


N_RANDOM = 24
_rng = np.random.default_rng(20261204)
RANDOM_CASES = [_random_case(_rng, i) for i in range(N_RANDOM)]


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"r{i}" for i in range(N_RANDOM)])
def test_random_forced(dev, case):
    """Seeded draws on configuration 7: c_in a multiple of 16 (the channels-last
    operand), any c_out (ragged tile rows), 1x1 to 5x5 kernels, strides 1-3,
    padding 0-2, dense, channel-slice or channels-last NCHW views, bias or none,
    split-K 1-3."""
    n, c, h, wd, co = case["n"], case["c"], case["h"], case["w"], case["co"]
    kh, kw, stride, pad, seed = case["kh"], case["kw"], case["stride"], case["pad"], case["seed"]
    x = oracle.normal((n, c, h, wd), seed)
    w = oracle.normal((co, c, kh, kw), seed + 1)
    b = oracle.normal((co,), seed + 2) if case["bias"] else None
    if case["view"] == "channel_slice":
        big = np.zeros((n, c + 3, h, wd), np.float32)
        big[:, 1:1 + c] = x
        X = torch.from_numpy(big).to(dev)[:, 1:1 + c]
    elif case["view"] == "nhwc":
        X = torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 3, 1))).to(dev).permute(0, 3, 1, 2)
    else:
        X = torch.from_numpy(x).to(dev)
    W = torch.from_numpy(w).to(dev)
    Bt = torch.from_numpy(b).to(dev) if b is not None else None
    with mt.forced_config(mt.FAMILY_DL, 7, case["split"]):
        y = mt.conv2d(X, W, Bt, stride, pad)
        name = mt.last_config()
    torch.cuda.synchronize()
    print(f"[case] {case} -> {name}", flush=True)
    assert name.startswith("dl 64x112 ") and name.endswith(" cfg=7"), name
    extra = 2e-6 * (1.0 + amax(b)) if b is not None else 0.0
    assert_close(y.cpu().numpy(), oracle.conv2d(x, w, b, stride, pad), c * kh * kw, amax(x),
                 amax(w), f"dl16 random {case}", extra=extra)


def test_output_beyond_2pow31_elements(dev):
    """1x1, 16 -> 8320 channels, batch 64, 65x65: 2.25e9 output elements
    (9.0 GB); images 62 and 63 start past 2^31, so a 32-bit index anywhere in
    the loaders or the scattered NCHW store would alias.  Sampled channels of
    the first and last images against the oracle."""
    n, c, hw, co = 64, 16, 65, 8320
    x = oracle.normal((n, c, hw, hw), 95)
    w = oracle.normal((co, c, 1, 1), 96)
    b = oracle.normal((co,), 97)
    with mt.forced_config(mt.FAMILY_DL, 7, 1):
        y = mt.conv2d(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev),
                      torch.from_numpy(b).to(dev), 1, 0)
        name = mt.last_config()
    torch.cuda.synchronize()
    print(f"[config] {name}", flush=True)
    assert name.endswith(" cfg=7"), name
    chans = np.array([0, 1, 4095, 4096, 8191, 8318, 8319], np.int64)
    for img in (0, 63):
        got = y[img, torch.from_numpy(chans).to(dev)].cpu().numpy()
        want = oracle.conv2d(x[img:img + 1], w[chans], b[chans], 1, 0)[0]
        assert_close(got, want, c, amax(x), amax(w), f"img {img} past 2^31",
                     extra=2e-6 * (1.0 + amax(b)))
    del y
    torch.cuda.empty_cache()
