"""GPU parity of the Linear GEMMs (fused bias, backward, bias gradient) and of
the conv-as-GEMM path against the CPU oracle and the reference's own vectors."""
import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def sync_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_config4_linear_forward_backward(dev):
    # benchmark config 4 (ResNet50-fc): X[256,2048] ~ N(0,1), W[1000,2048] He-init,
    # b = 0, dY[256,1000] ~ N(0, 0.01); Y = X·Wᵀ + b, dX = dY·W, dW = dYᵀ·X, db = Σ dY.
    x = oracle.normal((256, 2048), 42)
    w = oracle.normal((1000, 2048), 43, std=(2.0 / 2048) ** 0.5)
    b = np.zeros(1000, np.float32)
    dy = oracle.normal((256, 1000), 44, std=0.01)
    X, W, B, dY = g(x, dev), g(w, dev), g(b, dev), g(dy, dev)
    y = sync_np(mt.linear(X, W, B))
    print(f"[config] fwd {mt.last_config()}")
    dx, dw, db = mt.linear_backward(dY, X, W)
    dx, dw, db = sync_np(dx), sync_np(dw), sync_np(db)
    assert_close(y, oracle.linear(x, w, b), 2048, amax(x), amax(w), "C4 Y")
    wdx, wdw, wdb = oracle.linear_backward(dy, x, w)
    assert_close(dx, wdx, 1000, amax(dy), amax(w), "C4 dX")
    assert_close(dw, wdw, 256, amax(dy), amax(x), "C4 dW")
    assert_close(db, wdb, 256, amax(dy), 1.0, "C4 db")


def test_linear_nonzero_bias_and_grad_accumulation(dev):
    x = oracle.normal((100, 300), 1)
    w = oracle.normal((70, 300), 2, std=0.08)
    b = oracle.normal((70,), 3, std=0.5)
    dy = oracle.normal((100, 70), 4, std=0.1)
    X, W, B, dY = g(x, dev), g(w, dev), g(b, dev), g(dy, dev)
    y = sync_np(mt.linear(X, W, B))
    assert_close(y, oracle.linear(x, w, b), 300, amax(x), amax(w), "Y with bias", extra=1e-6)
    # accumulate_grad: a second backward adds into the first (beta = 1 epilogue)
    wdx, wdw, wdb = oracle.linear_backward(dy, x, w)
    dx, dw, db = mt.linear_backward(dY, X, W)
    mt.linear_backward(dY, X, W, need_dx=False, dw=dw, db=db, beta_w=1.0, beta_b=1.0)
    assert_close(sync_np(dw), 2 * wdw, 100, amax(dy), amax(x), "dW accumulated", extra=1e-6)
    assert_close(sync_np(db), 2 * wdb, 100, amax(dy), 1.0, "db accumulated", extra=1e-6)


def test_reference_layout_linear_via_views(dev):
    # The reference's Linear keeps W_ref [in,out] and computes matmul(x, W_ref) + b,
    # then dX = dY·W_refᵀ (view) and dW_ref = xᵀ (view)·dY (include/Module.hpp:92-114,
    # include/Autograd.hpp:117-147).  Same GEMMs through mt_gemm_f32 views.
    with np.load(GOLDEN, allow_pickle=False) as d:
        v = {k: d[k] for k in d.files}
    x, w_ref, b, dy = v["lin_x"], v["lin_w_ref"], v["lin_b"], v["lin_dy"]
    X, W, B, dY = g(x, dev), g(w_ref, dev), g(b, dev), g(dy, dev)
    y = sync_np(mt.gemm(X, W, bias=B, bias_axis=mt.BIAS_COL))
    dx = sync_np(mt.gemm(dY, W.t()))
    dw = sync_np(mt.gemm(X.t(), dY))
    db = sync_np(mt.colsum(dY))
    K = x.shape[1]
    assert_close(y, v["lin_y"], K, amax(x), amax(w_ref), "ref Linear Y", extra=1e-6)
    assert_close(dx, v["lin_dx"], w_ref.shape[1], amax(dy), amax(w_ref), "ref Linear dX")
    assert_close(dw, v["lin_dw_ref"], x.shape[0], amax(dy), amax(x), "ref Linear dW_ref")
    assert_close(db, v["lin_db"], x.shape[0], amax(dy), 1.0, "ref Linear db")


def test_golden_matmul_vectors(dev):
    with np.load(GOLDEN, allow_pickle=False) as d:
        v = {k: d[k] for k in d.files}
    # offset views: A = rows 2..4 of a [5,5] storage, B at offset 3
    As = g(v["offset_a_store"], dev)
    Bs = g(v["offset_b_store"], dev)
    A = torch.as_strided(As, (3, 5), (5, 1), 10)
    B = torch.as_strided(Bs, (5, 4), (4, 1), 3)
    assert_close(sync_np(mt.gemm(A, B)), v["offset_c"], 5, 1.0, 1.0, "golden offset views")
    bt = g(v["bT_bt"], dev)
    assert_close(sync_np(mt.gemm(g(v["bT_a"], dev), bt.t())), v["bT_c"], 47, 1.0, 1.0, "golden Bᵀ")
    row = g(v["expand_row"], dev)[None, :].expand(17, 40)
    assert_close(sync_np(mt.gemm(row, g(v["expand_b"], dev))), v["expand_c"], 40,
                 amax(v["expand_row"]), amax(v["expand_b"]), "golden expand")
    assert_close(sync_np(mt.gemm(g(v["dense_a"], dev), g(v["dense_b"], dev))), v["dense_c"], 96,
                 1.0, 1.0, "golden dense")
    out = mt.conv2d(g(v["conv_x"], dev), g(v["conv_w"], dev), g(v["conv_b"], dev), 2, 1)
    assert_close(sync_np(out), v["conv_out"], 27, amax(v["conv_x"]), amax(v["conv_w"]),
                 "golden conv", extra=1e-6)


def test_colsum_shapes(dev):
    # tall inputs (row slices, four loads in flight), ragged column groups,
    # a single row, an empty one
    for R, C in [(1, 1), (256, 1000), (1000, 3), (7, 130), (0, 5), (8192, 512), (4099, 70),
                 (63, 64), (65, 4)]:
        x = oracle.normal((R, C), R + C)
        got = sync_np(mt.colsum(g(x, dev)))
        assert_close(got, oracle.colsum(x) if R else np.zeros(C, np.float32), R, amax(x) if R else 0,
                     1.0, f"colsum {R}x{C}")
    x = oracle.normal((64, 48), 1)
    X = g(x, dev).t()  # transposed view [48,64]
    assert_close(sync_np(mt.colsum(X)), oracle.colsum(x.T), 48, amax(x), 1.0, "colsum view")
    # an unaligned column window (scalar loads) and beta
    big = oracle.normal((300, 37), 2)
    prev = oracle.normal((33,), 3)
    out = g(prev, dev)
    mt.colsum(g(big, dev)[:, 1:34], out=out, beta=0.5)
    want = oracle.colsum(np.ascontiguousarray(big[:, 1:34])).astype(np.float64) + 0.5 * prev
    assert_close(sync_np(out), want, 300, amax(big), 1.0, "colsum window + beta", extra=1e-6)


@pytest.mark.parametrize("B,fi,fo", [(8192, 512, 512), (4096, 256, 384)])
def test_linear_backward_db_in_split_k_reduction(dev, B, fi, fo):
    # tall batches: dW = dYᵀ·X takes split-K, and db rides on its reduction
    x = oracle.normal((B, fi), 31)
    w = oracle.normal((fo, fi), 32)
    dy = oracle.normal((B, fo), 33)
    prev = oracle.normal((fo,), 34)
    db = g(prev, dev)
    dX, dW, db = mt.linear_backward(g(dy, dev), g(x, dev), g(w, dev), db=db, beta_b=1.0)
    torch.cuda.synchronize()
    print(f"[config] {mt.last_config()}", flush=True)
    assert "split=1 " not in mt.last_config() + " ", mt.last_config()
    assert_close(sync_np(dW), oracle.matmul(np.ascontiguousarray(dy.T), x), B, amax(dy), amax(x),
                 "dW")
    assert_close(sync_np(db), oracle.colsum(dy).astype(np.float64) + prev, B, amax(dy), 1.0, "db",
                 extra=1e-6)
    assert_close(sync_np(dX), oracle.matmul(dy, w), fo, amax(dy), amax(w), "dX")


def seq(shape, start, step):
    return (start + step * np.arange(int(np.prod(shape)), dtype=np.float32)).reshape(shape)


def test_conv_reference_device_equivalence(dev):
    # reference test/spatial_test.cpp:209-230: [4,3,32,32] ⊛ [16,3,3,3], stride 2, pad 1,
    # sequential fills, bias 0.1; the reference allows rtol 1e-3 / atol 1e-4.
    x = seq((4, 3, 32, 32), 0.1, 0.01)
    w = seq((16, 3, 3, 3), -0.5, 0.02)
    b = np.full(16, 0.1, np.float32)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), g(b, dev), 2, 1))
    want = oracle.conv2d(x, w, b, 2, 1)
    np.testing.assert_allclose(out, want, rtol=1e-3, atol=1e-4)
    assert_close(out, want, 27, amax(x), amax(w), "spatial_test conv", extra=1e-5)


@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (1, 1, 3, 3, 1, 2, 2, 1, 0),
    (2, 5, 9, 7, 6, 3, 3, 1, 1),
    (3, 4, 11, 10, 6, 3, 2, 2, 2),
    (2, 16, 8, 8, 32, 1, 1, 1, 0),
    (1, 3, 17, 13, 8, 5, 5, 3, 1),
    (2, 8, 5, 5, 4, 7, 7, 1, 3),
    (1, 2, 2, 2, 3, 5, 5, 1, 0),   # kernel larger than the input: empty output
])
def test_conv_shapes(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), n + c)
    w = oracle.normal((co, c, kh, kw), co + kh)
    b = oracle.normal((co,), 5)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), g(b, dev), stride, pad))
    want = oracle.conv2d(x, w, b, stride, pad)
    assert out.shape == want.shape
    if want.size:
        assert_close(out, want, c * kh * kw, amax(x), amax(w), "conv", extra=1e-5)


def test_config5a_conv(dev):
    # benchmark config 5a: N=32, C=256, 14x14 -> 256, 3x3 s1 p1 (GEMM M=6272, K=2304, N=256).
    # 16 sampled output channels against the oracle's direct conv, plus the
    # channel-sum identity Σ_co out = conv(x, Σ_co w) + Σ b over every position.
    x = oracle.normal((32, 256, 14, 14), 42)
    w = oracle.normal((256, 256, 3, 3), 43, std=(2.0 / 2304) ** 0.5)
    b = np.zeros(256, np.float32)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), g(b, dev), 1, 1))
    print(f"[config] {mt.last_config()}")
    ch = np.arange(0, 256, 16)
    want = oracle.conv2d(x, w[ch], b[ch], 1, 1)
    assert_close(out[:, ch], want, 2304, amax(x), amax(w), "C5a sampled channels")
    wsum = w.astype(np.float64).sum(axis=0, keepdims=True).astype(np.float32)
    total = oracle.conv2d(x, wsum, None, 1, 1)[:, 0]
    err = np.max(np.abs(out.astype(np.float64).sum(axis=1) - total))
    bound = 256 * 1e-5 * 48 * amax(x) * amax(w) + 1e-3
    print(f"[parity] C5a channel-sum: max|err|={err:.3e} bound={bound:.3e}")
    assert err <= bound


@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 3, 9, 7, 4, 3, 3, 1, 1),
    (1, 2, 8, 8, 3, 3, 2, 2, 0),
    (3, 4, 5, 6, 2, 1, 1, 1, 0),
    (2, 2, 7, 7, 3, 5, 5, 3, 2),
    (4, 3, 32, 32, 16, 3, 3, 2, 1),   # the reference's device-equivalence conv shape
])
def test_conv_backward_shapes(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), 1)
    w = oracle.normal((co, c, kh, kw), 2)
    ho, wo = oracle.conv_out(h, pad, kh, stride), oracle.conv_out(wd, pad, kw, stride)
    dy = oracle.normal((n, co, ho, wo), 3)
    dx, dw, db = mt.conv2d_backward(g(x, dev), g(w, dev), g(dy, dev), stride, pad)
    dx, dw, db = sync_np(dx), sync_np(dw), sync_np(db)
    wdx, wdw, wdb = oracle.conv2d_backward(x, w, dy, stride, pad)
    assert_close(dx, wdx, co * kh * kw, amax(dy), amax(w), "conv dX")
    assert_close(dw, wdw, n * ho * wo, amax(dy), amax(x), "conv dW")
    assert_close(db, wdb, n * ho * wo, amax(dy), 1.0, "conv db")


def test_conv_forward_padded_stem(dev):
    """The 7x7 stride-2 RGB stem at batch 4: a dense input takes the NCHW-view
    kernel on the input and weights padded with a zero channel; a channel
    slice of a 4-channel tensor (not dense) keeps the column path.  Both with
    bias against the oracle."""
    n, c, hw, co = 4, 3, 112, 64
    x = oracle.normal((n, c, hw, hw), 71)
    w = oracle.normal((co, c, 7, 7), 72)
    b = oracle.normal((co,), 73)
    want = oracle.conv2d(x, w, b, 2, 3)
    y = mt.conv2d(g(x, dev), g(w, dev), g(b, dev), 2, 3)
    cfg = mt.last_config()
    print(f"[config] dense: {cfg}", flush=True)
    assert "b=im2col_nchw" in cfg or "b=im2col_halo" in cfg, cfg
    assert_close(sync_np(y), want, c * 49, amax(x), amax(w), "padded stem",
                 extra=2e-6 * (1.0 + amax(b)))
    wide = torch.zeros(n, c + 1, hw, hw, device=dev)
    wide[:, 1:] = g(x, dev)
    y = mt.conv2d(wide[:, 1:], g(w, dev), g(b, dev), 2, 3)
    cfg = mt.last_config()
    print(f"[config] slice: {cfg}", flush=True)
    assert "im2col" not in cfg, cfg
    assert_close(sync_np(y), want, c * 49, amax(x), amax(w), "stem on a slice",
                 extra=2e-6 * (1.0 + amax(b)))


@pytest.mark.parametrize("n,c,hw,co,k,stride,pad,padded", [
    (4, 3, 112, 64, 7, 2, 3, True),    # the RGB stem at batch 4: 3 -> 4 channels
    (2, 6, 16, 24, 3, 1, 1, True),     # 6 -> 8
    (2, 7, 12, 20, 3, 2, 1, True),     # 7 -> 8, stride 2
    (2, 5, 16, 24, 3, 1, 1, False),    # 5 -> 8 would waste 3/8: the column path
])
def test_conv_dw_padded_channels(dev, n, c, hw, co, k, stride, pad, padded):
    """dW + db of a layer whose c_in is not a multiple of 4: the implicit
    weight gradient on the input padded with zero channels (where that adds at
    most a third of the work), the real channels copied out with beta; against
    the oracle, accumulating into existing gradients, bit-identical on a
    repeat."""
    x = oracle.normal((n, c, hw, hw), 61)
    w = oracle.normal((co, c, k, k), 62)
    ho = oracle.conv_out(hw, pad, k, stride)
    dy = oracle.normal((n, co, ho, ho), 63)
    dw0 = oracle.normal((co, c, k, k), 64)
    db0 = oracle.normal((co,), 65)
    X, dY = g(x, dev), g(dy, dev)
    d = mt.Conv2dDesc(n, c, hw, hw, co, k, k, stride, pad)
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
    print(f"[config] {cfg}", flush=True)
    assert ("im2colT" in cfg) == padded, cfg
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    _, wdw, wdb = oracle.conv2d_backward(x, w, dy, stride, pad)
    K = n * ho * ho
    assert_close(outs[0][0], 0.5 * dw0.astype(np.float64) + wdw, K, amax(dy), amax(x),
                 "dW + 0.5 dW0", extra=1e-5)
    assert_close(outs[0][1], 2.0 * db0.astype(np.float64) + wdb, K, amax(dy), 1.0,
                 "db + 2 db0", extra=1e-5)


@pytest.mark.parametrize("n,co,ho,wo,off", [
    (32, 64, 112, 112, 0),   # the ResNet stem's dY (102 MB): 16-byte loads
    (32, 64, 56, 56, 1),     # dY one float off 16-byte alignment: scalar loads
    (5, 3, 7, 7, 0),         # odd positions per image: scalar loads
    (1, 300, 1, 3, 0),       # fewer items than threads
])
def test_conv_bias_grad_shapes(dev, n, co, ho, wo, off):
    """mt_conv2d_bwd_bias_f32 against the oracle's column sums of dY laid out
    [(img, position)][channel], with beta = 0.5 into an existing gradient, and
    bit-identical on a repeat."""
    dy = oracle.normal((n, co, ho, wo), 21)
    db0 = oracle.normal((co,), 22)
    flat = torch.empty(dy.size + off, device=dev)
    flat[off:] = g(dy.reshape(-1), dev)
    d = mt.Conv2dDesc(n, 1, ho, wo, co, 1, 1, 1, 0)
    outs = []
    for _ in range(2):
        dB = g(db0, dev)
        assert mt.lib().mt_conv2d_bwd_bias_f32(ctypes.byref(d), flat[off:].data_ptr(),
                                               dB.data_ptr(), 0.5, None) == 0
        outs.append(sync_np(dB))
    assert np.array_equal(outs[0], outs[1])
    want = oracle.colsum(np.ascontiguousarray(dy.transpose(0, 2, 3, 1).reshape(-1, co)))
    assert_close(outs[0], 0.5 * db0.astype(np.float64) + want, n * ho * wo, amax(dy), 1.0,
                 "conv db", extra=1e-6)


@pytest.mark.parametrize("n,c,hw,co,k,stride,pad", [
    (16, 8, 56, 16, 3, 1, 1),    # one output tile, K = 50176: implicit path, split-K reduction + db
    (16, 3, 112, 16, 7, 2, 3),   # c_in = 3: column-buffer path, db on its own
])
def test_conv_dw_many_splits(dev, n, c, hw, co, k, stride, pad):
    """Weight gradients with one or two output tiles and a long K = n·h_out·w_out
    take more than 16 splits (the workgroups would not fill the chip with 16);
    dW and db against the oracle, bit-identical on a repeat."""
    x = oracle.normal((n, c, hw, hw), 41)
    w = oracle.normal((co, c, k, k), 42)
    ho = oracle.conv_out(hw, pad, k, stride)
    dy = oracle.normal((n, co, ho, ho), 43)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    outs = []
    for _ in range(2):
        _, dw, db = mt.conv2d_backward(X, W, dY, stride, pad, need_dx=False)
        outs.append((sync_np(dw), sync_np(db)))
    cfg = mt.last_config()
    print(f"[config] {cfg}", flush=True)
    assert int(cfg.split("split=")[1].split()[0]) > 16, cfg
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    _, wdw, wdb = oracle.conv2d_backward(x, w, dy, stride, pad)
    assert_close(outs[0][0], wdw, n * ho * ho, amax(dy), amax(x), "dW")
    assert_close(outs[0][1], wdb, n * ho * ho, amax(dy), 1.0, "db")


def test_conv_bias_grad_near_2_31_items(dev):
    """2·(2^30 − 1) positions per channel, 17 GB of dY; the entry takes
    n·h_out·w_out < 2^31, and this close to the limit the channel sum runs its
    64-bit, image-by-image path.  Channel 0 holds 1, channel 1 holds 3, so the
    sums are n·hw and three times that; each thread's share is an exact
    integer in fp32 and only the final tree of 1024 partials rounds (relative
    error below 2^-20)."""
    n, hw = 2, (1 << 30) - 1
    free, _ = torch.cuda.mem_get_info(dev)
    if free < 20 << 30:
        pytest.skip("needs 20 GB of free device memory")
    dY = torch.empty(n, 2, hw, device=dev)
    dY[:, 0].fill_(1.0)
    dY[:, 1].fill_(3.0)
    d = mt.Conv2dDesc(n, 1, 1, hw, 2, 1, 1, 1, 0)
    dB = torch.tensor([5.0, 7.0], device=dev)
    assert mt.lib().mt_conv2d_bwd_bias_f32(ctypes.byref(d), dY.data_ptr(), dB.data_ptr(), 0.5,
                                           None) == 0
    got = sync_np(dB).astype(np.float64)
    want = np.array([2.5 + n * hw, 3.5 + 3.0 * n * hw])
    del dY
    torch.cuda.empty_cache()
    assert np.all(np.abs(got - want) <= want * 2.0 ** -20), (got, want)


@pytest.mark.parametrize("n,c,h,wd,co,stride,pad", [
    (4, 16, 10, 10, 24, 1, 1),    # implicit weight path (split-K: db in its reduction)
    (3, 8, 9, 11, 40, 2, 1),      # implicit, stride 2
    (2, 3, 7, 7, 5, 1, 1),        # c_in % 4 != 0: column-buffer path, db on its own
    (8, 64, 14, 14, 64, 1, 1),    # implicit with a larger K range
])
def test_conv_weight_bias_one_call(dev, n, c, h, wd, co, stride, pad):
    """mt_conv2d_bwd_weight_bias_f32 against the oracle with accumulation into
    existing gradients (beta_w = 0.5, beta_b = 2), bit-identical on a repeat,
    and db equal to the stand-alone bias entry within the bound."""
    x = oracle.normal((n, c, h, wd), 11)
    w = oracle.normal((co, c, 3, 3), 12)
    ho, wo = oracle.conv_out(h, pad, 3, stride), oracle.conv_out(wd, pad, 3, stride)
    dy = oracle.normal((n, co, ho, wo), 13)
    dw0 = oracle.normal((co, c, 3, 3), 14)
    db0 = oracle.normal((co,), 15)
    X, dY = g(x, dev), g(dy, dev)
    d = mt.Conv2dDesc(n, c, h, wd, co, 3, 3, stride, pad)
    ws = mt.workspace(mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), dev)
    outs = []
    for _ in range(2):
        dW, dB = g(dw0, dev), g(db0, dev)
        rc = mt.lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                                    dW.data_ptr(), 0.5, dB.data_ptr(), 2.0,
                                                    ws.data_ptr(), ws.numel(), None)
        assert rc == 0, mt.lib().mt_strerror(rc).decode()
        print(f"[config] {mt.last_config()}")
        outs.append((sync_np(dW), sync_np(dB)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    _, wdw, wdb = oracle.conv2d_backward(x, w, dy, stride, pad)
    dw, db = outs[0]
    assert_close(dw, 0.5 * dw0.astype(np.float64) + wdw, n * ho * wo, amax(dy), amax(x),
                 "dW + 0.5 dW0", extra=1e-5)
    assert_close(db, 2.0 * db0.astype(np.float64) + wdb, n * ho * wo, amax(dy), 1.0,
                 "db + 2 db0", extra=1e-5)
    alone = g(db0, dev)
    assert mt.lib().mt_conv2d_bwd_bias_f32(ctypes.byref(d), dY.data_ptr(), alone.data_ptr(),
                                           2.0, None) == 0
    assert_close(db, sync_np(alone).astype(np.float64), n * ho * wo, amax(dy), 1.0,
                 "db against the bias entry", extra=1e-5)
    # grad_bias = NULL: the weight gradient alone, bit-identical to its own entry
    dWa, dWb = g(dw0, dev), g(dw0, dev)
    assert mt.lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                                  dWa.data_ptr(), 0.5, None, 0.0, ws.data_ptr(),
                                                  ws.numel(), None) == 0
    assert mt.lib().mt_conv2d_bwd_weight_f32(ctypes.byref(d), X.data_ptr(), dY.data_ptr(),
                                             dWb.data_ptr(), 0.5, ws.data_ptr(), ws.numel(),
                                             None) == 0
    assert np.array_equal(sync_np(dWa), sync_np(dWb))
    assert np.array_equal(sync_np(dWa), dw)


def test_config5a_conv_backward_adjoint(dev):
    # benchmark config 5a shape: dX and dW through the GEMM path, checked by the
    # size-independent adjoint identities <dY, conv(x,w)> = <dX, x> = <dW, w>
    # (fp64 sums over every element), plus 8 sampled dW output channels and two
    # whole dX images against the oracle's conv2d_backward_{weight,input}_cpu.
    x = oracle.normal((32, 256, 14, 14), 42)
    w = oracle.normal((256, 256, 3, 3), 43, std=(2.0 / 2304) ** 0.5)
    dy = oracle.normal((32, 256, 14, 14), 44, std=0.01)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    y = mt.conv2d(X, W, None, 1, 1)
    dx, dw, db = mt.conv2d_backward(X, W, dY, 1, 1)
    y, dx, dw, db = sync_np(y), sync_np(dx), sync_np(dw), sync_np(db)
    ip = float(np.sum(dy.astype(np.float64) * y))
    ipx = float(np.sum(dx.astype(np.float64) * x))
    ipw = float(np.sum(dw.astype(np.float64) * w))
    scale = float(np.sum(np.abs(dy.astype(np.float64) * y))) + 1.0
    print(f"[parity] C5a adjoint: <dY,y>={ip:.6f} <dX,x>={ipx:.6f} <dW,w>={ipw:.6f}")
    assert abs(ipx - ip) <= 1e-5 * scale and abs(ipw - ip) <= 1e-5 * scale
    ch = np.arange(0, 256, 32)
    _, wdw, wdb = oracle.conv2d_backward(x, w[ch], dy[:, ch], 1, 1)
    assert_close(dw[ch], wdw, 32 * 196, amax(dy), amax(x), "C5a dW sampled channels")
    assert_close(db, dy.astype(np.float64).sum(axis=(0, 2, 3)), 32 * 196, amax(dy), 1.0, "C5a db")
    # dX element-wise on two whole images (first and last): an image's input
    # gradient depends only on its own dY, so the oracle's
    # conv2d_backward_input_cpu over those images alone is the exact reference
    imgs = [0, 31]
    wdx, _, _ = oracle.conv2d_backward(x[imgs], w, dy[imgs], 1, 1)
    assert_close(dx[imgs], wdx, 256 * 9, amax(dy), amax(w), "C5a dX images 0 and 31")


# ---- implicit-GEMM convolution ------------------------------------------------
# c_in % 16 == 0: the kernel gathers im2col columns from a channels-last copy
# of the input (or the input itself when it is channels-last), 16 channels of
# one filter tap per K-chunk; no column buffer.  Kernel sizes, strides,
# padding, channel counts spanning several chunks per tap, N and c_out tails
# and split-K are covered.  Other channel counts take the explicit im2col path.

@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 16, 7, 7, 32, 1, 1, 1, 0),     # 1x1 (49 positions; a multiple of 4 takes the per-image product)
    (2, 16, 9, 7, 6, 3, 3, 1, 1),
    (3, 32, 11, 10, 6, 3, 2, 2, 2),    # 3x2 kernel, stride 2, pad 2
    (1, 16, 17, 13, 8, 5, 5, 3, 1),    # 5x5, stride 3
    (2, 16, 5, 5, 4, 7, 7, 1, 3),      # 7x7 on a 5x5 image: mostly padding
    (1, 48, 5, 7, 5, 1, 1, 1, 0),      # three chunks per tap
    (1, 512, 7, 7, 64, 3, 3, 1, 1),    # kg = 4608, np = 49: split-K, scalar reduce
    (1, 512, 8, 8, 64, 3, 3, 1, 1),    # np = 64: split-K, vector reduce + row bias
    (4, 16, 13, 13, 130, 3, 3, 1, 1),  # c_out tail (clamped weight rows), np = 676
])
def test_conv_implicit_shapes(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), 7 * n + c)
    w = oracle.normal((co, c, kh, kw), co + kh)
    b = oracle.normal((co,), 5)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), g(b, dev), stride, pad))
    cfg = mt.last_config()
    print(f"[config] {cfg}")
    assert "im2col" in cfg, cfg
    want = oracle.conv2d(x, w, b, stride, pad)
    assert_close(out, want, c * kh * kw, amax(x), amax(w), "implicit conv", extra=1e-5)


# The layout launches ahead of the channels-last kernels move 2048-element
# tiles shaped to the job (32x64, 64x32 when the inner extent is <= 32, 128x16
# when <= 16), reading along the inner dimension or, for the dY copy of the
# weight gradient, along the outer one; each geometry below puts one of the
# jobs on a tile shape the benchmark layer does not use, with partial tiles:
# 4x4 and 5x5 images (pixel extent 16 / 25), 40 images (dY copy extent 40),
# 3x3 and 1x1 filters (tap extent 9 / 1), 48 channels (ragged channel tiles).
@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,pad", [
    (2, 16, 4, 4, 16, 3, 3, 1),
    (3, 32, 5, 5, 16, 3, 3, 1),
    (40, 16, 5, 5, 48, 3, 3, 1),
    (5, 48, 6, 7, 32, 1, 1, 0),
    (2, 48, 9, 9, 80, 3, 3, 1),
])
def test_conv_layout_tile_shapes(dev, n, c, h, wd, co, kh, kw, pad):
    x = oracle.normal((n, c, h, wd), 500 + n)
    w = oracle.normal((co, c, kh, kw), 501 + co)
    b = oracle.normal((co,), 502)
    X, W = g(x, dev), g(w, dev)
    out = sync_np(mt.conv2d(X, W, g(b, dev), 1, pad))
    assert "b=im2col " in mt.last_config() + " ", mt.last_config()
    assert_close(out, oracle.conv2d(x, w, b, 1, pad), c * kh * kw, amax(x), amax(w),
                 "forward", extra=1e-5)
    ho, wo = oracle.conv_out(h, pad, kh, 1), oracle.conv_out(wd, pad, kw, 1)
    dy = oracle.normal((n, co, ho, wo), 503)
    dx, dw, db = mt.conv2d_backward(X, W, g(dy, dev), 1, pad)
    wdx, wdw, wdb = oracle.conv2d_backward(x, w, dy, 1, pad)
    assert_close(sync_np(dx), wdx, co * kh * kw, amax(dy), amax(w), "dX")
    assert_close(sync_np(dw), wdw, n * ho * wo, amax(dy), amax(x), "dW")
    assert_close(sync_np(db), wdb, n * ho * wo, amax(dy), 1.0, "db")


# The implicit GEMM over an NCHW view (K order (ci, r, s), the OIHW weights
# read in place): any c_in with c_in*kh*kw % 4 == 0, including K ranges that
# end in a partial chunk, fewer K than one chunk, rectangular kernels, strides
# 2 and 3, padding 0 and 2, and output-channel tails; forward and (stride 1,
# square kernels) the input gradient.  Its B operand is built from halo
# patches in LDS where they fit (b=im2col_halo), else gathered per chunk
# (b=im2col_nchw).
NCHW_PATHS = ("b=im2col_nchw", "b=im2col_halo")
@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 4, 9, 9, 8, 3, 3, 1, 1),       # kg = 36: a partial last chunk
    (1, 12, 7, 7, 10, 5, 5, 2, 2),     # kg = 300, stride 2
    (2, 8, 5, 5, 5, 1, 1, 1, 0),       # kg = 8: less than one chunk (1x1, 25 positions)
    (1, 20, 11, 9, 7, 3, 2, 1, 1),     # 3x2 kernel
    (3, 4, 10, 12, 66, 3, 3, 3, 0),    # stride 3, no padding, c_out tail
])
def test_conv_nchw_implicit_geometries(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), 400 + c)
    w = oracle.normal((co, c, kh, kw), 401 + co)
    b = oracle.normal((co,), 402)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), g(b, dev), stride, pad))
    cfg = mt.last_config()
    print(f"[config] {cfg}")
    assert any(k in cfg for k in NCHW_PATHS), cfg
    assert_close(out, oracle.conv2d(x, w, b, stride, pad), c * kh * kw, amax(x), amax(w),
                 "NCHW implicit conv", extra=1e-5)
    if stride == 1 and kh == kw and pad <= kh - 1 and (co * kh * kw) % 4 == 0:
        ho, wo = oracle.conv_out(h, pad, kh, 1), oracle.conv_out(wd, pad, kw, 1)
        dy = oracle.normal((n, co, ho, wo), 403)
        dx, _, _ = mt.conv2d_backward(g(x, dev), g(w, dev), g(dy, dev), 1, pad, need_dw=False,
                                      need_db=False)
        cfg = mt.last_config()
        print(f"[config] dX {cfg}")
        assert any(k in cfg for k in NCHW_PATHS), cfg
        wdx, _, _ = oracle.conv2d_backward(x, w, dy, 1, pad)
        assert_close(sync_np(dx), wdx, co * kh * kw, amax(dy), amax(w), "NCHW implicit dX")


def test_conv_nchw_unaligned_weight(dev):
    """Weights that are not 16-byte aligned (a view one float into a buffer)
    are copied to the workspace the query reserves, then read as A."""
    n, c, h, wd, co = 2, 4, 9, 10, 12
    x = oracle.normal((n, c, h, wd), 404)
    w = oracle.normal((co, c, 3, 3), 405)
    buf = torch.zeros(w.size + 1, dtype=torch.float32, device=dev)
    buf[1:] = g(w.reshape(-1), dev)
    W = buf[1:].view(co, c, 3, 3)
    assert W.data_ptr() % 16 != 0
    out = sync_np(mt.conv2d(g(x, dev), W, None, 1, 1))
    cfg = mt.last_config()
    print(f"[config] {cfg}")
    assert any(k in cfg for k in NCHW_PATHS), cfg
    assert_close(out, oracle.conv2d(x, w, None, 1, 1), c * 9, amax(x), amax(w),
                 "unaligned weight")


# The halo-patch kernel (gemm_f32_dlh): bands that span image boundaries
# (images smaller than one tile, a 3-row image), strides 1-3, kernels 2x2 to
# 5x5 and 3x2 / 1x3, padding 0-2, K ranges ending in a partial chunk
# (c*kh*kw % 16 != 0) and patches of one partial channel group, every dl tile
# configuration (those whose bands fit; the others gather per chunk), and
# split factors whose K ranges start inside a patch.  A forced configuration
# takes the halo kernel wherever its patches fit (the automatic choice also
# weighs whether they pay), so the forced runs cover it.
@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 20, 14, 14, 24, 3, 3, 1, 1),    # two patches, the second partial
    (5, 4, 3, 5, 7, 3, 3, 1, 1),        # 3x5 images: a band spans many images
    (3, 12, 9, 11, 16, 3, 3, 2, 1),     # stride 2
    (2, 8, 13, 10, 9, 5, 5, 1, 2),      # 5x5, pad 2
    (2, 8, 20, 30, 9, 3, 3, 3, 1),      # stride 3
    (2, 4, 10, 9, 8, 2, 2, 1, 0),       # 2x2 (kg 16)
    (1, 36, 7, 8, 20, 3, 2, 1, 1),      # 3x2, three patches
    (2, 28, 6, 17, 12, 1, 3, 1, 1),     # 1x3
])
def test_conv_halo_geometries(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), 410 + c)
    w = oracle.normal((co, c, kh, kw), 411 + co)
    b = oracle.normal((co,), 412)
    want = oracle.conv2d(x, w, b, stride, pad)
    X, W, B = g(x, dev), g(w, dev), g(b, dev)
    out = sync_np(mt.conv2d(X, W, B, stride, pad))
    cfg = mt.last_config()
    print(f"[config] {cfg}")
    seen = [cfg]
    K = c * kh * kw
    assert_close(out, want, K, amax(x), amax(w), "halo conv", extra=1e-5)
    for tc in range(4):
        for sp in (1, 2, 3, 5):
            with mt.forced_config(mt.FAMILY_DL, tc, sp):
                out = sync_np(mt.conv2d(X, W, B, stride, pad))
                cfg = mt.last_config()
            print(f"[config] cfg {tc} split {sp}: {cfg}")
            # (a tile's band may exceed the patch limit at the larger tiles)
            assert any(k in cfg for k in NCHW_PATHS), cfg
            seen.append(cfg)
            assert_close(out, want, K, amax(x), amax(w), f"halo conv cfg {tc} split {sp}",
                         extra=1e-5)
    assert sum("b=im2col_halo" in c for c in seen) >= 4, seen
    if stride == 1 and kh == kw and pad <= kh - 1 and (co * kh * kw) % 4 == 0 and co % 16:
        ho, wo = oracle.conv_out(h, pad, kh, 1), oracle.conv_out(wd, pad, kw, 1)
        dy = oracle.normal((n, co, ho, wo), 413)
        with mt.forced_config(mt.FAMILY_DL, 2, 2):
            dx, _, _ = mt.conv2d_backward(X, W, g(dy, dev), 1, pad, need_dw=False,
                                          need_db=False)
            cfg = mt.last_config()
        print(f"[config] dX {cfg}")
        assert "b=im2col_halo" in cfg, cfg
        wdx, _, _ = oracle.conv2d_backward(x, w, dy, 1, pad)
        assert_close(sync_np(dx), wdx, co * kh * kw, amax(dy), amax(w), "halo dX")


def test_conv_halo_repeat_bitwise(dev):
    """The halo kernel sums in a fixed order: repeated calls give the same bits."""
    n, c, h, wd, co = 3, 20, 11, 13, 40
    X = g(oracle.normal((n, c, h, wd), 420), dev)
    W = g(oracle.normal((co, c, 3, 3), 421), dev)
    with mt.forced_config(mt.FAMILY_DL, 1, 2):
        a = sync_np(mt.conv2d(X, W, None, 1, 1))
        assert "b=im2col_halo" in mt.last_config(), mt.last_config()
        for _ in range(3):
            assert np.array_equal(sync_np(mt.conv2d(X, W, None, 1, 1)), a)


@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 8, 5, 5, 5, 1, 1, 1, 0),        # one tap: no patch reuse
    (1, 4, 5, 200, 6, 3, 3, 1, 1),      # 202 padded columns: the band is too wide
    (2, 8, 20, 20, 16, 3, 3, 1, 1),     # K 72: less than one patch, not worth it
])
def test_conv_nchw_gather_fallback(dev, n, c, h, wd, co, kh, kw, stride, pad):
    """Geometries the halo kernel does not take, or where its patches would not
    pay, run the per-chunk NCHW gather."""
    x = oracle.normal((n, c, h, wd), 430 + wd)
    w = oracle.normal((co, c, kh, kw), 431)
    out = sync_np(mt.conv2d(g(x, dev), g(w, dev), None, stride, pad))
    cfg = mt.last_config()
    print(f"[config] {cfg}")
    assert "b=im2col_nchw" in cfg, cfg
    assert_close(out, oracle.conv2d(x, w, None, stride, pad), c * kh * kw, amax(x), amax(w),
                 "NCHW gather conv")


@pytest.mark.parametrize("view", ["channel_slice", "spatial_crop", "nhwc", "batch_step"])
@pytest.mark.parametrize("c", [16, 3])   # 16: implicit path; 3 (kg = 27): explicit im2col
def test_conv_strided_input_views(dev, view, c):
    # Non-contiguous NCHW inputs are read in place (reference
    # conv2d_forward_kernel_strided, src/gpu_ops.cpp:2328-2399).  "nhwc" is a
    # channels-last tensor, which the implicit path uses without a copy.
    co, kh, kw, stride, pad = 6, 3, 3, 1, 1
    if view == "channel_slice":
        big = oracle.normal((2, c + 5, 9, 10), 11)
        X = g(big, dev)[:, 2:2 + c]
        xv = big[:, 2:2 + c]
    elif view == "spatial_crop":
        big = oracle.normal((2, c, 13, 15), 12)
        X = g(big, dev)[:, :, 1:10, 3:13]
        xv = big[:, :, 1:10, 3:13]
    elif view == "nhwc":
        nhwc = oracle.normal((2, 9, 10, c), 13)
        X = g(nhwc, dev).permute(0, 3, 1, 2)          # NCHW view of NHWC storage
        xv = nhwc.transpose(0, 3, 1, 2)
    else:
        big = oracle.normal((4, c, 9, 10), 14)
        X = g(big, dev)[::2]
        xv = big[::2]
    assert not X.is_contiguous()
    w = oracle.normal((co, c, kh, kw), 21)
    b = oracle.normal((co,), 22)
    out = sync_np(mt.conv2d(X, g(w, dev), g(b, dev), stride, pad))
    cfg = mt.last_config()
    print(f"[config] {view} c={c}: {cfg}")
    assert ("im2col" in cfg) == (c == 16), cfg
    want = oracle.conv2d(np.ascontiguousarray(xv), w, b, stride, pad)
    assert_close(out, want, c * kh * kw, amax(xv), amax(w), f"conv {view}", extra=1e-5)


# ---- bias gradient fused into the dW GEMM -------------------------------------
# db = Σ_batch dY is the row sum of dYᵀ, the A operand of dW = dYᵀ·X: the
# direct-to-LDS kernel accumulates it from the A fragments when the plan has
# no split-K; otherwise the column-sum kernel runs.  Both must give the same db.

def test_linear_fused_bias_grad_accumulates(dev):
    x = oracle.normal((128, 96), 31)
    w = oracle.normal((64, 96), 32, std=0.1)
    dy = oracle.normal((128, 64), 33, std=0.1)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    dw = torch.empty(64, 96, device=dev)
    db = torch.empty(64, device=dev)
    mt.linear_backward(dY, X, W, need_dx=False, dw=dw, db=db)
    print(f"[config] dW {mt.last_config()}")
    _, wdw, wdb = oracle.linear_backward(dy, x, w)
    assert_close(sync_np(db), wdb, 128, amax(dy), 1.0, "fused db")
    assert_close(sync_np(dw), wdw, 128, amax(dy), amax(x), "dW")
    mt.linear_backward(dY, X, W, need_dx=False, dw=dw, db=db, beta_w=1.0, beta_b=1.0)
    assert_close(sync_np(db), 2 * wdb, 128, amax(dy), 1.0, "fused db accumulated", extra=1e-6)
    assert_close(sync_np(dw), 2 * wdw, 128, amax(dy), amax(x), "dW accumulated", extra=1e-6)


def test_linear_bias_grad_with_split_k_dw(dev):
    x = oracle.normal((8192, 64), 41)
    w = oracle.normal((32, 64), 42, std=0.1)
    dy = oracle.normal((8192, 32), 43, std=0.1)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    _, dw, db = mt.linear_backward(dY, X, W, need_dx=False)
    print(f"[config] dW {mt.last_config()}")
    assert "split=1 " not in mt.last_config() + " "
    _, wdw, wdb = oracle.linear_backward(dy, x, w)
    assert_close(sync_np(db), wdb, 8192, amax(dy), 1.0, "db (column sums)")
    assert_close(sync_np(dw), wdw, 8192, amax(dy), amax(x), "dW split-K")


# ---- implicit dX: stride-1 backward-input as a forward convolution ------------
# dX = conv(dY, Wᵀ flipped, pad kh-1-pad) through the implicit-GEMM path
# (c_out % 16 == 0, square kernel, stride 1, pad <= kh-1); other geometries
# take the column-buffer path, covered by test_conv_backward_shapes.

@pytest.mark.parametrize("n,c,h,wd,co,k,pad", [
    (2, 5, 9, 7, 16, 3, 1),
    (1, 3, 8, 8, 32, 5, 2),
    (2, 4, 5, 7, 16, 1, 0),     # 1x1: pad' = 0 (35 positions)
    (1, 2, 7, 7, 16, 3, 0),     # pad 0: pad' = 2, output grows back to 7x7
    (1, 8, 5, 6, 16, 5, 4),     # pad = kh-1: pad' = 0
    (3, 7, 11, 10, 48, 3, 1),   # c_in tail (odd), three chunks per tap
])
def test_conv_backward_input_implicit(dev, n, c, h, wd, co, k, pad):
    x = oracle.normal((n, c, h, wd), 51)
    w = oracle.normal((co, c, k, k), 52)
    ho, wo = oracle.conv_out(h, pad, k, 1), oracle.conv_out(wd, pad, k, 1)
    dy = oracle.normal((n, co, ho, wo), 53)
    dx, _, _ = mt.conv2d_backward(g(x, dev), g(w, dev), g(dy, dev), 1, pad, need_dw=False,
                                  need_db=False)
    cfg = mt.last_config()
    print(f"[config] dX {cfg}")
    assert "im2col" in cfg, cfg
    wdx, _, _ = oracle.conv2d_backward(x, w, dy, 1, pad)
    assert_close(sync_np(dx), wdx, co * k * k, amax(dy), amax(w), "implicit conv dX")


# ---- implicit dW: weight gradient without a column buffer ---------------------
# dW[c_out, (r,s,ci)] = dYt · im2colᵀ(x) with the B operand gathered from a
# channels-last copy of x (c_in % 4 == 0, n*h_out*w_out % 4 == 0) and the
# columns scattered to OIHW by the epilogue.

@pytest.mark.parametrize("n,c,h,wd,co,kh,kw,stride,pad", [
    (2, 16, 9, 8, 6, 3, 3, 1, 1),
    (4, 8, 11, 10, 6, 3, 2, 2, 2),    # stride 2, 3x2 kernel, np = 196 (K tail 4)
    (1, 4, 8, 8, 5, 5, 5, 1, 2),
    (2, 12, 5, 6, 4, 1, 1, 1, 0),     # 1x1, np = 60 (K tail 12)
    (2, 64, 14, 14, 32, 3, 3, 1, 1),  # deep K (np = 392): split-K
])
def test_conv_backward_weight_implicit(dev, n, c, h, wd, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, wd), 61)
    w = oracle.normal((co, c, kh, kw), 62)
    ho, wo = oracle.conv_out(h, pad, kh, stride), oracle.conv_out(wd, pad, kw, stride)
    dy = oracle.normal((n, co, ho, wo), 63)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    _, dw, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dx=False, need_db=False)
    cfg = mt.last_config()
    print(f"[config] dW {cfg}")
    assert "im2colT" in cfg, cfg
    _, wdw, _ = oracle.conv2d_backward(x, w, dy, stride, pad)
    assert_close(sync_np(dw), wdw, n * ho * wo, amax(dy), amax(x), "implicit conv dW")
    # gradient accumulation: dW += ∂L/∂W through the epilogue's beta
    mt.conv2d_backward(X, W, dY, stride, pad, need_dx=False, need_db=False, dw=dw, beta_w=1.0)
    assert_close(sync_np(dw), 2 * wdw, n * ho * wo, amax(dy), amax(x), "implicit conv dW += ",
                 extra=1e-6)


# The weight gradient reads dY in NCHW as its A operand (a=kv_nchw) when a
# 16-byte group of a row is four pixels of one image (h_out*w_out % 4 == 0),
# K = n*h_out*w_out holds whole chunks (% 16 == 0) and dY is 16-byte aligned;
# otherwise dY is first copied to [c_out][n*h_out*w_out] (a=kv).  Both,
# including K ranges that start inside an image and split factors that cut
# images, against the oracle, and db summed alongside.
@pytest.mark.parametrize("n,c,h,wd,co,split,expect", [
    (4, 8, 6, 6, 24, 1, "a=kv_nchw"),    # hw 36, K 144
    (8, 12, 5, 8, 40, 3, "a=kv_nchw"),   # hw 40, K 320: splits cut images
    (3, 8, 6, 6, 24, 1, "a=kv "),        # K 108: not whole chunks
    (4, 8, 5, 5, 24, 1, "a=kv "),        # hw 25: groups straddle images
])
def test_conv_dw_dy_layout(dev, n, c, h, wd, co, split, expect):
    x = oracle.normal((n, c, h, wd), 440 + n)
    w = oracle.normal((co, c, 3, 3), 441)
    dy = oracle.normal((n, co, h, wd), 442)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    _, wdw, wdb = oracle.conv2d_backward(x, w, dy, 1, 1)
    with mt.forced_config(mt.FAMILY_DL, 3, split):
        _, dw, db = mt.conv2d_backward(X, W, dY, 1, 1, need_dx=False)
        cfg = mt.last_config()
    print(f"[config] dW {cfg}")
    assert expect in cfg + " ", cfg
    assert_close(sync_np(dw), wdw, n * h * wd, amax(dy), amax(x), "dW with dY layout")
    assert_close(sync_np(db), wdb, n * h * wd, amax(dy), 1.0, "db with dY layout")


def test_conv_dw_dy_unaligned(dev):
    """A dY view that is not 16-byte aligned is copied, not read in place.  The
    workspace query assumes 16-byte-aligned tensors, so the copy needs
    c_out*n*h_out*w_out floats (rounded up to 256 bytes) more; with only the
    queried size the call refuses (MT_ERR_WORKSPACE) before any launch."""
    n, c, h, wd, co = 4, 8, 6, 6, 24
    x = oracle.normal((n, c, h, wd), 450)
    w = oracle.normal((co, c, 3, 3), 451)
    dy = oracle.normal((n, co, h, wd), 452)
    buf = torch.zeros(dy.size + 1, dtype=torch.float32, device=dev)
    buf[1:] = g(dy.reshape(-1), dev)
    dY = buf[1:].view(n, co, h, wd)
    assert dY.data_ptr() % 16 != 0
    d = mt.Conv2dDesc(n, c, h, wd, co, 3, 3, 1, 1)
    need = mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d))
    copy = (co * n * h * wd * 4 + 255) // 256 * 256
    ws = mt.workspace(need + copy, dev)
    dW = torch.empty(co, c, 3, 3, device=dev)
    X = g(x, dev)
    assert mt.lib().mt_conv2d_bwd_weight_f32(ctypes.byref(d), X.data_ptr(),
                                             dY.data_ptr(), dW.data_ptr(), 0.0, ws.data_ptr(),
                                             need, None) == mt.MT_ERR_WORKSPACE
    assert mt.lib().mt_conv2d_bwd_weight_f32(ctypes.byref(d), X.data_ptr(),
                                             dY.data_ptr(), dW.data_ptr(), 0.0, ws.data_ptr(),
                                             ws.numel(), None) == 0
    cfg = mt.last_config()
    print(f"[config] dW {cfg}")
    assert "a=kv " in cfg + " ", cfg
    _, wdw, _ = oracle.conv2d_backward(x, w, dy, 1, 1)
    assert_close(sync_np(dW), wdw, n * h * wd, amax(dy), amax(x), "dW, unaligned dY")
