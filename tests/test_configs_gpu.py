"""Every kernel configuration against the CPU oracle.

The cost model picks one tile configuration per shape, so most configurations
would only ever run on the shapes that happen to select them.  Here each
(kernel family, tile configuration, split-K count) is forced through
mt_gemm_force_config and run on every operand layout, with K tails, batches,
the fused epilogues (bias, beta, scattered and scalar stores), the fused row
sums of the Linear weight gradient and the implicit-im2col convolution
operands.  Oracle: the reference's matmul_cpu / matmul_cpu_strided and
conv2d_cpu restated in oracle/oracle.c (include/TensorOps.hpp:139-189,
235-273); bound 1e-5·√K·max|A|·max|B| (tests/util_parity.py).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

# (family, configuration): 3 register-staged and 4 direct-to-LDS tiles that
# take every operand form; direct-to-LDS configurations 4-6 (DLP, the
# fragment-prefetching kernel with 256x256, 64x64 and 128x128 tiles) take only GEMMs
# with K % 16 == 0 and no implicit-im2col operand or fused row sums, and have
# tests of their own below.  (A CPU test pins the counts against the
# library.)
CONFIGS = [(mt.FAMILY_RS, c) for c in range(3)] + [(mt.FAMILY_DL, c) for c in range(4)]
DL_CONFIGS = [c for f, c in CONFIGS if f == mt.FAMILY_DL]
IDS = [f"{'rs' if f == mt.FAMILY_RS else 'dl'}{c}" for f, c in CONFIGS]
DLPS = [4, 5, 6]


def g(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def operand(a: np.ndarray, layout: str, dev) -> torch.Tensor:
    """The logical matrix `a` on the GPU, row-major or as a transposed view of
    column-major storage (so A is mn- and B k-contiguous)."""
    if layout == "row":
        return g(a, dev)
    return g(np.ascontiguousarray(a.T), dev).t()


def sync_np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check_config(family: int, cfg: int, splits: int = None) -> str:
    name = mt.last_config()
    print(f"[config] {name}", flush=True)
    assert name.startswith("dl " if family == mt.FAMILY_DL else "rs "), name
    assert name.endswith(f" cfg={cfg}"), name
    if splits is not None:
        assert f" split={splits} " in name, name
    return name


@pytest.mark.parametrize("fc", CONFIGS, ids=IDS)
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("la", ["row", "col"])
@pytest.mark.parametrize("lb", ["row", "col"])
def test_forced_config_layouts(dev, fc, splits, la, lb):
    family, cfg = fc
    # Tails in M, N (for every tile) and K; every dimension a multiple of 4 so
    # all four layouts are vector layouts (16-byte rows) for either family.
    M, N, K = 200, 136, 76
    a = oracle.uniform((M, K), 100 + cfg)
    b = oracle.uniform((K, N), 200 + cfg)
    A, B = operand(a, la, dev), operand(b, lb, dev)
    with mt.forced_config(family, cfg, splits):
        C = mt.gemm(A, B)
        check_config(family, cfg, splits)
    assert_close(sync_np(C), oracle.matmul(a, b), K, amax(a), amax(b),
                 f"forced {family}/{cfg} split {splits} a={la} b={lb}")


@pytest.mark.parametrize("fc", CONFIGS, ids=IDS)
@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("axis", [mt.BIAS_ROW, mt.BIAS_COL])
def test_forced_config_batched_bias_beta(dev, fc, splits, axis):
    family, cfg = fc
    batch, M, N, K = 3, 96, 72, 52
    a = oracle.uniform((batch, M, K), 300 + cfg)
    b = oracle.uniform((batch, K, N), 400 + cfg)
    c0 = oracle.uniform((batch, M, N), 500 + cfg)
    bias = oracle.uniform((M if axis == mt.BIAS_ROW else N,), 600 + cfg)
    C = g(c0, dev)
    with mt.forced_config(family, cfg, splits):
        mt.gemm(g(a, dev), g(b, dev), out=C, bias=g(bias, dev), bias_axis=axis, beta=0.5)
        check_config(family, cfg, splits)
    bb = bias[None, :, None] if axis == mt.BIAS_ROW else bias[None, None, :]
    want = oracle.bmm(a, b) + bb + 0.5 * c0
    assert_close(sync_np(C), want, K, amax(a), amax(b),
                 f"forced {family}/{cfg} batched bias {axis} beta", extra=2e-6)


@pytest.mark.parametrize("fc", CONFIGS, ids=IDS)
@pytest.mark.parametrize("splits", [1, 16])
def test_forced_config_scalar_epilogue(dev, fc, splits):
    # N % 4 != 0: element-wise stores (and element-wise split-K partials); the
    # output is a column slice of a wider buffer, B is k-contiguous.  16
    # splits of K = 132 come out as 9 (one 16-deep chunk each, the last 4 deep).
    family, cfg = fc
    M, N, K = 70, 130, 132
    a = oracle.uniform((M, K), 700 + cfg)
    b = oracle.uniform((K, N), 800 + cfg)
    wide = torch.zeros(M, N + 7, device=dev)
    with mt.forced_config(family, cfg, splits):
        mt.gemm(g(a, dev), operand(b, "col", dev), out=wide[:, 3:3 + N])
        check_config(family, cfg, 9 if splits == 16 else 1)
    got = sync_np(wide)
    assert_close(got[:, 3:3 + N], oracle.matmul(a, b), K, amax(a), amax(b),
                 f"forced {family}/{cfg} scalar epilogue")
    assert not got[:, :3].any() and not got[:, 3 + N:].any(), "wrote outside the view"


@pytest.mark.parametrize("family", [mt.FAMILY_RS])
def test_forced_rs_k0_writes_bias(dev, family):
    # K = 0: no operand is read; the output is the bias (the register-staged
    # family takes it; the direct-to-LDS family needs operands to stream).
    bias = oracle.uniform((40,), 901)
    A = torch.empty(33, 0, device=dev)
    B = torch.empty(0, 40, device=dev)
    with mt.forced_config(family, 2, 1):
        C = mt.gemm(A, B, bias=g(bias, dev), bias_axis=mt.BIAS_COL)
    np.testing.assert_array_equal(sync_np(C), np.broadcast_to(bias, (33, 40)))


@pytest.mark.parametrize("cfg", DL_CONFIGS + DLPS)
@pytest.mark.parametrize("rows", [301, 256])
def test_forced_dl_linear_dw_fused_row_sums(dev, cfg, rows):
    # dW = dYᵀ·X with db = Σ_rows dY fused into the same launch (both operands
    # mn-contiguous, no split): every direct-to-LDS tile, with and without a
    # K tail (K = rows), then accumulated with beta = 1.
    x = oracle.normal((rows, 96), 910 + cfg)
    w = oracle.normal((72, 96), 920 + cfg, std=0.1)
    dy = oracle.normal((rows, 72), 930 + cfg, std=0.1)
    dw = torch.empty(72, 96, device=dev)
    db = torch.empty(72, device=dev)
    with mt.forced_config(mt.FAMILY_DL, cfg, 1):
        mt.linear_backward(g(dy, dev), g(x, dev), g(w, dev), need_dx=False, dw=dw, db=db)
        check_config(mt.FAMILY_DL, cfg, 1)
    _, wdw, wdb = oracle.linear_backward(dy, x, w)
    assert_close(sync_np(dw), wdw, rows, amax(dy), amax(x), f"forced dl{cfg} dW")
    assert_close(sync_np(db), wdb, rows, amax(dy), 1.0, f"forced dl{cfg} fused db")
    with mt.forced_config(mt.FAMILY_DL, cfg, 1):
        mt.linear_backward(g(dy, dev), g(x, dev), g(w, dev), need_dx=False, dw=dw, db=db,
                           beta_w=1.0, beta_b=1.0)
    # two sums of `rows` products each: twice the bound (4·rows under the root)
    assert_close(sync_np(db), 2 * wdb, 4 * rows, amax(dy), 1.0,
                 f"forced dl{cfg} fused db, beta 1")
    assert_close(sync_np(dw), 2 * wdw, 4 * rows, amax(dy), amax(x),
                 f"forced dl{cfg} dW, beta 1")


@pytest.mark.parametrize("cfg", DL_CONFIGS)
@pytest.mark.parametrize("splits", [1, 4])
def test_forced_dl_implicit_conv(dev, cfg, splits):
    # Implicit-im2col forward (c_in % 16 == 0): B gathered from channels-last x.
    n, c, h, wd, co, k, stride, pad = 2, 32, 9, 10, 40, 3, 1, 1
    x = oracle.normal((n, c, h, wd), 940 + cfg)
    w = oracle.normal((co, c, k, k), 950 + cfg)
    b = oracle.normal((co,), 960 + cfg)
    with mt.forced_config(mt.FAMILY_DL, cfg, splits):
        out = mt.conv2d(g(x, dev), g(w, dev), g(b, dev), stride, pad)
        name = check_config(mt.FAMILY_DL, cfg, splits)
    assert "im2col" in name, name
    assert_close(sync_np(out), oracle.conv2d(x, w, b, stride, pad), c * k * k, amax(x), amax(w),
                 f"forced dl{cfg} implicit conv", extra=1e-5)


@pytest.mark.parametrize("cfg", DL_CONFIGS + DLPS)
@pytest.mark.parametrize("splits", [1, 3])
def test_forced_dl_implicit_conv_weight_grad(dev, cfg, splits):
    # Implicit dW (B = im2colᵀ of channels-last x, columns scattered to OIHW),
    # K = n*h_out*w_out = 180: a K tail, then gradient accumulation via beta.
    n, c, h, wd, co, k, stride, pad = 2, 8, 9, 10, 12, 3, 1, 1
    x = oracle.normal((n, c, h, wd), 970 + cfg)
    w = oracle.normal((co, c, k, k), 980 + cfg)
    ho, wo = oracle.conv_out(h, pad, k, stride), oracle.conv_out(wd, pad, k, stride)
    dy = oracle.normal((n, co, ho, wo), 990 + cfg)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)
    with mt.forced_config(mt.FAMILY_DL, cfg, splits):
        _, dw, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dx=False, need_db=False)
        name = check_config(mt.FAMILY_DL, cfg, splits)
        assert "im2colT" in name, name
        _, wdw, _ = oracle.conv2d_backward(x, w, dy, stride, pad)
        assert_close(sync_np(dw), wdw, n * ho * wo, amax(dy), amax(x), f"forced dl{cfg} conv dW")
        mt.conv2d_backward(X, W, dY, stride, pad, need_dx=False, need_db=False, dw=dw, beta_w=1.0)
    assert_close(sync_np(dw), 2 * wdw, n * ho * wo, amax(dy), amax(x),
                 f"forced dl{cfg} conv dW += ", extra=1e-6)


def test_forced_split_without_workspace_is_an_error(dev):
    a = g(oracle.uniform((64, 256), 1), dev)
    b = g(oracle.uniform((256, 64), 2), dev)
    c = torch.empty(64, 64, device=dev)
    with mt.forced_config(mt.FAMILY_DL, 2, 4):
        rc = mt.lib().mt_gemm_f32(mt.mat(a), mt.mat(b), mt.mat(c), None, None, 0, None)
    assert rc == mt.MT_ERR_WORKSPACE


@pytest.mark.parametrize("fc", CONFIGS + [(mt.FAMILY_DL, c) for c in DLPS],
                         ids=IDS + [f"dl{c}" for c in DLPS])
@pytest.mark.parametrize("splits", [1, 4])
def test_forced_config_special_values(dev, fc, splits):
    # IEEE special values go through every kernel as through matmul_cpu
    # (include/TensorOps.hpp:139-160): fp32 denormal operands and products are
    # kept (no flush to zero; exact here, every product and partial sum is a
    # multiple of 2^-149 well inside range), NaN and ±Inf reach the same
    # outputs with the same signs, and the accumulator starts at +0.
    family, cfg = fc
    M, N, K = 72, 68, 128
    with mt.forced_config(family, cfg, splits):
        a = np.full((M, K), 2.0 ** -70, np.float32)
        b = np.full((K, N), 2.0 ** -70, np.float32)            # products 2^-140: denormal
        c = mt.gemm(g(a, dev), g(b, dev))
        check_config(family, cfg, splits)
        np.testing.assert_array_equal(sync_np(c), oracle.matmul(a, b))
        assert sync_np(c)[0, 0] == np.float32(K * 2.0 ** -140) != 0

        a = oracle.uniform((M, K), 31)
        b = oracle.uniform((K, N), 32)
        a[3, 5], a[7, 2], b[4, 9], b[100, 60] = np.nan, np.inf, -np.inf, np.nan
        got, want = sync_np(mt.gemm(g(a, dev), g(b, dev))), oracle.matmul(a, b)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
        np.testing.assert_array_equal(np.isposinf(got), np.isposinf(want))
        np.testing.assert_array_equal(np.isneginf(got), np.isneginf(want))
        fin = np.isfinite(want)
        assert_close(np.where(fin, got, 0), np.where(fin, want, 0), K, 1.0, 1.0,
                     f"forced {family}/{cfg} finite entries next to NaN/Inf")

        z = np.zeros((M, K), np.float32) * -1.0                  # -0.0 operands
        got = sync_np(mt.gemm(g(z, dev), g(np.ones((K, N), np.float32), dev)))
        np.testing.assert_array_equal(np.signbit(got), np.signbit(oracle.matmul(z, np.ones((K, N), np.float32))))


def expected_splits(K: int, asked: int) -> int:
    kps = -(-(-(-K // asked)) // 16) * 16
    return -(-K // kps)


@pytest.mark.parametrize("DLP", DLPS)
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("la", ["row", "col"])
@pytest.mark.parametrize("lb", ["row", "col"])
@pytest.mark.parametrize("M,N,K", [(300, 264, 96), (260, 260, 16), (512, 256, 48),
                                   (1000, 1020, 272), (300, 264, 100), (260, 260, 8),
                                   (64, 68, 1036)])
def test_forced_dlp_layouts(dev, DLP, splits, la, lb, M, N, K):
    # The prefetching kernel on every vector layout: ragged M and N (clamped
    # loads, masked stores), 1, 2, 3 (odd: the unrolled loop's last step) and
    # 17 chunks per split, a single tile and a 4x4 grid; K tails of 4, 8 and
    # 12 (the last chunk partly from the zero page), also with K < 16.
    a = oracle.uniform((M, K), 1100 + K)
    b = oracle.uniform((K, N), 1200 + K)
    A, B = operand(a, la, dev), operand(b, lb, dev)
    with mt.forced_config(mt.FAMILY_DL, DLP, splits):
        C = mt.gemm(A, B)
        check_config(mt.FAMILY_DL, DLP, expected_splits(K, splits))
    assert_close(sync_np(C), oracle.matmul(a, b), K, amax(a), amax(b),
                 f"forced dl{DLP} split {splits} a={la} b={lb} {M}x{N}x{K}")


@pytest.mark.parametrize("DLP", DLPS)
@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("axis", [mt.BIAS_ROW, mt.BIAS_COL])
def test_forced_dlp_batched_bias_beta(dev, DLP, splits, axis):
    batch, M, N, K = 3, 96, 72, 64
    a = oracle.uniform((batch, M, K), 1300)
    b = oracle.uniform((batch, K, N), 1400)
    c0 = oracle.uniform((batch, M, N), 1500)
    bias = oracle.uniform((M if axis == mt.BIAS_ROW else N,), 1600)
    C = g(c0, dev)
    with mt.forced_config(mt.FAMILY_DL, DLP, splits):
        mt.gemm(g(a, dev), g(b, dev), out=C, bias=g(bias, dev), bias_axis=axis, beta=0.5)
        check_config(mt.FAMILY_DL, DLP, splits)
    bb = bias[None, :, None] if axis == mt.BIAS_ROW else bias[None, None, :]
    want = oracle.bmm(a, b) + bb + 0.5 * c0
    assert_close(sync_np(C), want, K, amax(a), amax(b),
                 f"forced dl{DLP} batched bias {axis} beta", extra=2e-6)


@pytest.mark.parametrize("DLP", DLPS)
def test_forced_dlp_strided_output_view(dev, DLP):
    # A row slice of a wider, 16-byte-aligned buffer (row stride 264 > N):
    # vector stores through c_m, neighbours untouched.
    M, N, K = 130, 256, 32
    a = oracle.uniform((M, K), 1700)
    b = oracle.uniform((K, N), 1701)
    wide = torch.zeros(M, N + 8, device=dev)
    with mt.forced_config(mt.FAMILY_DL, DLP, 1):
        mt.gemm(g(a, dev), g(b, dev), out=wide[:, 4:4 + N])
        check_config(mt.FAMILY_DL, DLP, 1)
    got = sync_np(wide)
    assert_close(got[:, 4:4 + N], oracle.matmul(a, b), K, amax(a), amax(b), "dlp strided out")
    assert not got[:, :4].any() and not got[:, 4 + N:].any(), "wrote outside the view"


@pytest.mark.parametrize("DLP", DLPS)
@pytest.mark.parametrize("splits", [1, 3])
def test_forced_dlp_scalar_and_misaligned_outputs(dev, DLP, splits):
    # N % 4 != 0 (element-wise stores and element-wise split-K partials; B is
    # k-contiguous so it stays a vector layout) and a C that starts 4 bytes
    # past a 16-byte boundary, with bias and beta.
    for M, N, K, off in [(300, 270, 96, 0), (260, 256, 48, 1)]:
        a = oracle.uniform((M, K), 1800 + N)
        b = oracle.uniform((K, N), 1900 + N)
        bias = oracle.uniform((N,), 1950 + N)
        c0 = oracle.uniform((M, N), 1960 + N)
        buf = torch.zeros(M * N + off, device=dev)
        C = buf[off:].view(M, N)
        C.copy_(g(c0, dev))
        with mt.forced_config(mt.FAMILY_DL, DLP, splits):
            mt.gemm(g(a, dev), operand(b, "col", dev), out=C, bias=g(bias, dev),
                    bias_axis=mt.BIAS_COL, beta=-1.5)
            check_config(mt.FAMILY_DL, DLP, expected_splits(K, splits))
        want = oracle.matmul(a, b) + bias[None, :] - 1.5 * c0
        assert_close(sync_np(C), want, K, amax(a), amax(b), f"dlp {M}x{N}x{K}+{off}", extra=2e-6)
        if off:
            assert sync_np(buf)[0] == 0, "wrote before the output"


def _not_dlp(name: str) -> None:
    print(f"[config] {name}", flush=True)
    assert not (name.startswith("dl ") and any(name.endswith(f" cfg={c}") for c in DLPS)), name


@pytest.mark.parametrize("DLP", DLPS)
def test_forced_dlp_outside_its_contract_uses_the_cost_model(dev, DLP):
    # A forced prefetching configuration where its contract does not hold: the
    # launch takes the cost model's plan instead, and the result is still
    # exact.  The implicit-im2col convolution forward keeps gemm_f32_dl:
    n, c, h, wd, co, k = 2, 32, 9, 10, 40, 3
    xc = oracle.normal((n, c, h, wd), 2003)
    wc = oracle.normal((co, c, k, k), 2004)
    with mt.forced_config(mt.FAMILY_DL, DLP, 1):
        out = mt.conv2d(g(xc, dev), g(wc, dev), None, 1, 1)
        name = mt.last_config()
        _not_dlp(name)
    assert "im2col" in name, name
    assert_close(sync_np(out), oracle.conv2d(xc, wc, None, 1, 1), c * k * k, amax(xc), amax(wc),
                 "dlp fallback implicit conv")
