"""GPU parity of the vector-ALU kernels of the HBM-bound shapes (GEMV for at
most 8 rows of A or columns of B, rank-k for K <= 16, forced where the cost model
prefers the MFMA kernels) against the CPU oracle
(the reference's matmul_cpu / matmul_cpu_strided restated in oracle/oracle.c).

The shapes include the reference benchmark's skinny rows
(test/benchmark.cpp:732,737-738: 1x4096·4096x4096, 4096x1·1x4096, and
63x4096·4096x4096, which keeps the MFMA kernels).  Bound:
max|err| <= 1e-5·√K·max|A|·max|B| (tests/util_parity.py), plus the bias and
beta terms where fused.
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu


def g(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gemm(A, B, **kw):
    C = mt.gemm(A, B, **kw)
    torch.cuda.synchronize()
    cfg = mt.last_config()
    print(f"[config] {cfg}", flush=True)
    return C, cfg


@pytest.mark.parametrize("M,N,K", [
    (1, 4096, 4096),    # the reference's vector x matrix row
    (1, 256, 17), (2, 1000, 100), (3, 4, 513), (5, 260, 2048), (8, 4096, 777),
    (7, 8, 64), (4, 12, 4099),
])
def test_gemv_row_major_b(dev, M, N, K):
    a = oracle.uniform((M, K), 100 + M)
    b = oracle.uniform((K, N), 200 + N)
    c, cfg = gemm(g(a, dev), g(b, dev))
    assert cfg.startswith("sk gemv_mv "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), f"{M}x{N}x{K} MV")


def test_gemv_large_b_takes_more_splits(dev):
    # B of 128 MiB (mn-contiguous): more, shorter splits than the 64 MiB rule
    M, N, K = 2, 4100, 8192
    a = oracle.uniform((M, K), 81)
    b = oracle.uniform((K, N), 82)
    c, cfg = gemm(g(a, dev), g(b, dev))
    assert cfg.startswith("sk gemv_mv "), cfg
    assert int(cfg.split("split=")[1].split()[0]) > 64, cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), "large-B GEMV")


@pytest.mark.parametrize("M,N,K", [
    (1, 4096, 4096), (1, 1000, 2048), (2, 17, 64), (3, 333, 1028), (4, 4096, 512),
    (6, 1, 12000),
])
def test_gemv_transposed_b(dev, M, N, K):
    # B = Bt.T: k-contiguous (the Linear layer's x·Wᵀ); up to 4 rows (more keep
    # the MFMA kernels: test_gemv_kv_rows_past_4_keep_mfma)
    a = oracle.uniform((M, K), 300 + M)
    bt = oracle.uniform((N, K), 400 + N)
    c, cfg = gemm(g(a, dev), g(bt, dev).t())
    assert cfg.startswith("sk gemv_kv ") or (N == 1 and cfg.startswith("sk gemv")), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, bt.T), K, amax(a), amax(bt), f"{M}x{N}x{K} KV")


@pytest.mark.parametrize("M,N,K,a_t", [
    (4096, 1, 4096, False),   # matrix x vector, A row-major: k-contiguous streamed operand
    (1000, 3, 2048, False),
    (4096, 1, 4096, True),    # A as a transpose view: mn-contiguous
    (520, 8, 300, True),
])
def test_gemv_few_columns(dev, M, N, K, a_t):
    a = oracle.uniform((M, K), 500 + M)
    b = oracle.uniform((K, N), 600 + N)
    A = g(a.T.copy(), dev).t() if a_t else g(a, dev)
    c, cfg = gemm(A, g(b, dev))
    assert cfg.startswith("sk gemv_mv_t " if a_t else "sk gemv_kv_t "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), f"{M}x{N}x{K} T")


@pytest.mark.parametrize("M,N,K,auto", [
    (4096, 4096, 1, True),   # the reference's outer product row: the cost model's pick
    (4096, 4096, 4, True), (2048, 2048, 2, True),
    # smaller outputs or larger K run the MFMA kernels unless forced
    (17, 256, 1, False), (1, 300, 2, False), (100, 1024, 3, False), (33, 2000, 4, False),
    (64, 1028, 5, False), (129, 256, 16, False), (3, 4097, 9, False), (2048, 2048, 16, False),
])
def test_rank_k(dev, M, N, K, auto):
    a = oracle.uniform((M, K), 700 + K)
    b = oracle.uniform((K, N), 800 + N)
    if auto:
        c, cfg = gemm(g(a, dev), g(b, dev))
    else:
        with mt.forced_config(mt.FAMILY_SKINNY, 1, 1):
            c, cfg = gemm(g(a, dev), g(b, dev))
    assert cfg.startswith("sk rankk "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), f"{M}x{N}x{K} rank-k")


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 4), (256, 8192, 1), (4096, 4096, 8), (512, 1024, 2)])
def test_rank_k_left_to_mfma_where_slower(dev, M, N, K):
    # measured faster on the MFMA kernels (K >= 8, or outputs under 2^22 /
    # 2^24 elements at K <= 2 / K <= 4)
    a = oracle.uniform((M, K), 710 + K)
    b = oracle.uniform((K, N), 810 + N)
    c, cfg = gemm(g(a, dev), g(b, dev))
    assert not cfg.startswith("sk "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), f"{M}x{N}x{K} mfma")


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 1), (2048, 2048, 2), (2050, 2048, 1)])
def test_rank_k_column_bias(dev, M, N, K):
    # the 16-byte fast path with a per-column bias (and a partial last row block)
    a = oracle.uniform((M, K), 720 + K)
    b = oracle.uniform((K, N), 820 + N)
    bias = oracle.uniform((N,), 821)
    c, cfg = gemm(g(a, dev), g(b, dev), bias=g(bias, dev), bias_axis=mt.BIAS_COL)
    assert cfg.startswith("sk rankk "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b) + bias[None, :], K, amax(a), amax(b),
                 f"{M}x{N}x{K} rank-k + column bias", extra=1e-6 * 4)


def test_rank_k_views_bias_beta(dev):
    # A and B as transpose views, C a strided window, per-row bias and beta = 1
    M, N, K = 300, 700, 7
    a = oracle.uniform((K, M), 11).T
    b = oracle.uniform((N, K), 12).T
    bias = oracle.uniform((M,), 13)
    base = oracle.uniform((M + 2, N + 9), 14)
    C = g(base, dev)
    win = C[1:M + 1, 3:N + 3]
    with mt.forced_config(mt.FAMILY_SKINNY, 1, 1):
        _, cfg = gemm(g(np.ascontiguousarray(a.T), dev).t(), g(np.ascontiguousarray(b.T), dev).t(),
                      out=win, bias=g(bias, dev), bias_axis=mt.BIAS_ROW, beta=1.0)
    assert cfg.startswith("sk rankk "), cfg
    got = C.cpu().numpy()
    want = base.copy()
    want[1:M + 1, 3:N + 3] = oracle.matmul(a, b) + bias[:, None] + base[1:M + 1, 3:N + 3]
    assert_close(got, want, K, amax(a), amax(b), "rank-k views+bias+beta", extra=1e-6 * 4)
    outside = np.ones_like(base, dtype=bool)
    outside[1:M + 1, 3:N + 3] = False
    assert np.array_equal(got[outside], base[outside])


@pytest.mark.parametrize("kv", [False, True])
def test_gemv_bias_beta_batch(dev, kv):
    # batched GEMV with a shared B, bias per column, beta = 0.5
    nb, M, N, K = 3, 2, 516, 1536
    a = oracle.uniform((nb, M, K), 21)
    b = oracle.uniform((K, N), 22)
    bias = oracle.uniform((N,), 23)
    c0 = oracle.uniform((nb, M, N), 24)
    B = g(b.T.copy(), dev).t() if kv else g(b, dev)
    C = g(c0, dev)
    gemm(g(a, dev), B.unsqueeze(0).expand(nb, K, N), out=C, bias=g(bias, dev),
         bias_axis=mt.BIAS_COL, beta=0.5)
    want = np.stack([oracle.matmul(a[i], b) for i in range(nb)]) + bias[None, None, :] + 0.5 * c0
    assert_close(C.cpu().numpy(), want, K, amax(a), amax(b), f"batched GEMV kv={kv}",
                 extra=1e-6 * 4)


@pytest.mark.parametrize("kv", [False, True])
@pytest.mark.parametrize("splits", [1, 2, 7, 64])
def test_gemv_forced_splits_deterministic(dev, kv, splits):
    M, N, K = 3, 1024, 4096
    a = oracle.uniform((M, K), 31)
    b = oracle.uniform((K, N), 32)
    B = g(b.T.copy(), dev).t() if kv else g(b, dev)
    A = g(a, dev)
    with mt.forced_config(mt.FAMILY_SKINNY, 0, splits):
        c1, cfg = gemm(A, B)
        c2, _ = gemm(A, B)
    assert cfg.startswith("sk gemv_kv " if kv else "sk gemv_mv "), cfg
    assert f"split={splits} " in cfg + " ", cfg
    assert torch.equal(c1, c2)
    assert_close(c1.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b),
                 f"forced splits {splits} kv={kv}")


def test_gemv_small_workspace_runs_unsplit(dev):
    M, N, K = 1, 4096, 4096
    a = oracle.uniform((M, K), 41)
    b = oracle.uniform((K, N), 42)
    A, B = g(a, dev), g(b, dev)
    C = torch.empty(M, N, device=dev)
    lib = mt.lib()
    assert lib.mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)) > 0
    gemm(A, B, out=C, ws=torch.empty(16, dtype=torch.uint8, device=dev))
    assert "split=1 " in mt.last_config() + " "
    assert_close(C.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), "unsplit GEMV")


def test_forced_mfma_family_keeps_skinny_shapes_off(dev):
    a = oracle.uniform((1, 512), 51)
    b = oracle.uniform((512, 512), 52)
    with mt.forced_config(mt.FAMILY_DL, 2, 1):
        c, cfg = gemm(g(a, dev), g(b, dev))
    assert cfg.startswith("dl "), cfg
    assert_close(c.cpu().numpy(), oracle.matmul(a, b), 512, 1, 1, "forced dl on a GEMV")


def test_special_values(dev):
    # IEEE specials reach the same entries as in the oracle; signed zeros agree
    M, N, K = 2, 256, 64
    a = oracle.uniform((M, K), 61)
    b = oracle.uniform((K, N), 62)
    a[0, 3] = np.inf
    b[5, 7] = np.nan
    b[9, 100:104] = 0.0
    a[1, :] = 0.0
    a[1, 0] = -0.0
    c, _ = gemm(g(a, dev), g(b, dev))
    got, want = c.cpu().numpy(), oracle.matmul(a, b)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.signbit(got[fin & (want == 0)]), np.signbit(want[fin & (want == 0)]))
    # rank-k: an outer product with a signed zero
    a1 = np.array([[-0.0], [2.0]], np.float32)
    b1 = np.full((1, 256), 3.0, np.float32)
    with mt.forced_config(mt.FAMILY_SKINNY, 1, 1):
        c1, cfg = gemm(g(a1, dev), g(b1, dev))
    assert cfg.startswith("sk rankk"), cfg
    np.testing.assert_array_equal(c1.cpu().numpy(), oracle.matmul(a1, b1))
    assert not np.any(np.signbit(c1.cpu().numpy()))


def test_benchmark_63_rows_keeps_mfma(dev):
    # 63x4096·4096x4096: 63 rows are past the GEMV kernels; sampled rows in fp64
    M, N, K = 63, 4096, 4096
    a = oracle.uniform((M, K), 71)
    b = oracle.uniform((K, N), 72)
    c, cfg = gemm(g(a, dev), g(b, dev))
    assert not cfg.startswith("sk "), cfg
    rows = [0, 17, 62]
    want = oracle.matmul_f64_rows(a, b, rows)
    assert_close(c.cpu().numpy()[rows], want, K, 1, 1, "63x4096x4096 sampled rows")


def test_gemv_kv_rows_past_4_keep_mfma(dev):
    # 6 and 8 rows against a k-contiguous B run faster on the MFMA kernels; the
    # 8-row GEMV kernel is still reached through the forced configuration
    for M in (6, 8):
        a = oracle.uniform((M, 1024), 90 + M)
        bt = oracle.uniform((512, 1024), 91)
        A, B = g(a, dev), g(bt, dev).t()
        c, cfg = gemm(A, B)
        assert not cfg.startswith("sk "), cfg
        want = oracle.matmul(a, bt.T)
        assert_close(c.cpu().numpy(), want, 1024, amax(a), amax(bt), f"{M} rows KV auto")
        with mt.forced_config(mt.FAMILY_SKINNY, 0, 4):
            c, cfg = gemm(A, B)
        assert cfg.startswith("sk gemv_kv rows=8 "), cfg
        assert_close(c.cpu().numpy(), want, 1024, amax(a), amax(bt), f"{M} rows KV forced")
