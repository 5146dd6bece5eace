"""The wave-split kernels (K split across the waves of one workgroup, on
32x32 or 16x16 MFMA blocks) against the CPU oracle, every configuration
forced through mt_gemm_force_config.

It takes every operand layout (16-byte fragment loads for k-contiguous
operands, scalar loads for the rest), K ranges with a partial last chunk,
fewer chunks than waves, batches with a shared operand, the fused bias/beta
epilogue, scattered and sliced outputs, and split-K across workgroups on top
of the split across waves.  Oracle: the reference's matmul_cpu /
matmul_cpu_strided restated in oracle/oracle.c (include/TensorOps.hpp:139-189);
bound 1e-5·√K·max|A|·max|B| (tests/util_parity.py).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

KSW = list(range(9))   # 0-3: 32x32 MFMA blocks, 4-8: 16x16 blocks


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def operand(a, layout, dev):
    """row: row-major; col: a transposed view of column-major storage;
    strided: every second column of a wider row-major buffer (no unit stride)."""
    if layout == "row":
        return g(a, dev)
    if layout == "col":
        return g(np.ascontiguousarray(a.T), dev).t()
    wide = np.zeros((a.shape[0], 2 * a.shape[1]), np.float32)
    wide[:, ::2] = a
    return g(wide, dev)[:, ::2]


def run(dev, cfg, M, N, K, la="row", lb="row", splits=1, seed=0, what=""):
    a = oracle.uniform((M, K), 300 + seed)
    b = oracle.uniform((K, N), 400 + seed)
    A, B = operand(a, la, dev), operand(b, lb, dev)
    with mt.forced_config(mt.FAMILY_KSW, cfg, splits):
        C = mt.gemm(A, B)
        name = mt.last_config()
    print(f"[config] {name}", flush=True)
    assert name.startswith("ksw ") and name.endswith(f" cfg={cfg}"), name
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b),
                 f"ksw{cfg} {M}x{N}x{K} a={la} b={lb} split={splits} {what}")
    return name


@pytest.mark.parametrize("cfg", KSW)
@pytest.mark.parametrize("la", ["row", "col", "strided"])
@pytest.mark.parametrize("lb", ["row", "col", "strided"])
def test_layouts_and_tails(dev, cfg, la, lb):
    # M, N tails on every tile shape; K = 16*37 + 12: a partial chunk, and 37
    # whole chunks spread unevenly over the waves
    run(dev, cfg, 83, 70, 604, la, lb, seed=cfg)


@pytest.mark.parametrize("cfg", KSW)
@pytest.mark.parametrize("K", [1, 5, 16, 17, 48, 64, 100, 512, 2048])
def test_k_ranges(dev, cfg, K):
    """Fewer chunks than waves, a lone partial chunk, exact multiples."""
    run(dev, cfg, 64, 96, K, "row", "col" if K % 4 == 0 else "row", seed=K)


@pytest.mark.parametrize("cfg", KSW)
@pytest.mark.parametrize("splits", [2, 3, 5])
def test_split_k_on_top(dev, cfg, splits):
    name = run(dev, cfg, 96, 128, 1000, "row", "row", splits=splits, seed=splits)
    assert f"split={splits} " in name


@pytest.mark.parametrize("cfg", KSW)
def test_batched_bias_beta_sliced_output(dev, cfg):
    Bn, M, N, K = 3, 70, 66, 300
    a = oracle.uniform((Bn, M, K), 1)
    w = oracle.uniform((K, N), 2)
    bias = oracle.uniform((N,), 3)
    c0 = oracle.uniform((Bn, M, N + 5), 4)
    A = g(a, dev)
    Wb = g(w, dev).unsqueeze(0).expand(Bn, K, N)          # shared operand, batch stride 0
    big = g(c0, dev)
    C = big[:, :, 2:2 + N]                                  # strided, unaligned output
    with mt.forced_config(mt.FAMILY_KSW, cfg, 1):
        mt.gemm(A, Wb, out=C, bias=g(bias, dev), bias_axis=mt.BIAS_COL, beta=0.5)
        name = mt.last_config()
    assert name.startswith("ksw "), name
    torch.cuda.synchronize()
    got = big.cpu().numpy()
    want = np.stack([oracle.matmul(a[i], w) for i in range(Bn)]).astype(np.float64)
    want = want + bias + 0.5 * c0[:, :, 2:2 + N]
    assert_close(got[:, :, 2:2 + N], want, K, amax(a), amax(w), f"ksw{cfg} batched", extra=1e-5)
    # nothing outside the output view was written
    assert np.array_equal(got[:, :, :2], c0[:, :, :2])
    assert np.array_equal(got[:, :, 2 + N:], c0[:, :, 2 + N:])


@pytest.mark.parametrize("cfg", KSW)
def test_deterministic(dev, cfg):
    a = oracle.uniform((256, 2048), 7)
    b = oracle.uniform((2048, 200), 8)
    A, B = g(a, dev), g(b, dev)
    with mt.forced_config(mt.FAMILY_KSW, cfg, 1):
        c1 = mt.gemm(A, B).cpu().numpy()
        c2 = mt.gemm(A, B).cpu().numpy()
    assert np.array_equal(c1, c2)
