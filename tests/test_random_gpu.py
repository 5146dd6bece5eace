"""Randomised GEMMs through the cost model's own plans, against the CPU oracle.

The other parity tests pin one kernel path at a time.  Here 64 seeded
draws mix everything a caller can hand over at once: sizes from 1 to ~2000
in each dimension (tails everywhere, K from 1 to ~3000), row-major operands,
transpose views, row slices with an offset, doubly strided views, outputs
that are fresh or a column window of a wider buffer, a fused bias on either
axis and beta*C accumulation.  Whatever configuration and split the planner
picks (printed per case), the result must meet the GEMM parity bound
1e-5*sqrt(K)*max|A|*max|B| against the reference's matmul_cpu restated in
oracle/oracle.c (include/TensorOps.hpp:139-189), on every row for small
cases and on sampled rows (fp64) for large ones.
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

N_CASES = 64


def _dim(rng) -> int:
    r = rng.random()
    if r < 0.35:
        return int(rng.integers(1, 80))
    if r < 0.8:
        return int(rng.integers(80, 700))
    return int(rng.integers(700, 2100))


def _operand(a: np.ndarray, kind: str, rng, dev) -> torch.Tensor:
    """The logical matrix `a` on the GPU in the storage form `kind`."""
    rows, cols = a.shape
    if kind == "row":
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if kind == "col":                      # transpose view of column-major storage
        return torch.from_numpy(np.ascontiguousarray(a.T)).to(dev).t()
    if kind == "slice":                    # rows [off, off+rows) of a taller matrix
        off = int(rng.integers(1, 9))
        big = np.zeros((rows + off + 3, cols), np.float32)
        big[off:off + rows] = a
        return torch.from_numpy(big).to(dev)[off:off + rows]
    # "strided": every second column of a wider matrix (a gather layout)
    big = np.zeros((rows, 2 * cols), np.float32)
    big[:, ::2] = a
    return torch.from_numpy(big).to(dev)[:, ::2]


def _round4(x: int) -> int:
    return (x + 3) // 4 * 4


CASES = []
_rng = np.random.default_rng(20261201)
for _i in range(N_CASES):
    # every second case has dimensions that are multiples of 4, so that
    # row-major and transposed operands are 16-byte vector layouts (the
    # direct-to-LDS kernels); the others mostly take the gather kernel
    _r = _round4 if _i % 2 else (lambda x: x)
    CASES.append(dict(
        M=_r(_dim(_rng)), N=_r(_dim(_rng)),
        K=_r(int(_rng.integers(1, 3000)) if _rng.random() < 0.9 else _dim(_rng)),
        la=str(_rng.choice(["row", "col", "slice", "strided"], p=[0.4, 0.3, 0.2, 0.1])),
        lb=str(_rng.choice(["row", "col", "slice", "strided"], p=[0.4, 0.3, 0.2, 0.1])),
        out=str(_rng.choice(["fresh", "window"])),
        bias=str(_rng.choice(["none", "row", "col"])),
        beta=float(_rng.choice([0.0, 0.0, 0.5, -1.0])),
        seed=1000 + _i))


@pytest.mark.parametrize("case", CASES, ids=[f"r{i}" for i in range(N_CASES)])
def test_random_gemm_auto_plan(dev, case):
    M, N, K = case["M"], case["N"], case["K"]
    rng = np.random.default_rng(case["seed"])
    a = oracle.uniform((M, K), case["seed"])
    b = oracle.uniform((K, N), case["seed"] + 1)
    A = _operand(a, case["la"], rng, dev)
    B = _operand(b, case["lb"], rng, dev)
    c0 = oracle.uniform((M, N), case["seed"] + 2)
    if case["out"] == "window":
        lead = int(rng.integers(1, 6))
        wide = torch.zeros(M, N + lead + 2, device=dev)
        C = wide[:, lead:lead + N]
    else:
        wide, lead = None, 0
        C = torch.empty(M, N, device=dev)
    beta = case["beta"]
    if beta != 0.0:
        C.copy_(torch.from_numpy(c0).to(dev))
    kw = {}
    bias = None
    if case["bias"] != "none":
        bias = oracle.uniform((M if case["bias"] == "row" else N,), case["seed"] + 3)
        kw = dict(bias=torch.from_numpy(bias).to(dev),
                  bias_axis=mt.BIAS_ROW if case["bias"] == "row" else mt.BIAS_COL)
    mt.gemm(A, B, out=C, beta=beta, **kw)
    torch.cuda.synchronize()
    print(f"[case] {case} -> {mt.last_config()}", flush=True)
    got = C.cpu().numpy()

    small = M * N * K <= 40_000_000
    rows = np.arange(M) if small else np.unique(np.r_[0, M - 1, rng.integers(0, M, 12)])
    want = oracle.matmul(a, b) if small else oracle.matmul_f64_rows(a, b, rows)
    want = np.asarray(want, np.float64)[rows] if small else np.asarray(want, np.float64)
    if bias is not None:
        want = want + (bias[rows, None] if case["bias"] == "row" else bias[None, :])
    if beta != 0.0:
        want = want + beta * c0[rows]
    extra = 2e-6 * (1.0 + abs(beta)) if (bias is not None or beta != 0.0) else 0.0
    assert_close(got[rows], want, K, amax(a), amax(b),
                 f"random {M}x{N}x{K} a={case['la']} b={case['lb']}", extra=extra)
    if wide is not None:
        w = wide.cpu().numpy()
        assert not w[:, :lead].any() and not w[:, lead + N:].any(), "wrote outside the window"


# ---- batched ------------------------------------------------------------------
# 24 seeded batched GEMMs (the reference's bmm, include/TensorOps.hpp:933-991,
# restated as ora_bmm): batch 1-12, each operand dense, per-batch transposed
# (a permuted view), every second batch of a larger stack, or one matrix
# expanded over the batch (stride 0); the output fresh or every second batch
# of a larger stack, with a bias or beta*C now and then.

def _batched(a: np.ndarray, kind: str, dev) -> torch.Tensor:
    nb, rows, cols = a.shape
    if kind == "dense":
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if kind == "trans":
        return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1))).to(dev).permute(0, 2, 1)
    if kind == "step":
        big = np.zeros((2 * nb, rows, cols), np.float32)
        big[::2] = a
        return torch.from_numpy(big).to(dev)[::2]
    # "expand": every batch is a[0]
    return torch.from_numpy(np.ascontiguousarray(a[0])).to(dev).expand(nb, rows, cols)


BCASES = []
_brng = np.random.default_rng(20261203)
for _i in range(24):
    _r = _round4 if _i % 2 else (lambda x: x)
    _ka = str(_brng.choice(["dense", "trans", "step", "expand"], p=[0.4, 0.3, 0.15, 0.15]))
    _kb = str(_brng.choice(["dense", "trans", "step", "expand"], p=[0.4, 0.3, 0.15, 0.15]))
    if _ka == "expand" and _kb == "expand":
        _kb = "dense"
    BCASES.append(dict(batch=int(_brng.integers(1, 13)), M=_r(int(_brng.integers(1, 400))),
                       N=_r(int(_brng.integers(1, 400))), K=_r(int(_brng.integers(1, 700))),
                       la=_ka, lb=_kb, out=str(_brng.choice(["fresh", "step"])),
                       bias=str(_brng.choice(["none", "none", "row", "col"])),
                       beta=float(_brng.choice([0.0, 0.0, 0.5])), seed=3000 + 10 * _i))


@pytest.mark.parametrize("case", BCASES, ids=[f"b{i}" for i in range(len(BCASES))])
def test_random_batched_auto_plan(dev, case):
    nb, M, N, K = case["batch"], case["M"], case["N"], case["K"]
    a = oracle.uniform((nb, M, K), case["seed"])
    b = oracle.uniform((nb, K, N), case["seed"] + 1)
    if case["la"] == "expand":
        a = np.broadcast_to(a[:1], a.shape).copy()
    if case["lb"] == "expand":
        b = np.broadcast_to(b[:1], b.shape).copy()
    A, B = _batched(a, case["la"], dev), _batched(b, case["lb"], dev)
    c0 = oracle.uniform((nb, M, N), case["seed"] + 2)
    if case["out"] == "step":
        big = torch.zeros(2 * nb, M, N, device=dev)
        C = big[::2]
    else:
        big, C = None, torch.empty(nb, M, N, device=dev)
    beta = case["beta"]
    if beta != 0.0:
        C.copy_(torch.from_numpy(c0).to(dev))
    kw, bias = {}, None
    if case["bias"] != "none":
        bias = oracle.uniform((M if case["bias"] == "row" else N,), case["seed"] + 3)
        kw = dict(bias=torch.from_numpy(bias).to(dev),
                  bias_axis=mt.BIAS_ROW if case["bias"] == "row" else mt.BIAS_COL)
    mt.gemm(A, B, out=C, beta=beta, **kw)
    torch.cuda.synchronize()
    print(f"[case] {case} -> {mt.last_config()}", flush=True)
    want = oracle.bmm(a, b).astype(np.float64)
    if bias is not None:
        want = want + (bias[None, :, None] if case["bias"] == "row" else bias[None, None, :])
    if beta != 0.0:
        want = want + beta * c0
    extra = 2e-6 * (1.0 + abs(beta)) if (bias is not None or beta != 0.0) else 0.0
    assert_close(C.cpu().numpy(), want, K, amax(a), amax(b),
                 f"random bmm {nb}x{M}x{N}x{K} a={case['la']} b={case['lb']}", extra=extra)
    if big is not None:
        assert not big[1::2].cpu().numpy().any(), "wrote into the skipped batches"
