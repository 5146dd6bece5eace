"""Randomised Linear layers (F::linear and its backward) through the planner's picks.

The config-4 tests pin the benchmark shape, and the forced-configuration tests
pin one kernel at a time.  Here 32 seeded draws vary batch, in- and
out-features from 1 to ~1500 (tails everywhere; half the draws in multiples
of 4, which the direct-to-LDS kernels take; batches small and large, so that
the weight gradient's K = batch runs from one partial chunk to many and the
plan goes from the fused row sums to split-K with the column-sum kernel),
with and without a bias, and half of them accumulate into existing gradients
(beta = 1, as MatmulBackward does when a gradient already exists:
include/Autograd.hpp:117-147).  Y = X·Wᵀ + b, dX = dY·W, dW = dYᵀ·X and
db = Σ_rows dY must meet the GEMM parity bound against the oracle's
restatement of the reference's CPU matmul (include/TensorOps.hpp:139-189,
include/Module.hpp:92-114), whatever kernel the cost model picked (printed
per case).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

N_CASES = 32


def _dim(rng, big: int) -> int:
    r = rng.random()
    if r < 0.3:
        return int(rng.integers(1, 40))
    if r < 0.75:
        return int(rng.integers(40, 400))
    return int(rng.integers(400, big))


# batch x in x out at most 3e7, so that the oracle's four single-threaded
# GEMMs per case take about a second: the largest extent halves until it fits
MAX_WORK = 30_000_000

CASES = []
_rng = np.random.default_rng(20261202)
for _i in range(N_CASES):
    d = [_dim(_rng, 4200), _dim(_rng, 1500), _dim(_rng, 1300)]
    while d[0] * d[1] * d[2] > MAX_WORK:
        j = int(np.argmax(d))
        d[j] = (d[j] + 1) // 2
    # every other case with extents in multiples of 4, as layer sizes usually
    # are: 16-byte rows, so the direct-to-LDS kernels (and the fused row sums
    # of the weight gradient) take them; the rest take the gather layouts
    if _i % 2 == 0:
        d = [(e + 3) // 4 * 4 for e in d]
    CASES.append(dict(seed=1000 + 7 * _i, batch=d[0], fin=d[1], fout=d[2],
                      bias=bool(_rng.random() < 0.75), accumulate=bool(_rng.random() < 0.5)))


def g(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def sync_np(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("case", CASES, ids=[f"c{i}" for i in range(N_CASES)])
def test_random_linear_forward_backward(dev, case):
    s, B, fi, fo = case["seed"], case["batch"], case["fin"], case["fout"]
    print(f"[case] seed={s} batch={B} in={fi} out={fo} bias={case['bias']} "
          f"accumulate={case['accumulate']}", flush=True)
    x = oracle.normal((B, fi), s)
    w = oracle.normal((fo, fi), s + 1, std=(2.0 / fi) ** 0.5)
    b = oracle.normal((fo,), s + 2) if case["bias"] else None
    dy = oracle.normal((B, fo), s + 3, std=0.1)
    X, W, dY = g(x, dev), g(w, dev), g(dy, dev)

    y = mt.linear(X, W, g(b, dev) if b is not None else None)
    print(f"[config] fwd {mt.last_config()}", flush=True)
    assert_close(sync_np(y), oracle.linear(x, w, b), fi, amax(x), amax(w), "Y",
                 extra=1e-5 * (amax(b) if b is not None else 0.0))

    wdx, wdw, wdb = oracle.linear_backward(dy, x, w)
    if case["accumulate"]:
        # existing gradients G0 (beta = 1): the results are G0 + the new terms
        dw0 = oracle.normal((fo, fi), s + 4, std=0.1)
        db0 = oracle.normal((fo,), s + 5, std=0.1)
        dw, db = g(dw0, dev), g(db0, dev)
        _, dw, db = mt.linear_backward(dY, X, W, need_dx=False, dw=dw, db=db,
                                       beta_w=1.0, beta_b=1.0)
        print(f"[config] dW + db {mt.last_config()}", flush=True)
        assert_close(sync_np(dw), dw0.astype(np.float64) + wdw, B, amax(dy), amax(x),
                     "dW accumulated", extra=1e-6 * amax(dw0))
        assert_close(sync_np(db), db0.astype(np.float64) + wdb, B, amax(dy), 1.0,
                     "db accumulated", extra=1e-6 * amax(db0))
        dx, _, _ = mt.linear_backward(dY, X, W, need_dw=False, need_db=False)
        print(f"[config] dX {mt.last_config()}", flush=True)
    else:
        # one call for all three, as Linear's backward makes it
        dx, dw, db = mt.linear_backward(dY, X, W)
        print(f"[config] backward, last launch: {mt.last_config()}", flush=True)
        assert_close(sync_np(dw), wdw, B, amax(dy), amax(x), "dW")
        assert_close(sync_np(db), wdb, B, amax(dy), 1.0, "db")
    assert_close(sync_np(dx), wdx, fo, amax(dy), amax(w), "dX")


def test_random_linear_cases_reach_both_bias_gradient_forms():
    # the draw covers weight gradients with few rows (fused row sums) and with
    # many (split-K plans, where the column-sum kernel gives db)
    assert min(c["batch"] for c in CASES) < 40 and max(c["batch"] for c in CASES) > 1500
    assert sum(all(c[k] % 4 == 0 for k in ("batch", "fin", "fout")) for c in CASES) >= N_CASES // 2
    assert any(c["accumulate"] for c in CASES) and not all(c["accumulate"] for c in CASES)
