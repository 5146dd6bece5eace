"""Concurrent callers: the C ABI keeps no shared mutable state beyond
per-thread caches (plans, the forced configuration, the last-config string)
and an atomic per-device CU count, so GEMMs launched from several host
threads, each on its own stream, give bit-for-bit the results of the same
calls made one after another -- the reference's launchers are likewise
stateless apart from MemoryPool, which it locks (include/MemoryPool.hpp:26-71)."""
import threading

import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(256, 512, 512, 1), (300, 200, 76, 1), (64, 64, 4096, 1), (512, 512, 64, 8),
          (1000, 520, 256, 1)]


def inputs(dev):
    out = []
    for i, (M, N, K, b) in enumerate(SHAPES):
        a = torch.from_numpy(oracle.uniform((b, M, K) if b > 1 else (M, K), 10 + i)).to(dev)
        w = torch.from_numpy(oracle.uniform((b, K, N) if b > 1 else (K, N), 20 + i)).to(dev)
        out.append((a, w))
    return out


def run_all(pairs, stream):
    with torch.cuda.stream(stream):
        res = [mt.gemm(a, w, stream=stream) for a, w in pairs]
    stream.synchronize()
    return [r.cpu().numpy() for r in res]


def test_concurrent_threads_match_serial(dev):
    pairs = inputs(dev)
    want = run_all(pairs, torch.cuda.Stream())
    got, errors = {}, []

    def worker(t):
        try:
            s = torch.cuda.Stream()
            outs = []
            for _ in range(5):
                outs = run_all(pairs, s)
            got[t] = outs
        except Exception as e:   # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t in range(4):
        for i, (g, w) in enumerate(zip(got[t], want)):
            assert np.array_equal(g, w), f"thread {t} shape {SHAPES[i]}"


def test_forced_config_is_per_thread(dev):
    a = torch.from_numpy(oracle.uniform((300, 200), 1)).to(dev)
    b = torch.from_numpy(oracle.uniform((200, 260), 2)).to(dev)
    seen = {}
    ready, go = threading.Barrier(2), threading.Event()

    def forced():
        with mt.forced_config(mt.FAMILY_RS, 1, 1):
            ready.wait()
            go.wait()
            mt.gemm(a, b)
            seen["forced"] = mt.last_config()

    def auto():
        ready.wait()
        mt.gemm(a, b)
        seen["auto"] = mt.last_config()
        go.set()

    threads = [threading.Thread(target=forced), threading.Thread(target=auto)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    print(seen)
    assert seen["forced"].startswith("rs 128x128") and seen["forced"].endswith("cfg=1")
    assert not seen["auto"].startswith("rs "), seen["auto"]


def test_explicit_stream_without_context(dev):
    """stream= without a `with torch.cuda.stream(...)` block: the workspace and
    the output the call allocates belong to that stream, so work queued on
    the current stream right after the call cannot be handed the workspace
    while the split-K kernels still use it."""
    a = oracle.uniform((300, 1000), 31)
    b = oracle.uniform((1000, 260), 32)
    A = torch.from_numpy(a).to(dev)
    B = torch.from_numpy(b).to(dev)
    torch.cuda.synchronize()
    want = oracle.matmul(a, b)
    s = torch.cuda.Stream()
    outs = []
    for _ in range(4):
        with mt.forced_config(mt.FAMILY_DL, 2, 8):   # 64x64 tiles, 8 K splits: partials
            outs.append(mt.gemm(A, B, stream=s))
        assert "split=8" in mt.last_config(), mt.last_config()
        # allocations and writes on the current stream, while s may still run
        junk = [torch.full((1 << 18,), 7.0, device=dev) for _ in range(16)]
        del junk
    s.synchronize()
    torch.cuda.synchronize()
    for C in outs:
        got = C.cpu().numpy()
        err = float(np.max(np.abs(got.astype(np.float64) - want)))
        assert err <= oracle.tolerance(1000, 1.0, 1.0), err
