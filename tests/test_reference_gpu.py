"""The reference's own GPU matmul on this MI355X, beside this build's.

oracle/_ref/libref_gpu.so is the reference's src/gpu_ops.cpp compiled
unchanged for gfx950 (oracle/Makefile, target ref_gpu), driven through its
public launchers: matmul_gpu -> sgemm_kernel_v2 (src/gpu_ops.cpp:932-1144) for
contiguous operands and matmul_gpu_strided -> matmul_kernel_strided (909-930,
1199-1223) for the transposed view of config 3.  Each test checks the
reference kernel's result against the CPU oracle (so the comparison is with a
working reference), times both implementations the same way (warm-up, then
back-to-back calls between HIP events, as test/benchmark.cpp:162-190), and
prints one summary line.  Skipped where the reference tree was absent at build
time.
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not oracle.ref_gpu_available(),
                                 reason="oracle/_ref/libref_gpu.so not built (no reference tree)")]


def time_ours(fn, warmup, reps):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def report(name, M, N, K, ref_ms, our_ms):
    fl = 2.0 * M * N * K
    print(f"[reference-vs-build] {name}: reference {ref_ms * 1e3:.1f} us "
          f"({fl / ref_ms / 1e9:.2f} TFLOP/s), this build {our_ms * 1e3:.1f} us "
          f"({fl / our_ms / 1e9:.2f} TFLOP/s), speed-up {ref_ms / our_ms:.1f}x", flush=True)


@pytest.mark.parametrize("name,M,N,K", [("config 2 (4096^3)", 4096, 4096, 4096),
                                        ("config 1 (256x512x512)", 256, 512, 512)])
def test_reference_contiguous_matmul(dev, name, M, N, K):
    a = oracle.uniform((M, K), 42)
    b = oracle.uniform((K, N), 43)
    ref_c, ref_ms = oracle.ref_gpu_matmul(a, b, which=0, warmup=2, reps=5 if M > 1024 else 50)
    rows = [0, 1, M // 3, M // 2, M - 1]
    want = oracle.matmul_f64_rows(a, b, rows)
    assert_close(ref_c[rows], want, K, amax(a), amax(b), f"reference v2 kernel {name}")
    A, B = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    C = torch.empty(M, N, device=dev)
    ws = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)), dev)
    our_ms = time_ours(lambda: mt.gemm(A, B, out=C, ws=ws), 3, 20 if M > 1024 else 200)
    assert_close(C.cpu().numpy()[rows], want, K, amax(a), amax(b), f"this build {name}")
    report(name, M, N, K, ref_ms, our_ms)


def test_reference_transposed_view_matmul(dev):
    # config 3: C = A · Bᵀ with B [2048,1024] read through its transpose view
    M = N = 2048
    K = 1024
    a = oracle.normal((M, K), 42)
    bt = oracle.normal((N, K), 43)
    ref_c, ref_ms = oracle.ref_gpu_matmul(a, bt, which=1, warmup=1, reps=3)
    rows = [0, 7, 1000, M - 1]
    want = oracle.matmul_f64_rows(a, np.ascontiguousarray(bt.T), rows)
    assert_close(ref_c[rows], want, K, amax(a), amax(bt), "reference strided kernel config 3")
    A, Bt = torch.from_numpy(a).to(dev), torch.from_numpy(bt).to(dev)
    C = torch.empty(M, N, device=dev)
    ws = mt.workspace(mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(Bt.t()), mt.mat(C)), dev)
    our_ms = time_ours(lambda: mt.gemm(A, Bt.t(), out=C, ws=ws), 3, 50)
    assert_close(C.cpu().numpy()[rows], want, K, amax(a), amax(bt), "this build config 3")
    report("config 3 (2048x2048x1024, Bᵀ view)", M, N, K, ref_ms, our_ms)
