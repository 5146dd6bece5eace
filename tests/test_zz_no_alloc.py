"""mt_gemm_noalloc_f32 -- the GEMM entry point that allocates nothing -- against
mt_gemm_f32 with a workspace, through the C ABI.

Its split-K partials live in the library's static per-GPU buffer instead of a
caller workspace; the plan is the one mt_gemm_f32 picks, so the results must
agree bit for bit, and both must meet the parity bound against the CPU oracle
(the reference's matmul_cpu restated, include/TensorOps.hpp:139-160;
1e-5·√K·max|A|·max|B|).  Two calls in a row, the second smaller, share that
buffer; a problem needing more scratch than it holds is rejected without a
launch; a captured HIP graph of the call replays like the eager call.
"""
import ctypes

import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def noalloc(A, B, C, ep=None, stream=None):
    s = (stream or torch.cuda.current_stream()).cuda_stream
    return mt.lib().mt_gemm_noalloc_f32(mt.mat(A), mt.mat(B), mt.mat(C),
                                        ctypes.byref(ep) if ep is not None else None, s)


def with_workspace(A, B, C, ep=None):
    ma, mb, mc = mt.mat(A), mt.mat(B), mt.mat(C)
    n = mt.lib().mt_gemm_workspace_f32(ma, mb, mc)
    ws = mt.workspace(n, A.device)
    rc = mt.lib().mt_gemm_f32(ma, mb, mc, ctypes.byref(ep) if ep is not None else None,
                              ws.data_ptr() if ws is not None else None, n,
                              torch.cuda.current_stream().cuda_stream)
    return rc, n


def test_two_calls_in_a_row_match_the_workspace_entry_point(dev):
    # split-K plans, so the static buffer is used; the second call is smaller
    # and leaves most of the first call's partials behind in the buffer
    cases = [((128, 96, 8192), 1, True), ((64, 64, 4096), 2, False)]
    for (M, N, K), seed, bias in cases:
        a = oracle.uniform((M, K), 10 + seed)
        b = oracle.uniform((K, N), 20 + seed)
        bv = oracle.uniform((N,), 30 + seed)
        A, B, Bias = g(a, dev), g(b, dev), g(bv, dev)
        ep = mt.EpilogueF32(Bias.data_ptr(), 1, mt.BIAS_COL, 0.0) if bias else None
        C_ref = torch.full((M, N), 3.0, device=dev)
        C_na = torch.full((M, N), -3.0, device=dev)
        rc, n = with_workspace(A, B, C_ref, ep)
        assert rc == mt.MT_OK
        ref_cfg = mt.last_config()
        assert 0 < n <= mt.NOALLOC_SCRATCH_BYTES
        assert noalloc(A, B, C_na, ep) == mt.MT_OK
        cfg = mt.last_config()
        print(f"[noalloc] {M}x{N}x{K}: {cfg} (workspace path: {ref_cfg})", flush=True)
        assert cfg == ref_cfg and "split=1 " not in cfg + " ", cfg
        torch.cuda.synchronize()
        got, want = C_na.cpu().numpy(), C_ref.cpu().numpy()
        assert np.array_equal(got, want), f"{M}x{N}x{K}: differs from mt_gemm_f32"
        exp = oracle.matmul(a, b).astype(np.float64) + (bv if bias else 0.0)
        assert_close(got, exp, K, amax(a), amax(b), f"noalloc {M}x{N}x{K}", extra=1e-6)


def test_gemv_split_partials_in_the_static_buffer(dev):
    """The vector-ALU GEMV's split-K partials also go to the static buffer:
    two calls in a row (the second smaller), each equal to mt_gemm_f32."""
    for (M, N, K), seed in (((1, 4096, 4096), 3), ((3, 1024, 2048), 4)):
        a = oracle.uniform((M, K), 10 + seed)
        b = oracle.uniform((K, N), 20 + seed)
        A, B = g(a, dev), g(b, dev)
        C_ref = torch.full((M, N), 3.0, device=dev)
        C_na = torch.full((M, N), -3.0, device=dev)
        rc, n = with_workspace(A, B, C_ref)
        assert rc == mt.MT_OK
        ref_cfg = mt.last_config()
        assert 0 < n <= mt.NOALLOC_SCRATCH_BYTES
        assert noalloc(A, B, C_na) == mt.MT_OK
        cfg = mt.last_config()
        print(f"[noalloc] {M}x{N}x{K}: {cfg} (workspace path: {ref_cfg})", flush=True)
        assert cfg == ref_cfg and cfg.startswith("sk gemv") and "split=1 " not in cfg + " ", cfg
        torch.cuda.synchronize()
        got, want = C_na.cpu().numpy(), C_ref.cpu().numpy()
        assert np.array_equal(got, want), f"{M}x{N}x{K}: differs from mt_gemm_f32"
        assert_close(got, oracle.matmul(a, b), K, amax(a), amax(b), f"noalloc GEMV {M}x{N}x{K}")


def test_plan_without_split_k(dev):
    """Config 1's shape: its plan has no split-K (the wave-split kernel), so the
    buffer is not written, and the result still equals mt_gemm_f32's."""
    a, b = oracle.uniform((256, 512), 1), oracle.uniform((512, 512), 2)
    A, B = g(a, dev), g(b, dev)
    C_ref = torch.empty(256, 512, device=dev)
    C_na = torch.empty(256, 512, device=dev)
    assert with_workspace(A, B, C_ref)[0] == mt.MT_OK
    assert noalloc(A, B, C_na) == mt.MT_OK
    assert "split=1 " in mt.last_config() + " ", mt.last_config()
    torch.cuda.synchronize()
    assert torch.equal(C_na, C_ref)
    assert_close(C_na.cpu().numpy(), oracle.matmul(a, b), 512, amax(a), amax(b), "noalloc C1")


def test_too_much_scratch_is_rejected(dev):
    """16 forced K splits of 128x128 tiles over a 1024x1024 output need 64 MiB
    of partials: rejected with MT_ERR_SCRATCH_LIMIT, C untouched."""
    A = torch.ones(1024, 8192, device=dev)
    B = torch.ones(8192, 1024, device=dev)
    C = torch.full((1024, 1024), 5.0, device=dev)
    with mt.forced_config(mt.FAMILY_DL, 1, 16):
        assert mt.lib().mt_gemm_workspace_f32(mt.mat(A), mt.mat(B), mt.mat(C)) > \
            mt.NOALLOC_SCRATCH_BYTES
        assert noalloc(A, B, C) == mt.MT_ERR_SCRATCH_LIMIT
    assert b"MT_NOALLOC_SCRATCH_BYTES" in mt.lib().mt_strerror(mt.MT_ERR_SCRATCH_LIMIT)
    torch.cuda.synchronize()
    assert torch.all(C == 5.0)


def test_invalid_arguments_are_rejected(dev):
    A = torch.ones(8, 4, device=dev)
    B = torch.ones(5, 8, device=dev)     # inner dimensions differ
    C = torch.empty(8, 8, device=dev)
    assert noalloc(A, B, C) == mt.MT_ERR_INVALID


def test_graph_capture_replays(dev):
    """The call captured into a HIP graph (where allocation is not allowed)
    replays bit for bit like the eager call, input changes included."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    A = torch.rand(64, 8192, device=dev, generator=gen)
    B = torch.rand(8192, 64, device=dev, generator=gen)
    C = torch.empty(64, 64, device=dev)
    assert noalloc(A, B, C) == mt.MT_OK      # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = noalloc(A, B, C)
    assert rc == mt.MT_OK
    for rep in range(3):
        A.mul_(0.5).add_(0.25)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = C.clone()
        assert noalloc(A, B, C) == mt.MT_OK
        torch.cuda.synchronize()
        assert torch.equal(replayed, C), f"replay {rep} differs from the eager call"
