"""GPU parity of mt_gemm_f32 against the CPU oracle (the reference's matmul_cpu /
matmul_cpu_strided restated in oracle/oracle.c) on identical seeded inputs.

Bound: max|err| <= 1e-5·√K·max|A|·max|B| (tests/util_parity.py).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu


def to_gpu(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run(A: torch.Tensor, B: torch.Tensor, **kw) -> np.ndarray:
    C = mt.gemm(A, B, **kw)
    torch.cuda.synchronize()
    print(f"[config] {mt.last_config()}", flush=True)
    return C.cpu().numpy()


def test_known_answer_2x3x2(dev):
    # reference test/tensor_test.cpp:258-316 (CPU and GPU matmul)
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    c = run(to_gpu(a, dev), to_gpu(b, dev))
    np.testing.assert_array_equal(c, np.array([[58, 64], [139, 154]], np.float32))


def test_fill_2_and_3(dev):
    # reference test/engien_test.cpp:80-96: 2x3 of 2s times 3x2 of 3s = 18 everywhere
    c = run(torch.full((2, 3), 2.0, device=dev), torch.full((3, 2), 3.0, device=dev))
    np.testing.assert_array_equal(c, np.full((2, 2), 18.0, np.float32))


def test_config1_mlp_linear_shape(dev):
    # benchmark config 1: C[256,512] = A[256,512]·B[512,512], U(-1,1), seeds 42/43
    a = oracle.uniform((256, 512), 42)
    b = oracle.uniform((512, 512), 43)
    c = run(to_gpu(a, dev), to_gpu(b, dev))
    assert_close(c, oracle.matmul(a, b), 512, amax(a), amax(b), "C1 256x512x512")


@pytest.mark.parametrize("M,N,K", [
    (257, 511, 383),   # every tail at once (reference benchmark shape)
    (1, 4096, 4096),   # GEMV row
    (4096, 1, 4096),   # GEMV column
    (4096, 4096, 1),   # outer product (K = 1)
    (63, 4096, 64),
    (130, 70, 33),
    (5, 7, 3),
    (256, 256, 4099),  # K tail with split-K
    (64, 64, 8192),    # skinny output, deep K: split-K
])
def test_shapes_and_tails(dev, M, N, K):
    a = oracle.uniform((M, K), 7 + M)
    b = oracle.uniform((K, N), 11 + N)
    c = run(to_gpu(a, dev), to_gpu(b, dev))
    assert_close(c, oracle.matmul(a, b), K, amax(a), amax(b), f"{M}x{N}x{K}")


def test_k_zero_gives_zeros_and_bias(dev):
    # reference F6b: K = 0 must give zeros (the reference v2 kernel reads an
    # uninitialised LDS buffer); with a fused bias it gives the bias.
    A = torch.empty((33, 0), device=dev)
    B = torch.empty((0, 17), device=dev)
    c = run(A, B)
    np.testing.assert_array_equal(c, np.zeros((33, 17), np.float32))
    bias = torch.arange(17, dtype=torch.float32, device=dev)
    c = run(A, B, bias=bias, bias_axis=mt.BIAS_COL)
    np.testing.assert_array_equal(c, np.broadcast_to(np.arange(17, dtype=np.float32), (33, 17)))


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(300, 260, 200), (64, 96, 32), (512, 512, 512)])
def test_transpose_views(dev, ta, tb, M, N, K):
    # NN / NT / TN / TT through transpose views (strides swapped, not materialised),
    # as MatmulBackward hands them over (reference include/Autograd.hpp:124-142).
    a = oracle.normal((M, K), 42)
    b = oracle.normal((K, N), 43)
    A = to_gpu(a.T.copy(), dev).t() if ta else to_gpu(a, dev)
    B = to_gpu(b.T.copy(), dev).t() if tb else to_gpu(b, dev)
    assert A.is_contiguous() != ta and B.is_contiguous() != tb
    c = run(A, B)
    a_view = a.T.copy().T if ta else a
    b_view = b.T.copy().T if tb else b
    assert_close(c, oracle.matmul(a_view, b_view), K, amax(a), amax(b), f"ta={ta} tb={tb}")


def test_row_slice_offset(dev):
    # reference F1: a row slice is "contiguous" with offset != 0; the reference
    # GPU path drops the offset, this backend honours it.
    a = oracle.normal((300, 96), 42)
    b = oracle.normal((96, 130), 43)
    A = to_gpu(a, dev)[37:]
    assert A.storage_offset() == 37 * 96
    c = run(A, to_gpu(b, dev))
    assert_close(c, oracle.matmul(a[37:], b), 96, amax(a), amax(b), "slice rows 37:")


@pytest.mark.parametrize("off", [1, 2, 3])
def test_unaligned_offsets_take_scalar_path(dev, off):
    a = oracle.uniform((200 * 64 + 8,), 5)
    b = oracle.uniform((64 * 72 + 8,), 6)
    A = to_gpu(a, dev)[off:off + 200 * 64].view(200, 64)
    B = to_gpu(b, dev)[off:off + 64 * 72].view(64, 72)
    c = run(A, B)
    assert "ks" in mt.last_config() or "ms" in mt.last_config()
    av = a[off:off + 200 * 64].reshape(200, 64)
    bv = b[off:off + 64 * 72].reshape(64, 72)
    assert_close(c, oracle.matmul(av, bv), 64, amax(av), amax(bv), f"offset {off}")


def test_expand_stride_zero(dev):
    # expand views (stride 0, reference include/TensorImpl.hpp:204-228)
    row = oracle.uniform((1, 128), 3)
    col = oracle.uniform((96, 1), 4)
    A = to_gpu(row, dev).expand(80, 128)           # [80,128] strides (0,1)
    B = to_gpu(col, dev).expand(96, 128)           # [96,128] strides (1,0)
    assert A.stride() == (0, 1) and B.stride() == (1, 0)
    c = run(A[:, :96], B)
    av = np.broadcast_to(row, (80, 128))[:, :96]
    bv = np.broadcast_to(col, (96, 128))
    assert_close(c, oracle.matmul(av, bv), 96, amax(av), amax(bv), "expand")


def test_doubly_strided_views(dev):
    # every-other-column and every-third-row views: no unit stride anywhere
    a = oracle.normal((150, 200), 8)
    b = oracle.normal((300, 90), 9)
    A = to_gpu(a, dev)[::2, ::2]        # [75,100] strides (400,2)
    B = to_gpu(b, dev)[::3]             # [100,90] strides (270,1)
    Bs = B[:, ::2]                      # [100,45] strides (270,2)
    c = run(A, Bs)
    av, bv = a[::2, ::2], b[::3][:, ::2]
    assert_close(c, oracle.matmul(av, bv), 100, amax(av), amax(bv), "doubly strided")


@pytest.mark.parametrize("axis", [mt.BIAS_ROW, mt.BIAS_COL])
def test_bias_epilogue(dev, axis):
    a = oracle.uniform((200, 300), 1)
    b = oracle.uniform((300, 170), 2)
    bias = oracle.uniform((200 if axis == mt.BIAS_ROW else 170,), 3)
    c = run(to_gpu(a, dev), to_gpu(b, dev), bias=to_gpu(bias, dev), bias_axis=axis)
    want = oracle.matmul(a, b) + (bias[:, None] if axis == mt.BIAS_ROW else bias[None, :])
    assert_close(c, want, 300, amax(a), amax(b), f"bias axis {axis}", extra=1e-6)


def test_beta_accumulate(dev):
    a = oracle.uniform((128, 256), 1)
    b = oracle.uniform((256, 192), 2)
    c0 = oracle.uniform((128, 192), 3)
    C = to_gpu(c0, dev)
    mt.gemm(to_gpu(a, dev), to_gpu(b, dev), out=C, beta=1.0)
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), oracle.matmul(a, b) + c0, 256, amax(a), amax(b), "beta=1",
                 extra=1e-6)


def test_split_k_is_deterministic(dev):
    a = oracle.uniform((64, 8192), 21)
    b = oracle.uniform((8192, 64), 22)
    A, B = to_gpu(a, dev), to_gpu(b, dev)
    c1 = run(A, B)
    assert "split=1 " not in mt.last_config() + " "
    c2 = run(A, B)
    np.testing.assert_array_equal(c1, c2)


def test_batched_config5b(dev):
    # benchmark config 5b: [64]x[512,64]·[64,512], U(-1,1) seeds 42/43; one launch
    a = oracle.uniform((64, 512, 64), 42)
    b = oracle.uniform((64, 64, 512), 43)
    c = mt.bmm(to_gpu(a, dev), to_gpu(b, dev))
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), oracle.bmm(a, b), 64, amax(a), amax(b), "C5b bmm")


def test_batched_shared_weight(dev):
    # batch stride 0 on A: one weight for every batch entry (conv-style)
    a = oracle.uniform((1, 96, 80), 1)
    b = oracle.uniform((7, 80, 50), 2)
    A = to_gpu(a, dev).expand(7, 96, 80)
    c = mt.gemm(A, to_gpu(b, dev))
    torch.cuda.synchronize()
    assert_close(c.cpu().numpy(), oracle.bmm(np.broadcast_to(a, (7, 96, 80)), b), 80,
                 amax(a), amax(b), "shared A")


def test_config2_4096_properties(dev):
    # benchmark config 2 (4096^3): the full oracle would take minutes, so check
    # (1) 24 sampled rows against the oracle's fp64 brute force over the full K,
    # (2) the checksum identity C·1 = A·(B·1) in fp64 over all rows.
    a = oracle.uniform((4096, 4096), 42)
    b = oracle.uniform((4096, 4096), 43)
    C = mt.gemm(to_gpu(a, dev), to_gpu(b, dev))
    torch.cuda.synchronize()
    print(f"[config] {mt.last_config()}", flush=True)
    c = C.cpu().numpy()
    rows = np.linspace(0, 4095, 24).astype(np.int64)
    assert_close(c[rows], oracle.matmul_f64_rows(a, b, rows), 4096, amax(a), amax(b),
                 "C2 sampled rows")
    rowsum = c.astype(np.float64).sum(axis=1)
    want = a.astype(np.float64) @ b.astype(np.float64).sum(axis=1)
    err = np.max(np.abs(rowsum - want))
    bound = 4096 * 1e-5 * 64
    print(f"[parity] C2 checksum: max|err|={err:.3e} bound={bound:.3e}")
    assert err <= bound


def test_config3_transpose_and_slice_views(dev):
    # benchmark config 3: C = A·Bᵀ with B [2048,1024] passed as a transpose view,
    # and the slice A[128:] (offset 131072); N(0,1) seeds 42/43.  Sampled rows
    # against the oracle (full K).
    a = oracle.normal((2048, 1024), 42)
    b = oracle.normal((2048, 1024), 43)
    A, B = to_gpu(a, dev), to_gpu(b, dev)
    rows = np.array([0, 1, 127, 128, 129, 1000, 2047 - 128, 2047], np.int64)
    c = run(A, B.t())
    assert_close(c[rows], oracle.matmul_f64_rows(a, b.T, rows), 1024, amax(a), amax(b), "C3a")
    As = A[128:]
    assert As.storage_offset() == 131072
    c = run(As, B.t())
    r2 = rows[rows < 1920]
    assert_close(c[r2], oracle.matmul_f64_rows(a[128:], b.T, r2), 1024, amax(a), amax(b), "C3b")
    # the view result equals the result on materialised copies
    c_mat = run(As.contiguous(), B.t().contiguous())
    assert_close(c, c_mat, 1024, amax(a), amax(b), "C3b view == copy")


# ---- direct-to-LDS kernel (both operands in a 16-byte vector layout) ---------
# Tails in M and N (clamped rows), K not a multiple of 16 (bounds-checked last
# chunk), split-K over such a K, one-row/one-column operands, batch and the
# bias/beta epilogue, for all four (k- / mn-contiguous) layout pairs.

def _views(a, b, ta, tb, dev):
    A = to_gpu(a.T.copy(), dev).t() if ta else to_gpu(a, dev)
    B = to_gpu(b.T.copy(), dev).t() if tb else to_gpu(b, dev)
    return A, B


# Vector-layout operands go to the direct-to-LDS kernel or, for small output
# tile counts, to the wave-split kernel; the cost model picks.  Shapes with at
# most 8 rows or columns (4 against a k-contiguous operand), or K <= 16, go to
# the vector-ALU kernels ("sk",
# tests/test_skinny_gpu.py); the direct-to-LDS kernel is then also forced on
# them (configurations 2 and 5, the plain and the prefetching 64x64 tile),
# so that its one-row / one-column tails stay covered.  (Every configuration
# of both MFMA families is also forced on these layouts in
# test_configs_gpu.py and test_ksw_gpu.py.)
VECTOR_PATHS = ("dl ", "ksw ", "sk ")


def _also_forced_dl(A, B, want, K, am, bm, what):
    if not mt.last_config().startswith("sk "):
        return
    for cfg in (2, 5):
        with mt.forced_config(mt.FAMILY_DL, cfg, 1):
            c = run(A, B)
            assert mt.last_config().startswith("dl "), mt.last_config()
        assert_close(c, want, K, am, bm, f"{what} forced dl cfg {cfg}")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(260, 132, 1000), (64, 64, 20), (516, 4, 36), (8, 1028, 4)])
def test_dl_layouts_and_tails(dev, ta, tb, M, N, K):
    a = oracle.uniform((M, K), 100 + M)
    b = oracle.uniform((K, N), 200 + N)
    A, B = _views(a, b, ta, tb, dev)
    c = run(A, B)
    assert mt.last_config().startswith(VECTOR_PATHS), mt.last_config()
    want = oracle.matmul(a, b)
    what = f"dl {M}x{N}x{K} ta={ta} tb={tb}"
    assert_close(c, want, K, amax(a), amax(b), what)
    _also_forced_dl(A, B, want, K, amax(a), amax(b), what)


@pytest.mark.parametrize("M,N,K", [(128, 128, 4100), (96, 64, 6004), (1, 256, 64), (256, 1, 64),
                                   (1000, 1000, 256)])
def test_dl_split_k_and_edges(dev, M, N, K):
    a = oracle.uniform((M, K), 300 + K)
    b = oracle.uniform((K, N), 400 + K)
    A, B = to_gpu(a, dev), to_gpu(b, dev)
    c = run(A, B)
    assert mt.last_config().startswith(VECTOR_PATHS), mt.last_config()
    want = oracle.matmul(a, b)
    assert_close(c, want, K, amax(a), amax(b), f"dl {M}x{N}x{K}")
    np.testing.assert_array_equal(c, run(A, B))   # deterministic, also under split-K
    _also_forced_dl(A, B, want, K, amax(a), amax(b), f"dl {M}x{N}x{K}")


def test_dl_batched_transposed(dev):
    a = oracle.uniform((5, 72, 100), 1)
    b = oracle.uniform((5, 132, 100), 2)              # used as bᵀ: [5,100,132] view
    A = to_gpu(a, dev)
    B = to_gpu(b, dev).transpose(1, 2)
    c = mt.gemm(A, B)
    torch.cuda.synchronize()
    assert mt.last_config().startswith(VECTOR_PATHS), mt.last_config()
    want = oracle.bmm(a, np.ascontiguousarray(b.transpose(0, 2, 1)))
    assert_close(c.cpu().numpy(), want, 100, amax(a), amax(b), "dl batched Bᵀ")


@pytest.mark.parametrize("axis", [mt.BIAS_ROW, mt.BIAS_COL])
def test_dl_bias_and_beta(dev, axis):
    a = oracle.uniform((200, 300), 5)
    b = oracle.uniform((300, 172), 6)
    bias = oracle.uniform((200 if axis == mt.BIAS_ROW else 172,), 7)
    c0 = oracle.uniform((200, 172), 8)
    C = to_gpu(c0, dev)
    mt.gemm(to_gpu(a, dev), to_gpu(b, dev), out=C, beta=1.0, bias=to_gpu(bias, dev),
            bias_axis=axis)
    torch.cuda.synchronize()
    assert mt.last_config().startswith(VECTOR_PATHS), mt.last_config()
    want = oracle.matmul(a, b) + c0 + (bias[:, None] if axis == mt.BIAS_ROW else bias[None, :])
    assert_close(C.cpu().numpy(), want, 300, amax(a), amax(b), f"dl bias {axis} + beta",
                 extra=1e-6)


# ---- epilogue paths -----------------------------------------------------------
# Four consecutive output columns go out as one 16-byte store when C is
# unit-stride, aligned and N % 4 == 0; every other output (strided, transposed,
# misaligned, N % 4 != 0) takes the per-element path.  Same for split-K partials.

@pytest.mark.parametrize("kind", ["transposed", "col_stride2", "offset1", "row_slice"])
def test_output_views(dev, kind):
    M, N, K = 96, 132, 80
    a = oracle.uniform((M, K), 61)
    b = oracle.uniform((K, N), 62)
    if kind == "transposed":
        buf = torch.full((N, M), 7.0, device=dev)
        out = buf.t()                                  # strides (1, M)
    elif kind == "col_stride2":
        buf = torch.full((M, 2 * N), 7.0, device=dev)
        out = buf[:, ::2]                              # strides (2N, 2)
    elif kind == "offset1":
        buf = torch.full((M * N + 1,), 7.0, device=dev)
        out = buf[1:].view(M, N)                       # 4-byte aligned only
    else:
        buf = torch.full((M + 8, N), 7.0, device=dev)
        out = buf[8:]                                  # aligned row slice
    mt.gemm(to_gpu(a, dev), to_gpu(b, dev), out=out)
    torch.cuda.synchronize()
    print(f"[config] {mt.last_config()}", flush=True)
    assert_close(out.cpu().numpy(), oracle.matmul(a, b), K, amax(a), amax(b), f"out {kind}")
    # nothing outside the view was touched
    mask = torch.ones_like(buf, dtype=torch.bool)
    if kind == "transposed":
        mask[:] = False
    elif kind == "col_stride2":
        mask[:, ::2] = False
    elif kind == "offset1":
        mask[1:] = False
    else:
        mask[8:] = False
    assert torch.all(buf[mask] == 7.0)


@pytest.mark.parametrize("N", [66, 68])
def test_split_k_partials_ragged_n(dev, N):
    a = oracle.uniform((64, 8192), 71)
    b = oracle.uniform((8192, N), 72)
    c = run(to_gpu(a, dev), to_gpu(b, dev))
    assert "split=1 " not in mt.last_config() + " "
    assert_close(c, oracle.matmul(a, b), 8192, amax(a), amax(b), f"split-K N={N}")


@pytest.mark.parametrize("axis", [mt.BIAS_ROW, mt.BIAS_COL])
def test_split_k_vector_reduce_bias_beta(dev, axis):
    # split-K partials summed by the 16-byte reduction with the bias and
    # beta*C epilogue applied there
    M, N, K = 64, 132, 8192
    a = oracle.uniform((M, K), 81)
    b = oracle.uniform((K, N), 82)
    bias = oracle.uniform((M if axis == mt.BIAS_ROW else N,), 83)
    c0 = oracle.uniform((M, N), 84)
    C = to_gpu(c0, dev)
    mt.gemm(to_gpu(a, dev), to_gpu(b, dev), out=C, beta=1.0, bias=to_gpu(bias, dev),
            bias_axis=axis)
    torch.cuda.synchronize()
    assert "split=1 " not in mt.last_config() + " ", mt.last_config()
    want = oracle.matmul(a, b) + c0 + (bias[:, None] if axis == mt.BIAS_ROW else bias[None, :])
    assert_close(C.cpu().numpy(), want, K, amax(a), amax(b), f"split-K bias {axis} + beta",
                 extra=1e-6)


# ---- maximum sizes: outputs past 2^31 elements (64-bit addressing) ---------------

@pytest.mark.parametrize("path,forced", [("dl", None), ("dl", 4), ("dl", 5), ("rs", None),
                                         ("ksw", 0), ("ksw", 4)],
                         ids=["dl", "dl4", "dl5", "rs", "ksw0", "ksw4"])
def test_output_beyond_2pow31_elements(dev, path, forced):
    # C[40000, 60000] = 2.4e9 elements (9.6 GB): rows past 35791 start beyond
    # 2^31, so any 32-bit element index in a kernel or epilogue would alias.
    # The cost model's pick, the two prefetching configurations and the
    # wave-split kernel forced.
    M, N, K = 40000, 60000, 32
    a = oracle.uniform((M, K), 91)
    b = oracle.uniform((K, N), 92)
    A = to_gpu(a, dev)
    if path == "rs":    # unaligned view of A: the register-staged kernel
        buf = torch.empty(M * K + 1, device=dev)
        buf[1:].copy_(A.reshape(-1))
        A = buf[1:].view(M, K)
    if forced is None:
        C = mt.gemm(A, to_gpu(b, dev))
    else:
        family = mt.FAMILY_KSW if path == "ksw" else mt.FAMILY_DL
        with mt.forced_config(family, forced, 1):
            C = mt.gemm(A, to_gpu(b, dev))
    torch.cuda.synchronize()
    cfg = mt.last_config()
    print(f"[config] {cfg}", flush=True)
    assert cfg.startswith(path + " "), cfg
    if forced is not None:
        assert cfg.endswith(f" cfg={forced}"), cfg
    rows = np.array([0, 1, 35790, 35791, 35792, 39998, 39999], np.int64)
    got = C[torch.from_numpy(rows).to(dev)].cpu().numpy()
    assert_close(got, oracle.matmul(a[rows], b), K, amax(a), amax(b), f"{path} rows past 2^31")
    del C, A
    torch.cuda.empty_cache()


@pytest.mark.parametrize("forced", [None, 4])
def test_batched_output_beyond_2pow31_elements(dev, forced):
    # 3 x [32768, 32768]: batch 2 starts at element 2^31 of C.
    Bt, M, N, K = 3, 32768, 32768, 16
    a = oracle.uniform((Bt, M, K), 93)
    b = oracle.uniform((Bt, K, N), 94)
    if forced is None:
        C = mt.gemm(to_gpu(a, dev), to_gpu(b, dev))
    else:
        with mt.forced_config(mt.FAMILY_DL, forced, 1):
            C = mt.gemm(to_gpu(a, dev), to_gpu(b, dev))
    torch.cuda.synchronize()
    print(f"[config] {mt.last_config()}", flush=True)
    if forced is not None:
        assert mt.last_config().endswith(f" cfg={forced}"), mt.last_config()
    for bz in (0, 2):
        rows = np.array([0, 17, M - 1], np.int64)
        got = C[bz, torch.from_numpy(rows).to(dev)].cpu().numpy()
        assert_close(got, oracle.matmul(a[bz][rows], b[bz]), K, amax(a), amax(b),
                     f"batch {bz} rows")
    del C
    torch.cuda.empty_cache()
