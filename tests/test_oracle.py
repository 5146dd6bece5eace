"""CPU tests that pin the oracle (oracle/oracle.c) before it is trusted as the
checker of the GPU path.

Pins, per oracle function:
  ora_matmul / ora_matmul_strided: the reference's known answers
      (test/tensor_test.cpp:258-283, 368-419, 490-510; test/engien_test.cpp:80-96),
      bit-exact agreement with the reference's own CPU code (oracle/_ref) and
      with the committed reference vectors, fp64 brute force, and invariants
      ((AB)ᵀ = BᵀAᵀ bit-exact, I·B = B, K = 1 outer product, K = 0 zeros).
  ora_bmm: equals a per-batch loop (the reference bmm's intent, F2).
  ora_conv2d: known answer (test/spatial_test.cpp:155-185), bit-exact vs the
      reference build and the committed vectors, im2col·GEMM equivalence.
  ora_colsum (Linear bias gradient): bit-exact vs the reference's
      unbroadcast/sum_cpu through the Linear vectors.
  ora_fill_*: std::mt19937's standard known answer and g++'s std::mt19937.
A planted mistake (a transposed operand) must fail the fp64 check.
"""
import shutil
import subprocess
import textwrap
from pathlib import Path

import numpy as np
import pytest

import oracle
from util_parity import assert_close, tol

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"
needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built here")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


# ---- generator ----------------------------------------------------------------------
def test_mt19937_standard_known_answer():
    # [rand.predef]: the 10000th output of a default-seeded std::mt19937 is 4123659995
    assert int(oracle.mt19937_stream(5489, 10000)[-1]) == 4123659995


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_mt19937_matches_libstdcxx(tmp_path):
    src = tmp_path / "mt.cpp"
    src.write_text(textwrap.dedent("""
        #include <random>
        #include <cstdio>
        int main() { for (unsigned s : {42u, 43u}) { std::mt19937 g(s);
          for (int i = 0; i < 1000; ++i) std::printf("%u\\n", (unsigned)g()); } }
    """))
    exe = tmp_path / "mt"
    subprocess.run(["g++", "-O1", "-o", str(exe), str(src)], check=True)
    want = np.array(subprocess.run([str(exe)], capture_output=True, text=True,
                                   check=True).stdout.split(), dtype=np.uint64)
    got = np.concatenate([oracle.mt19937_stream(42, 1000), oracle.mt19937_stream(43, 1000)])
    np.testing.assert_array_equal(got, want)


def test_uniform_and_normal_transforms():
    u = oracle.uniform((200000,), 42)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1 / 3) < 0.01
    # the transform is exact: 24-bit grid of [-1, 1)
    assert np.all(np.mod((u.astype(np.float64) + 1.0) * 2 ** 23, 1.0) == 0.0)
    n = oracle.normal((200000,), 43, std=0.01)
    assert abs(n.mean()) < 1e-4 and abs(n.std() - 0.01) < 2e-4
    np.testing.assert_array_equal(oracle.uniform((10,), 7), oracle.uniform((10,), 7))
    assert not np.array_equal(oracle.uniform((10,), 7), oracle.uniform((10,), 8))


# ---- reference known answers ---------------------------------------------------------------
def test_known_answer_matmul():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, b), [[58, 64], [139, 154]])


def test_known_answer_matmul_gradients():
    # MatmulBackward with dC = ones: dA = dC·Bᵀ = [15,19,23] per row, dB = Aᵀ·dC = [5,7,9] per row
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    dc = np.ones((2, 2), np.float32)
    np.testing.assert_array_equal(oracle.matmul(dc, b.T), [[15, 19, 23], [15, 19, 23]])
    np.testing.assert_array_equal(oracle.matmul(a.T, dc), [[5, 5], [7, 7], [9, 9]])
    # bias gradient of D = A·B + C with C [2]: unbroadcast -> column sums = [2, 2]
    np.testing.assert_array_equal(oracle.colsum(dc), [2, 2])
    # test/engien_test.cpp:80-96 and tensor_test.cpp:490-510: 2s · 3s
    a2, b2 = np.full((2, 3), 2, np.float32), np.full((3, 2), 3, np.float32)
    np.testing.assert_array_equal(oracle.matmul(a2, b2), np.full((2, 2), 18))
    np.testing.assert_array_equal(oracle.matmul(dc, b2.T), np.full((2, 3), 6))
    np.testing.assert_array_equal(oracle.matmul(a2.T, dc), np.full((3, 2), 4))


def test_known_answer_conv2d():
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    w = np.ones((1, 1, 2, 2), np.float32)
    out = oracle.conv2d(x, w, np.zeros(1, np.float32), 1, 0)
    np.testing.assert_array_equal(out.reshape(-1), [12, 16, 24, 28])


# ---- the reference's own code -----------------------------------------------------------------
def test_golden_vectors(gold):
    g = gold
    a = np.lib.stride_tricks.as_strided(g["offset_a_store"][10:], (3, 5), (20, 4))
    b = np.lib.stride_tricks.as_strided(g["offset_b_store"][3:], (5, 4), (16, 4))
    np.testing.assert_array_equal(oracle.matmul(a, b), g["offset_c"])
    np.testing.assert_array_equal(oracle.matmul(g["bT_a"], g["bT_bt"].T), g["bT_c"])
    row = np.broadcast_to(g["expand_row"][None, :], (17, 40))
    np.testing.assert_array_equal(oracle.matmul(row, g["expand_b"]), g["expand_c"])
    np.testing.assert_array_equal(oracle.matmul(g["dense_a"], g["dense_b"]), g["dense_c"])
    np.testing.assert_array_equal(oracle.conv2d(g["conv_x"], g["conv_w"], g["conv_b"], 2, 1),
                                  g["conv_out"])
    w = g["lin_w_ref"].T  # PyTorch layout [out,in] of the reference's W_ref [in,out]
    np.testing.assert_array_equal(oracle.linear(g["lin_x"], w, g["lin_b"]), g["lin_y"])
    dx, dw, db = oracle.linear_backward(g["lin_dy"], g["lin_x"], w)
    np.testing.assert_array_equal(dx, g["lin_dx"])
    np.testing.assert_array_equal(dw, g["lin_dw_ref"].T)
    np.testing.assert_array_equal(db, g["lin_db"])
    # conv backward from the reference's autograd, three images (per-image
    # accumulation of dW and db), stride 1 and 2
    for tag in ("s1", "s2"):
        st, pad = (int(v) for v in g[f"cbwd_{tag}_geom"])
        dx, dw, db = oracle.conv2d_backward(g[f"cbwd_{tag}_x"], g[f"cbwd_{tag}_w"],
                                            g[f"cbwd_{tag}_dy"], st, pad)
        np.testing.assert_array_equal(dx, g[f"cbwd_{tag}_dx"])
        np.testing.assert_array_equal(dw, g[f"cbwd_{tag}_dw"])
        np.testing.assert_array_equal(db, g[f"cbwd_{tag}_db"])


def test_golden_binary_matches_npz(gold):
    """The raw fixture the C++ host tests read holds the same arrays."""
    import struct
    raw = (GOLDEN.with_suffix(".bin")).read_bytes()
    assert raw[:8] == b"MTGOLD01"
    (count,) = struct.unpack_from("<I", raw, 8)
    pos, seen = 12, {}
    for _ in range(count):
        (ln,) = struct.unpack_from("<I", raw, pos)
        name = raw[pos + 4:pos + 4 + ln].decode()
        pos += 4 + ln
        (nd,) = struct.unpack_from("<I", raw, pos)
        dims = struct.unpack_from(f"<{nd}Q", raw, pos + 4)
        pos += 4 + 8 * nd
        n = int(np.prod(dims)) if nd else 1
        seen[name] = np.frombuffer(raw, "<f4", n, pos).reshape(dims)
        pos += 4 * n
    assert pos == len(raw) and sorted(seen) == sorted(gold)
    for k in gold:
        np.testing.assert_array_equal(seen[k], gold[k])


@needs_ref
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 13, 5), (64, 128, 96), (130, 70, 33)])
def test_matches_reference_build_dense(M, K, N):
    a = oracle.uniform((M, K), M)
    b = oracle.uniform((K, N), N + 100)
    c = np.empty((M, N), np.float32)
    oracle.ref().ref_matmul_f32(oracle._fp(a), oracle._fp(b), oracle._fp(c), M, K, N)
    np.testing.assert_array_equal(oracle.matmul(a, b), c)


@needs_ref
@pytest.mark.parametrize("case", ["at", "bt", "both", "slice", "expand_b"])
def test_matches_reference_build_views(case):
    M, K, N = 37, 29, 41
    store_a = oracle.normal((64 * 64,), 1)
    store_b = oracle.normal((64 * 64,), 2)
    # (offset, row_stride, col_stride) of each view inside its storage
    va = {"at": (0, 1, 40), "both": (5, 1, 50), "slice": (3 * 31, 31, 1)}.get(case, (0, K, 1))
    vb = {"bt": (0, 1, 33), "both": (7, 1, 45), "expand_b": (0, 0, 1)}.get(case, (0, N, 1))
    c = np.empty((M, N), np.float32)
    oracle.ref().ref_matmul_view_f32(oracle._fp(store_a), store_a.size, *va,
                                     oracle._fp(store_b), store_b.size, *vb, M, K, N,
                                     oracle._fp(c))
    a = np.lib.stride_tricks.as_strided(store_a[va[0]:], (M, K), (va[1] * 4, va[2] * 4))
    b = np.lib.stride_tricks.as_strided(store_b[vb[0]:], (K, N), (vb[1] * 4, vb[2] * 4))
    np.testing.assert_array_equal(oracle.matmul(a, b), c)


@needs_ref
def test_matches_reference_build_conv_and_linear():
    x = oracle.normal((3, 4, 11, 10), 3)
    w = oracle.normal((6, 4, 3, 2), 4)
    bias = oracle.normal((6,), 5)
    for stride, pad in [(1, 0), (1, 1), (2, 2), (3, 1)]:
        want = oracle.conv2d(x, w, bias, stride, pad)
        got = np.empty_like(want)
        oracle.ref().ref_conv2d_f32(oracle._fp(x), oracle._fp(w), oracle._fp(bias),
                                    oracle._fp(got), 3, 4, 11, 10, 6, 3, 2, stride, pad)
        np.testing.assert_array_equal(want, got)
    B, fin, fout = 9, 31, 14
    x = oracle.normal((B, fin), 6)
    w_ref = oracle.normal((fin, fout), 7)
    b = oracle.normal((fout,), 8)
    dy = oracle.normal((B, fout), 9)
    outs = [np.empty(s, np.float32) for s in [(B, fout), (B, fin), (fin, fout), (fout,)]]
    oracle.ref().ref_linear_f32(oracle._fp(x), oracle._fp(w_ref), oracle._fp(b), oracle._fp(dy),
                                B, fin, fout, *[oracle._fp(o) for o in outs])
    np.testing.assert_array_equal(oracle.linear(x, w_ref.T, b), outs[0])
    dx, dw, db = oracle.linear_backward(dy, x, w_ref.T)
    np.testing.assert_array_equal(dx, outs[1])
    np.testing.assert_array_equal(dw, outs[2].T)
    np.testing.assert_array_equal(db, outs[3])


# ---- what the mathematics fixes -------------------------------------------------------------
@pytest.mark.parametrize("M,K,N", [(33, 47, 29), (128, 300, 64), (5, 1000, 3)])
def test_fp64_brute_force(M, K, N):
    a = oracle.uniform((M, K), 1)
    b = oracle.uniform((K, N), 2)
    assert_close(oracle.matmul(a, b), oracle.matmul_f64_rows(a, b, range(M)), K, 1.0, 1.0,
                 f"oracle vs fp64 {M}x{K}x{N}")
    np.testing.assert_allclose(oracle.matmul_f64_rows(a, b, range(M)),
                               a.astype(np.float64) @ b.astype(np.float64), rtol=0, atol=1e-9)


def test_invariants():
    a = oracle.normal((31, 17), 1)
    b = oracle.normal((17, 23), 2)
    # (AB)ᵀ = BᵀAᵀ, bit-exact: the same products summed in the same k order
    np.testing.assert_array_equal(oracle.matmul(b.T, a.T), oracle.matmul(a, b).T)
    np.testing.assert_array_equal(oracle.matmul(np.eye(31, dtype=np.float32), a), a)
    np.testing.assert_array_equal(oracle.matmul(a, np.eye(17, dtype=np.float32)), a)
    u, v = a[:, :1], b[:1, :]
    np.testing.assert_array_equal(oracle.matmul(u, v), u * v)
    np.testing.assert_array_equal(oracle.matmul(np.zeros((4, 0), np.float32),
                                                np.zeros((0, 6), np.float32)), np.zeros((4, 6)))
    # views equal their materialised copies
    big = oracle.normal((40, 50), 3)
    view = big[5:36:2, 3:20]
    np.testing.assert_array_equal(oracle.matmul(view, b), oracle.matmul(view.copy(), b))


def test_bmm_is_a_loop_of_matmul():
    a = oracle.uniform((4, 9, 7), 1)
    b = oracle.uniform((4, 7, 5), 2)
    c = oracle.bmm(a, b)
    for z in range(4):
        np.testing.assert_array_equal(c[z], oracle.matmul(a[z], b[z]))


def test_conv_equals_im2col_gemm():
    x = oracle.normal((2, 3, 8, 7), 1)
    w = oracle.normal((4, 3, 3, 3), 2)
    bias = oracle.normal((4,), 3)
    stride, pad = 2, 1
    out = oracle.conv2d(x, w, bias, stride, pad)
    n, c, h, wd = x.shape
    ho, wo = out.shape[2:]
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    col = np.empty((c * 9, n * ho * wo), np.float32)
    for ci in range(c):
        for r in range(3):
            for s in range(3):
                patch = xp[:, ci, r:r + stride * ho:stride, s:s + stride * wo:stride]
                col[(ci * 3 + r) * 3 + s] = patch.reshape(-1)
    g = oracle.matmul(w.reshape(4, -1), col).reshape(4, n, ho, wo).transpose(1, 0, 2, 3)
    assert_close(out, g + bias[None, :, None, None], c * 9, np.abs(x).max(), np.abs(w).max(),
                 "conv vs im2col gemm", extra=1e-6)


def test_linear_gradient_formulas_by_finite_difference():
    # L(X, W, b) = Σ dY ⊙ (X·Wᵀ + b) in fp64; its exact derivatives must match the
    # oracle's backward formulas (the reference's gradcheck recipe,
    # test/spatial_test.cpp:66-123, on a linear function).
    x = oracle.normal((6, 5), 1).astype(np.float64)
    w = oracle.normal((4, 5), 2).astype(np.float64)
    dy = oracle.normal((6, 4), 3).astype(np.float64)
    L = lambda X, W, B: float(np.sum(dy * (X @ W.T + B)))  # noqa: E731
    b = np.zeros(4)
    eps = 1e-3

    def fd(f, p):
        g = np.zeros_like(p)
        for idx in np.ndindex(p.shape):
            q = p.copy(); q[idx] += eps; hi = f(q)
            q[idx] -= 2 * eps; lo = f(q)
            g[idx] = (hi - lo) / (2 * eps)
        return g

    dx, dw, db = oracle.linear_backward(dy.astype(np.float32), x.astype(np.float32),
                                        w.astype(np.float32))
    np.testing.assert_allclose(dx, fd(lambda X: L(X, w, b), x), atol=1e-5)
    np.testing.assert_allclose(dw, fd(lambda W: L(x, W, b), w), atol=1e-5)
    np.testing.assert_allclose(db, fd(lambda B: L(x, w, B), b), atol=1e-5)


def test_planted_transpose_mistake_is_caught():
    # A plausible bug -- reading B transposed -- must fail the fp64 parity check.
    a = oracle.uniform((24, 24), 1)
    b = oracle.uniform((24, 24), 2)
    wrong = oracle.matmul(a, b.T)
    with pytest.raises(AssertionError):
        assert_close(wrong, oracle.matmul_f64_rows(a, b, range(24)), 24, 1.0, 1.0, "planted")
    # and a dropped last k term as well
    dropped = oracle.matmul(a[:, :-1], b[:-1])
    assert np.max(np.abs(dropped - oracle.matmul_f64_rows(a, b, range(24)))) > tol(24, 1, 1)


@needs_ref
@pytest.mark.parametrize("n,c,h,w,co,kh,kw,stride,pad", [
    (2, 3, 9, 7, 4, 3, 3, 1, 1), (1, 2, 8, 8, 3, 3, 2, 2, 0), (3, 4, 5, 6, 2, 1, 1, 1, 0),
    (2, 2, 7, 7, 3, 5, 5, 3, 2)])
def test_conv_backward_matches_reference_build(n, c, h, w, co, kh, kw, stride, pad):
    x = oracle.normal((n, c, h, w), 1)
    wt = oracle.normal((co, c, kh, kw), 2)
    ho, wo = oracle.conv_out(h, pad, kh, stride), oracle.conv_out(w, pad, kw, stride)
    dy = oracle.normal((n, co, ho, wo), 3)
    dx, dw, db = oracle.conv2d_backward(x, wt, dy, stride, pad)
    rdx, rdw, rdb = np.empty_like(dx), np.empty_like(dw), np.empty_like(db)
    oracle.ref().ref_conv2d_bwd_f32(*[oracle._fp(t) for t in (x, wt, dy, rdx, rdw, rdb)],
                                    n, c, h, w, co, kh, kw, stride, pad)
    np.testing.assert_array_equal(dx, rdx)
    np.testing.assert_array_equal(dw, rdw)
    np.testing.assert_array_equal(db, rdb)


def test_conv_backward_adjoint_identities():
    # conv is bilinear: <dY, conv(x, w)> = <dX(dY, w), x> = <dW(dY, x), w>  (bias 0)
    x = oracle.normal((2, 3, 8, 9), 1)
    w = oracle.normal((4, 3, 3, 3), 2)
    for stride, pad in [(1, 1), (2, 0), (2, 2)]:
        y = oracle.conv2d(x, w, None, stride, pad)
        dy = oracle.normal(y.shape, 3)
        dx, dw, db = oracle.conv2d_backward(x, w, dy, stride, pad)
        ip = float(np.sum(dy.astype(np.float64) * y))
        assert abs(float(np.sum(dx.astype(np.float64) * x)) - ip) <= 1e-4 * (1 + abs(ip))
        assert abs(float(np.sum(dw.astype(np.float64) * w)) - ip) <= 1e-4 * (1 + abs(ip))
        np.testing.assert_allclose(db, dy.astype(np.float64).sum(axis=(0, 2, 3)), atol=1e-4)
