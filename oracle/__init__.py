"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the fp32 GEMM family.

Python (numpy + ctypes) front end of ``oracle/liboracle.so``, a plain-C
restatement of miniTensor's CPU reference path (see oracle.c for the
reference file:line of every function), and of ``oracle/_ref/libref.so``, the
reference's own CPU code compiled from its headers (present only where it was
built).  Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg
use this package; the product never does.

Inputs are generated with std::mt19937 (fully specified by the C++ standard)
and fixed transforms, so the same seed gives the same tensors everywhere:
  uniform(lo, hi): lo + (hi-lo)·((x >> 8)·2⁻²⁴)
  normal(mean, σ): mean + σ·√(-2 ln(1-u₁))·cos(2π u₂)   (one value per pair)
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref.so"

_f = ctypes.POINTER(ctypes.c_float)
_d = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.POINTER(ctypes.c_int64)
_sz = ctypes.c_size_t

_lib = None
_ref = None


def build() -> None:
    """Compile liboracle.so (and libref.so when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if Path("/root/reference/include/TensorOps.hpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(LIB_PATH))
        h.ora_mt19937_seed.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        h.ora_mt19937_next.argtypes = [ctypes.c_void_p]
        h.ora_mt19937_next.restype = ctypes.c_uint32
        h.ora_fill_uniform.argtypes = [_f, _sz, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        h.ora_fill_normal.argtypes = [_f, _sz, ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        h.ora_matmul.argtypes = [_f, _f, _f, _sz, _sz, _sz]
        h.ora_matmul_strided.argtypes = [_f, _sz, _sz, _f, _sz, _sz, _f, _sz, _sz, _sz, _sz, _sz]
        h.ora_bmm.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz]
        h.ora_conv2d.argtypes = [_f, _f, _f, _f] + [_sz] * 9
        h.ora_colsum.argtypes = [_f, _sz, _sz, _sz, _sz, _f]
        h.ora_conv2d_bwd_input.argtypes = [_f, _f, _f] + [_sz] * 9
        h.ora_conv2d_bwd_weight.argtypes = [_f, _f, _f] + [_sz] * 9
        h.ora_conv2d_bwd_bias.argtypes = [_f, _f] + [_sz] * 4
        h.ora_matmul_f64_rows.argtypes = [_f, _sz, _sz, _f, _sz, _sz, _i64, _sz, _sz, _sz, _d]
        _lib = h
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def ref() -> ctypes.CDLL:
    """The reference's own CPU code (oracle/_ref/libref.so)."""
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise RuntimeError(f"{REF_PATH} not built (needs the reference tree)")
        h = ctypes.CDLL(str(REF_PATH))
        h.ref_matmul_f32.argtypes = [_f, _f, _f, _sz, _sz, _sz]
        h.ref_matmul_view_f32.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _sz,
                                          _sz, _sz, _sz, _f]
        h.ref_conv2d_f32.argtypes = [_f, _f, _f, _f] + [_sz] * 9
        h.ref_linear_f32.argtypes = [_f, _f, _f, _f, _sz, _sz, _sz, _f, _f, _f, _f]
        h.ref_conv2d_bwd_f32.argtypes = [_f, _f, _f, _f, _f, _f] + [_sz] * 9
        _ref = h
    return _ref


def _fp(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.dtype == np.float32
    return a.ctypes.data_as(_f)


# ---- seeded inputs -------------------------------------------------------------
def uniform(shape: Sequence[int], seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(tuple(shape), dtype=np.float32)
    lib().ora_fill_uniform(_fp(out), out.size, seed, lo, hi)
    return out


def normal(shape: Sequence[int], seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(tuple(shape), dtype=np.float32)
    lib().ora_fill_normal(_fp(out), out.size, seed, mean, std)
    return out


def mt19937_stream(seed: int, n: int) -> np.ndarray:
    state = ctypes.create_string_buffer(624 * 4 + 8)
    lib().ora_mt19937_seed(state, seed)
    return np.array([lib().ora_mt19937_next(state) for _ in range(n)], dtype=np.uint64)


# ---- reference CPU path ----------------------------------------------------------
def _elem_strides(a: np.ndarray):
    assert a.dtype == np.float32
    for s in a.strides:
        if s % 4 != 0 or s < 0:
            raise ValueError("oracle views need non-negative element strides")
    return tuple(s // 4 for s in a.strides)


def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """matmul_cpu / matmul_cpu_strided on 2-D numpy views (any non-negative strides)."""
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = np.empty((M, N), dtype=np.float32)
    if a.flags.c_contiguous and b.flags.c_contiguous:
        lib().ora_matmul(_fp(a), _fp(b), _fp(c), M, K, N)
    else:
        asm, ask = _elem_strides(a)
        bsk, bsn = _elem_strides(b)
        pa = ctypes.cast(ctypes.c_void_p(a.ctypes.data), _f)
        pb = ctypes.cast(ctypes.c_void_p(b.ctypes.data), _f)
        lib().ora_matmul_strided(pa, asm, ask, pb, bsk, bsn, _fp(c), N, 1, M, K, N)
    return c


def bmm(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    Bn, M, K = a.shape
    _, _, N = b.shape
    c = np.empty((Bn, M, N), dtype=np.float32)
    lib().ora_bmm(_fp(a), _fp(b), _fp(c), Bn, M, K, N)
    return c


def conv_out(inp: int, pad: int, k: int, stride: int) -> int:
    return 0 if inp + 2 * pad < k else (inp + 2 * pad - k) // stride + 1


def conv2d(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray], stride: int, pad: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w)
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    out = np.empty((n, co, conv_out(h, pad, kh, stride), conv_out(wd, pad, kw, stride)), np.float32)
    lib().ora_conv2d(_fp(x), _fp(w), _fp(np.ascontiguousarray(b)) if b is not None else None,
                     _fp(out), n, c, h, wd, co, kh, kw, stride, pad)
    return out


def conv2d_backward(x: np.ndarray, w: np.ndarray, dy: np.ndarray, stride: int, pad: int):
    """conv2d_backward_{input,weight,bias}_cpu: returns (dX, dW, db)."""
    x, w, dy = (np.ascontiguousarray(t) for t in (x, w, dy))
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    dx = np.empty_like(x)
    dw = np.empty_like(w)
    db = np.empty((co,), np.float32)
    lib().ora_conv2d_bwd_input(_fp(dy), _fp(w), _fp(dx), n, c, h, wd, co, kh, kw, stride, pad)
    lib().ora_conv2d_bwd_weight(_fp(dy), _fp(x), _fp(dw), n, c, h, wd, co, kh, kw, stride, pad)
    lib().ora_conv2d_bwd_bias(_fp(dy), _fp(db), n, co, dy.shape[2], dy.shape[3])
    return dx, dw, db


def colsum(x: np.ndarray) -> np.ndarray:
    rs, cs = _elem_strides(x)
    out = np.empty((x.shape[1],), np.float32)
    px = ctypes.cast(ctypes.c_void_p(x.ctypes.data), _f)
    lib().ora_colsum(px, rs, cs, x.shape[0], x.shape[1], _fp(out))
    return out


def linear(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray]) -> np.ndarray:
    """F::linear in PyTorch layout as the reference computes Linear: matmul(x, wᵀ-view) + b."""
    y = matmul(x, w.T)
    if b is not None:
        y = y + b[None, :].astype(np.float32)
    return y


def linear_backward(dy: np.ndarray, x: np.ndarray, w: np.ndarray):
    """MatmulBackward through transpose views (dX = dY·W, dW = dYᵀ·X) and sum_cpu for db."""
    dx = matmul(dy, w)
    dw = matmul(dy.T, x)
    db = colsum(dy)
    return dx, dw, db


# ---- checkers ----------------------------------------------------------------------
def matmul_f64_rows(a: np.ndarray, b: np.ndarray, rows: Sequence[int]) -> np.ndarray:
    """fp64 brute force of the selected rows of a·b (full K)."""
    asm, ask = _elem_strides(a)
    bsk, bsn = _elem_strides(b)
    r = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    out = np.empty((len(r), b.shape[1]), np.float64)
    pa = ctypes.cast(ctypes.c_void_p(a.ctypes.data), _f)
    pb = ctypes.cast(ctypes.c_void_p(b.ctypes.data), _f)
    lib().ora_matmul_f64_rows(pa, asm, ask, pb, bsk, bsn, r.ctypes.data_as(_i64), len(r),
                              a.shape[1], b.shape[1], out.ctypes.data_as(_d))
    return out


def tolerance(K: int, amax: float, bmax: float) -> float:
    return 1e-5 * (max(K, 1) ** 0.5) * amax * bmax
