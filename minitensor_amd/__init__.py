"""minitensor_amd -- MI355X (gfx950) fp32 GEMM backend for miniTensor.

The product is the C-ABI library ``minitensor_amd/lib/libmtgemm.so`` (declared in
``include/mtgemm.h``) and the header-only C++20 host layer in
``minitensor_amd/cpp``.  This module binds the same C ABI from Python with
ctypes; torch is used only for device memory and streams.  There is no CPU or
library fallback: every call goes through the HIP kernels, and a missing
library raises.

Reference semantics mirrored (dionkadi/miniTensor):
  matmul  include/TensorOps.hpp:993-1045   2-D only, A.cols == B.rows, fresh C
  bmm     include/TensorOps.hpp:933-991    3-D [B,M,K]·[B,K,N]
  conv2d  include/TensorOps.hpp:1076-1110  NCHW, output size via safe_out_size
  linear  F::linear (absent upstream): x·wᵀ + b in PyTorch layout
Errors: shape/device errors raise ValueError (the reference's
std::invalid_argument); runtime failures raise RuntimeError.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "lib" / "libmtgemm.so"

MT_OK = 0
MT_ERR_INVALID = -1
MT_ERR_WORKSPACE = -2
MT_ERR_HIP = -3
MT_ERR_UNSUPPORTED = -4
MT_ERR_SCRATCH_LIMIT = -5
NOALLOC_SCRATCH_BYTES = 32 << 20   # MT_NOALLOC_SCRATCH_BYTES

BIAS_NONE, BIAS_ROW, BIAS_COL = 0, 1, 2


class MatF32(ctypes.Structure):
    _fields_ = [
        ("base", ctypes.c_void_p),
        ("offset", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
        ("col_stride", ctypes.c_int64),
        ("batch", ctypes.c_int64),
        ("batch_stride", ctypes.c_int64),
    ]


class EpilogueF32(ctypes.Structure):
    _fields_ = [
        ("bias", ctypes.c_void_p),
        ("bias_stride", ctypes.c_int64),
        ("bias_axis", ctypes.c_int32),
        ("beta", ctypes.c_float),
    ]


class Conv2dDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in
                ("n", "c_in", "h", "w", "c_out", "kh", "kw", "stride", "pad")]


_P = ctypes.POINTER
_SIGS = {
    "mt_gemm_f32": (ctypes.c_int, [_P(MatF32), _P(MatF32), _P(MatF32), _P(EpilogueF32),
                                   ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "mt_gemm_workspace_f32": (ctypes.c_size_t, [_P(MatF32), _P(MatF32), _P(MatF32)]),
    "mt_gemm_noalloc_f32": (ctypes.c_int, [_P(MatF32), _P(MatF32), _P(MatF32), _P(EpilogueF32),
                                           ctypes.c_void_p]),
    "mt_colsum_f32": (ctypes.c_int, [_P(MatF32), ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                     ctypes.c_void_p]),
    "mt_linear_forward_f32": (ctypes.c_int, [_P(MatF32), _P(MatF32), ctypes.c_void_p,
                                             ctypes.c_int64, _P(MatF32), ctypes.c_void_p,
                                             ctypes.c_size_t, ctypes.c_void_p]),
    "mt_linear_workspace_f32": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "mt_linear_backward_f32": (ctypes.c_int, [_P(MatF32), _P(MatF32), _P(MatF32), _P(MatF32),
                                              _P(MatF32), ctypes.c_float, ctypes.c_void_p,
                                              ctypes.c_int64, ctypes.c_float, ctypes.c_void_p,
                                              ctypes.c_size_t, ctypes.c_void_p]),
    "mt_conv2d_fwd_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_size_t, ctypes.c_void_p]),
    "mt_conv2d_fwd_strided_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p,
                                                  _P(ctypes.c_int64), ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_size_t,
                                                  ctypes.c_void_p]),
    "mt_conv2d_workspace_f32": (ctypes.c_size_t, [_P(Conv2dDesc)]),
    "mt_conv2d_bwd_weight_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                                ctypes.c_size_t, ctypes.c_void_p]),
    "mt_conv2d_bwd_input_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p, ctypes.c_void_p,
                                               ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                               ctypes.c_void_p]),
    "mt_conv2d_bwd_bias_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p, ctypes.c_void_p,
                                              ctypes.c_float, ctypes.c_void_p]),
    "mt_conv2d_bwd_weight_bias_f32": (ctypes.c_int, [_P(Conv2dDesc), ctypes.c_void_p,
                                                     ctypes.c_void_p, ctypes.c_void_p,
                                                     ctypes.c_float, ctypes.c_void_p,
                                                     ctypes.c_float, ctypes.c_void_p,
                                                     ctypes.c_size_t, ctypes.c_void_p]),
    "mt_conv2d_bwd_workspace_f32": (ctypes.c_size_t, [_P(Conv2dDesc)]),
    "mt_fill_f32": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                                   ctypes.c_void_p]),
    "mt_axpby_f32": (ctypes.c_int, [_P(MatF32), ctypes.c_float, _P(MatF32), ctypes.c_float,
                                    ctypes.c_void_p]),
    "mt_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "mt_version": (ctypes.c_int, []),
    "mt_last_config": (ctypes.c_char_p, []),
    "mt_gemm_config_count": (ctypes.c_int, [ctypes.c_int]),
    "mt_gemm_force_config": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
}

_lib_handle: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """The loaded libmtgemm.so; raises if it has not been built."""
    global _lib_handle
    if _lib_handle is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m minitensor_amd.build` "
                "(there is no CPU fallback)")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib_handle = h
    return _lib_handle


def _check(rc: int, what: str) -> None:
    if rc == MT_OK:
        return
    msg = f"{what}: {lib().mt_strerror(rc).decode()} ({rc})"
    if rc == MT_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("minitensor_amd kernels take GPU tensors only")
        if t.dtype != torch.float32:
            raise ValueError("minitensor_amd kernels take float32 tensors only")


def mat(t: torch.Tensor) -> MatF32:
    """Descriptor of a 2-D view or a 3-D batched view (no copy, offset kept)."""
    if t.dim() == 2:
        rows, cols = t.shape
        rs, cs = t.stride()
        batch, bs = 1, 0
    elif t.dim() == 3:
        batch, rows, cols = t.shape
        bs, rs, cs = t.stride()
    else:
        raise ValueError("expected a 2-D or 3-D tensor")
    base = t.untyped_storage().data_ptr()
    return MatF32(base, t.storage_offset(), rows, cols, rs, cs, batch, bs)


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _on(stream):
    """Makes `stream` current for the body of an API call, so that the
    outputs, workspaces and operand copies it allocates belong to the stream
    its kernels run on (torch's caching allocator recycles a block only after
    the work queued on its stream), and so that those copies are ordered
    before the kernels that read them."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _api(fn):
    """Runs fn under _on(stream) for its `stream` argument, however passed."""
    import functools
    import inspect

    sig = inspect.signature(fn)
    pos = list(sig.parameters).index("stream")

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        stream = args[pos] if len(args) > pos else kwargs.get("stream")
        with _on(stream):
            return fn(*args, **kwargs)
    return wrapper


def workspace(nbytes: int, device) -> Optional[torch.Tensor]:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


@_api
def gemm(A: torch.Tensor, B: torch.Tensor, out: Optional[torch.Tensor] = None,
         bias: Optional[torch.Tensor] = None, bias_axis: int = BIAS_NONE, beta: float = 0.0,
         ws: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """C = A·B (+bias) (+beta·C) on the GPU through mt_gemm_f32; views are read in place."""
    _require_gpu(A, B, out, bias)
    if A.dim() != B.dim() or A.dim() not in (2, 3):
        raise ValueError("gemm: A and B must both be 2-D or both 3-D")
    if A.shape[-1] != B.shape[-2]:
        raise ValueError("gemm: inner dimension mismatch")
    M, N = A.shape[-2], B.shape[-1]
    if A.dim() == 3:
        batch = max(A.shape[0], B.shape[0])
        shape = (batch, M, N)
    else:
        shape = (M, N)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=A.device)
    elif tuple(out.shape) != shape:
        raise ValueError("gemm: out has the wrong shape")
    ma, mb, mc = mat(A), mat(B), mat(out)
    ep = None
    if bias is not None or beta != 0.0:
        if bias is not None and bias_axis == BIAS_NONE:
            raise ValueError("gemm: bias given without an axis")
        ep = EpilogueF32(_ptr(bias), bias.stride(-1) if bias is not None else 0,
                         bias_axis if bias is not None else BIAS_NONE, float(beta))
    if ws is None:
        ws = workspace(lib().mt_gemm_workspace_f32(ma, mb, mc), A.device)
    rc = lib().mt_gemm_f32(ma, mb, mc, ctypes.byref(ep) if ep is not None else None,
                           _ptr(ws), ws.numel() if ws is not None else 0, _stream(stream))
    _check(rc, "mt_gemm_f32")
    return out


def matmul(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """The reference's matmul for GPU tensors: 2-D only, fresh contiguous C."""
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError("matmul currently only supports 2D tensors.")
    if A.shape[1] != B.shape[0]:
        raise ValueError("Dimension mismatch: A columns must match B rows.")
    return gemm(A, B)


def bmm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """The reference's bmm: A [B,M,K], B [B,K,N] -> C [B,M,N], one batched launch."""
    if A.dim() != 3 or B.dim() != 3:
        raise ValueError("bmm requires 3D tensors.")
    if A.shape[0] != B.shape[0]:
        raise ValueError("bmm: batch dimension mismatch.")
    if A.shape[2] != B.shape[1]:
        raise ValueError("bmm: inner dimension mismatch (A.K != B.K).")
    return gemm(A, B)


@_api
def linear(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None,
           stream=None) -> torch.Tensor:
    """F::linear: y = x·wᵀ + b with w [out,in] (bias fused in the GEMM epilogue)."""
    _require_gpu(x, w, b, out)
    if x.dim() != 2 or w.dim() != 2 or x.shape[1] != w.shape[1]:
        raise ValueError("linear: expected x [B,in] and w [out,in]")
    if b is not None and (b.dim() != 1 or b.shape[0] != w.shape[0]):
        raise ValueError("linear: bias must be [out]")
    if out is None:
        out = torch.empty((x.shape[0], w.shape[0]), dtype=torch.float32, device=x.device)
    if ws is None:
        ws = workspace(lib().mt_linear_workspace_f32(x.shape[0], x.shape[1], w.shape[0]), x.device)
    rc = lib().mt_linear_forward_f32(mat(x), mat(w), _ptr(b), b.stride(0) if b is not None else 0,
                                     mat(out), _ptr(ws), ws.numel() if ws is not None else 0,
                                     _stream(stream))
    _check(rc, "mt_linear_forward_f32")
    return out


@_api
def linear_backward(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, need_dx: bool = True,
                    need_dw: bool = True, need_db: bool = True, dx=None, dw=None, db=None,
                    beta_w: float = 0.0, beta_b: float = 0.0, ws=None, stream=None):
    """dX = dY·W, dW = dYᵀ·X (+beta_w·dW), db = Σ_rows dY (+beta_b·db)."""
    _require_gpu(dy, x, w, dx, dw, db)
    Bn, in_f, out_f = x.shape[0], x.shape[1], w.shape[0]
    dev = x.device
    if need_dx and dx is None:
        dx = torch.empty((Bn, in_f), dtype=torch.float32, device=dev)
    if need_dw and dw is None:
        dw = torch.empty((out_f, in_f), dtype=torch.float32, device=dev)
    if need_db and db is None:
        db = torch.empty((out_f,), dtype=torch.float32, device=dev)
    if ws is None:
        ws = workspace(lib().mt_linear_workspace_f32(Bn, in_f, out_f), dev)
    rc = lib().mt_linear_backward_f32(
        mat(dy), mat(x), mat(w),
        ctypes.byref(mat(dx)) if need_dx else None,
        ctypes.byref(mat(dw)) if need_dw else None, float(beta_w),
        _ptr(db) if need_db else None, db.stride(0) if need_db else 0, float(beta_b),
        _ptr(ws), ws.numel() if ws is not None else 0, _stream(stream))
    _check(rc, "mt_linear_backward_f32")
    return dx, dw, db


@_api
def colsum(x: torch.Tensor, out: Optional[torch.Tensor] = None, beta: float = 0.0,
           stream=None) -> torch.Tensor:
    _require_gpu(x, out)
    if out is None:
        out = torch.empty((x.shape[1],), dtype=torch.float32, device=x.device)
    rc = lib().mt_colsum_f32(mat(x), out.data_ptr(), out.stride(0), float(beta), _stream(stream))
    _check(rc, "mt_colsum_f32")
    return out


def conv_out_size(inp: int, pad: int, k: int, stride: int) -> int:
    """The reference's safe_out_size (include/TensorOps.hpp:17-20)."""
    if inp + 2 * pad < k:
        return 0
    return (inp + 2 * pad - k) // stride + 1


@_api
def conv2d(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor] = None, stride: int = 1,
           padding: int = 0, ws: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """The reference's conv2d forward on NCHW tensors as one fused GEMM.

    x may be any NCHW view (read in place through its strides); the weight
    and bias are made dense."""
    _require_gpu(x, w, b)
    if x.dim() != 4 or w.dim() != 4 or x.shape[1] != w.shape[1]:
        raise ValueError("conv2d: expected input [N,C,H,W] and weight [Cout,C,kh,kw]")
    if b is not None and (b.dim() != 1 or b.shape[0] != w.shape[0]):
        raise ValueError("conv2d: bias must be [Cout]")
    w = w.contiguous()
    b = b.contiguous() if b is not None else None
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    d = Conv2dDesc(n, c, h, wd, co, kh, kw, stride, padding)
    ho, wo = conv_out_size(h, padding, kh, stride), conv_out_size(wd, padding, kw, stride)
    out = torch.empty((n, co, ho, wo), dtype=torch.float32, device=x.device)
    if ws is None:
        ws = workspace(lib().mt_conv2d_workspace_f32(ctypes.byref(d)), x.device)
    strides = (ctypes.c_int64 * 4)(*x.stride())
    rc = lib().mt_conv2d_fwd_strided_f32(ctypes.byref(d), x.data_ptr(), strides, w.data_ptr(),
                                         _ptr(b), out.data_ptr(), _ptr(ws),
                                         ws.numel() if ws is not None else 0, _stream(stream))
    _check(rc, "mt_conv2d_fwd_strided_f32")
    return out


@_api
def conv2d_backward(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, stride: int = 1,
                    padding: int = 0, need_dx: bool = True, need_dw: bool = True,
                    need_db: bool = True, ws: Optional[torch.Tensor] = None, stream=None,
                    dw: Optional[torch.Tensor] = None, beta_w: float = 0.0):
    """Conv2D backward on dense NCHW tensors: returns (dX, dW, db), None where not asked.

    dW = beta_w·dw + ∂L/∂W when an existing dense `dw` is passed (gradient
    accumulation)."""
    _require_gpu(x, w, dy)
    x, w, dy = x.contiguous(), w.contiguous(), dy.contiguous()
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    d = Conv2dDesc(n, c, h, wd, co, kh, kw, stride, padding)
    if tuple(dy.shape) != (n, co, conv_out_size(h, padding, kh, stride),
                           conv_out_size(wd, padding, kw, stride)):
        raise ValueError("conv2d_backward: grad_output has the wrong shape")
    if ws is None:
        ws = workspace(lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d)), x.device)
    wp, wn = _ptr(ws), (ws.numel() if ws is not None else 0)
    dx = db = None
    if not need_dw:
        dw = None
    s = _stream(stream)
    if need_dx:
        dx = torch.empty_like(x)
        _check(lib().mt_conv2d_bwd_input_f32(ctypes.byref(d), dy.data_ptr(), w.data_ptr(),
                                             dx.data_ptr(), wp, wn, s), "mt_conv2d_bwd_input_f32")
    if need_db:
        db = torch.empty((co,), dtype=torch.float32, device=x.device)
    if need_dw:
        if dw is None:
            dw = torch.empty_like(w)
        elif tuple(dw.shape) != tuple(w.shape) or not dw.is_contiguous():
            raise ValueError("conv2d_backward: dw must be a dense tensor shaped like w")
        # dW and db in one call (db can ride on the dW GEMM's reduction launch)
        _check(lib().mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), x.data_ptr(), dy.data_ptr(),
                                                   dw.data_ptr(), float(beta_w), _ptr(db), 0.0,
                                                   wp, wn, s),
               "mt_conv2d_bwd_weight_bias_f32")
    elif need_db:
        _check(lib().mt_conv2d_bwd_bias_f32(ctypes.byref(d), dy.data_ptr(), db.data_ptr(), 0.0, s),
               "mt_conv2d_bwd_bias_f32")
    return dx, dw, db


@_api
def axpby(x: torch.Tensor, y: torch.Tensor, alpha: float = 1.0, beta: float = 0.0,
          stream=None) -> torch.Tensor:
    """y = alpha·x + beta·y in place over 2-D/3-D views (x may have batch 1:
    broadcast).  The strided copy / accumulate kernel of the host layer."""
    _require_gpu(x, y)
    rc = lib().mt_axpby_f32(mat(x), float(alpha), mat(y), float(beta), _stream(stream))
    _check(rc, "mt_axpby_f32")
    return y


def last_config() -> str:
    return lib().mt_last_config().decode()


FAMILY_AUTO, FAMILY_RS, FAMILY_DL, FAMILY_KSW, FAMILY_SKINNY = 0, 1, 2, 3, 4


def config_count(family: int) -> int:
    """Tile configurations of a kernel family (FAMILY_RS, _DL, _KSW or _SKINNY)."""
    return lib().mt_gemm_config_count(int(family))


@contextlib.contextmanager
def forced_config(family: int, cfg: int, splits: int = 1):
    """Force one kernel configuration on this thread's GEMM launches inside the
    block (where the operand layouts allow that family); a tuning and test
    hook.  Query workspace sizes inside the block: they include the forced
    split-K partials."""
    _check(lib().mt_gemm_force_config(int(family), int(cfg), int(splits)), "mt_gemm_force_config")
    try:
        yield
    finally:
        lib().mt_gemm_force_config(FAMILY_AUTO, 0, 1)


def tolerance(K: int, amax: float, bmax: float) -> float:
    """The parity bound: 1e-5·√K·max|A|·max|B| (fp32 accumulation order differs)."""
    return 1e-5 * (max(K, 1) ** 0.5) * amax * bmax
