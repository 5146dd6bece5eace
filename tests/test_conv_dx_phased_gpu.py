"""GPU parity of the input gradient of strided (and non-square stride-1)
convolutions computed by stride phase: one implicit GEMM per phase of the input
pixels (ih % s, iw % s), no column buffer and no col2im.  Checked against the
oracle's restatement of the reference's conv2d_backward_input_cpu
(include/TensorOps.hpp:275-317) on the same seeded inputs; bound
max|err| <= 1e-5·√K·max|dY|·max|W| with K = c_out·kh·kw (tests/util_parity.py).

Shapes: the ResNet downsampling layers (3x3 stride 2 pad 1 and the 1x1
stride-2 shortcut, c_in 64-256) at reduced batch, and geometries that reach the
phase rules' corners: stride 3, a 2x2 stride-2 pad-1 kernel (a phase whose
sub-convolution has negative padding), phases with unequal padding per axis
(3x3 stride 2 pad 0), odd extents, a 7x7 stride-2 stem with 3 input channels,
phases that no tap reaches (1x1 stride 2: zeros), non-square and over-padded
stride-1 kernels, and c_out not a multiple of 16 (the NCHW kernel, dY read in
place) or with phase weights that are not 16-byte rows (the column-buffer
path, kept as the fallback).
"""
import numpy as np
import pytest
import torch

import minitensor_amd as mt
import oracle
from util_parity import amax, assert_close

pytestmark = pytest.mark.gpu

CASES = [
    # n, c_in, h, w, c_out, kh, kw, stride, pad, path
    (2, 64, 28, 28, 64, 3, 3, 2, 1, "cl"),       # ResNet 3x3 stride-2 (layer2 at 1/2 scale)
    (2, 128, 28, 28, 128, 3, 3, 2, 1, "cl"),
    (2, 256, 14, 14, 256, 3, 3, 2, 1, "cl"),
    (2, 64, 26, 26, 128, 1, 1, 2, 0, "cl"),      # 1x1 stride-2 shortcut: 3 of 4 phases zero
    # (a 1x1 layer whose output has a multiple of 4 positions per image takes
    # the per-image product instead, tests/test_conv_pointwise_gpu.py)
    (2, 256, 14, 14, 512, 1, 1, 2, 0, "cl"),
    (3, 32, 15, 13, 48, 3, 3, 2, 1, "cl"),       # odd extents
    (2, 16, 11, 12, 32, 3, 3, 2, 0, "cl"),       # unequal padding per axis in a phase
    (2, 16, 10, 9, 16, 2, 2, 2, 1, "cl"),        # negative sub-convolution padding
    (2, 16, 17, 16, 32, 5, 5, 3, 2, "cl"),       # stride 3
    (2, 3, 32, 30, 64, 7, 7, 2, 3, "cl"),        # the stem: 3 input channels
    (2, 32, 12, 12, 32, 3, 5, 1, 1, "cl"),       # stride 1, non-square kernel
    (2, 16, 9, 9, 32, 3, 3, 1, 3, "cl"),         # stride 1, padding past kh - 1
    (2, 24, 14, 14, 12, 3, 3, 2, 1, "nchw"),     # c_out % 16 != 0: NCHW kernel
    (2, 8, 13, 11, 20, 3, 3, 2, 1, "nchw"),
    (2, 8, 12, 12, 6, 3, 3, 2, 1, "col"),        # phase weights of 6 floats: fallback
    (1, 16, 8, 8, 16, 3, 3, 4, 1, "cl"),         # stride 4: phases of one pixel
    (1, 16, 9, 9, 16, 3, 3, 5, 1, "col"),        # stride 5: fallback
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[1]}-{c[4]}-{c[5]}x{c[6]}-s{c[7]}p{c[8]}-{c[9]}"
                                             for c in CASES])
def test_dx_by_phase(dev, case):
    # The library picks the phased or the column path by modelled cost (small
    # layers like these mostly take the column path); a forced direct-to-LDS
    # configuration skips that rule, so the phase GEMMs run on every case that
    # they can take, under three tile configurations (7: the 64x112 tile of
    # 16x16 blocks, channels-last phases only; elsewhere the cost model's).
    n, c, h, w, co, kh, kw, stride, pad, path = case
    ho, wo = oracle.conv_out(h, pad, kh, stride), oracle.conv_out(w, pad, kw, stride)
    x = oracle.normal((n, c, h, w), 11 + c)
    wt = oracle.normal((co, c, kh, kw), 12 + co, std=(2.0 / (c * kh * kw)) ** 0.5)
    dy = oracle.normal((n, co, ho, wo), 13 + kh)
    X, W, dY = (torch.from_numpy(t).to(dev) for t in (x, wt, dy))
    want, _, _ = oracle.conv2d_backward(x, wt, dy, stride, pad)
    dX, _, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dw=False, need_db=False)
    torch.cuda.synchronize()
    print(f"[config] {case} auto: {mt.last_config()}", flush=True)
    assert_close(dX.cpu().numpy(), want, co * kh * kw, amax(dy), amax(wt), f"dX {case} auto")
    for cfg_i in (1, 3, 7):
        with mt.forced_config(mt.FAMILY_DL, cfg_i, 1):
            dX, _, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dw=False, need_db=False)
            torch.cuda.synchronize()
            cfg = mt.last_config()
            dX2, _, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dw=False, need_db=False)
            torch.cuda.synchronize()
        print(f"[config] {case} forced {cfg_i}: {cfg}", flush=True)
        if path == "cl":
            assert "b=im2col " in cfg + " " and cfg.endswith(f" cfg={cfg_i}"), cfg
        elif path == "nchw":
            assert "b=im2col_nchw" in cfg or "b=im2col_halo" in cfg, cfg
        else:
            assert "im2col" not in cfg, cfg
        got = dX.cpu().numpy()
        assert_close(got, want, co * kh * kw, amax(dy), amax(wt), f"dX {case} forced {cfg_i}")
        # deterministic: a second call gives the same bits
        assert np.array_equal(got.view(np.uint32), dX2.cpu().numpy().view(np.uint32))


def test_dx_by_phase_exact_workspace(dev):
    # the workspace the query reports is enough, and the call refuses less
    n, c, h, w, co, kh, kw, stride, pad = 2, 64, 28, 28, 128, 3, 3, 2, 1
    import ctypes
    d = mt.Conv2dDesc(n, c, h, w, co, kh, kw, stride, pad)
    need = mt.lib().mt_conv2d_bwd_workspace_f32(ctypes.byref(d))
    x = torch.randn(n, c, h, w, device=dev)
    wt = torch.randn(co, c, kh, kw, device=dev) * 0.05
    dy = torch.randn(n, co, 14, 14, device=dev)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    dx = torch.empty_like(x)
    lib = mt.lib()
    rc = lib.mt_conv2d_bwd_input_f32(ctypes.byref(d), dy.data_ptr(), wt.data_ptr(), dx.data_ptr(),
                                     ws.data_ptr(), need, None)
    assert rc == mt.MT_OK
    rc = lib.mt_conv2d_bwd_input_f32(ctypes.byref(d), dy.data_ptr(), wt.data_ptr(), dx.data_ptr(),
                                     ws.data_ptr(), 1024, None)
    assert rc == mt.MT_ERR_WORKSPACE
    torch.cuda.synchronize()
    want, _, _ = oracle.conv2d_backward(x.cpu().numpy(), wt.cpu().numpy(), dy.cpu().numpy(),
                                        stride, pad)
    assert_close(dx.cpu().numpy(), want, co * kh * kw, float(dy.abs().max()),
                 float(wt.abs().max()), "dX with the queried workspace")


def test_dx_by_phase_forced_split(dev):
    # every phase GEMM under a forced split-K configuration: partials and
    # their reduction through the three-level column scatter
    n, c, h, w, co, kh, kw, stride, pad = 2, 32, 15, 14, 64, 3, 3, 2, 1
    x = oracle.normal((n, c, h, w), 21)
    wt = oracle.normal((co, c, kh, kw), 22)
    dy = oracle.normal((n, co, 8, 7), 23)
    want, _, _ = oracle.conv2d_backward(x, wt, dy, stride, pad)
    X, W, dY = (torch.from_numpy(t).to(dev) for t in (x, wt, dy))
    for cfg in (1, 2, 3, 7):
        with mt.forced_config(mt.FAMILY_DL, cfg, 3):
            dX, _, _ = mt.conv2d_backward(X, W, dY, stride, pad, need_dw=False, need_db=False)
            torch.cuda.synchronize()
            name = mt.last_config()
        print(f"[config] forced {cfg}: {name}", flush=True)
        assert "b=im2col " in name + " " and "split=1 " not in name + " ", name
        assert_close(dX.cpu().numpy(), want, co * kh * kw, amax(dy), amax(wt),
                     f"dX forced cfg {cfg} split 3")
