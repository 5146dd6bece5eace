"""CPU tests of the C ABI: the library loads, exports every entry point that
include/mtgemm.h declares, and rejects invalid arguments before touching the
GPU (error behaviour of the reference's matmul: include/TensorOps.hpp:995-1005)."""
import ctypes
import re
from pathlib import Path

import pytest

import minitensor_amd as mt

HEADER_DIR = Path(__file__).resolve().parents[1] / "include"


def declared_functions():
    names = set()
    for h in HEADER_DIR.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(mt_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_the_abi():
    names = declared_functions()
    for n in ["mt_gemm_f32", "mt_gemm_workspace_f32", "mt_conv2d_fwd_f32",
              "mt_linear_forward_f32", "mt_linear_backward_f32", "mt_colsum_f32"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = mt.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_version_and_strerror():
    lib = mt.lib()
    assert lib.mt_version() == 1
    assert lib.mt_strerror(mt.MT_ERR_INVALID) == b"invalid argument"
    assert lib.mt_strerror(mt.MT_ERR_WORKSPACE).startswith(b"workspace")
    assert lib.mt_strerror(12345) == b"unknown status"


def M(rows, cols, rs=None, cs=1, batch=1, bs=0, off=0, base=0x1000):
    return mt.MatF32(base, off, rows, cols, cols if rs is None else rs, cs, batch, bs)


BAD = {
    "inner dimension mismatch": (M(4, 5), M(6, 3), M(4, 3)),
    "C rows mismatch": (M(4, 5), M(5, 3), M(5, 3)),
    "C cols mismatch": (M(4, 5), M(5, 3), M(4, 4)),
    "negative stride": (M(4, 5, rs=-5), M(5, 3), M(4, 3)),
    "negative offset": (M(4, 5, off=-1), M(5, 3), M(4, 3)),
    "batch mismatch": (M(4, 5, batch=3, bs=20), M(5, 3, batch=2, bs=15), M(4, 3, batch=3, bs=12)),
    "negative batch": (M(4, 5), M(5, 3), M(4, 3, batch=-1)),
    "C rows alias (stride 0)": (M(4, 5), M(5, 3), M(4, 3, rs=0)),
    "C cols alias (stride 0)": (M(4, 5), M(5, 3), M(4, 3, cs=0)),
    "null C": (M(4, 5), M(5, 3), M(4, 3, base=0)),
    "null A with K > 0": (M(4, 5, base=0), M(5, 3), M(4, 3)),
    "dimension too large": (M(1 << 31, 5), M(5, 3), M(1 << 31, 3)),
}


@pytest.mark.parametrize("case", sorted(BAD))
def test_gemm_rejects_invalid_arguments(case):
    a, b, c = BAD[case]
    rc = mt.lib().mt_gemm_f32(a, b, c, None, None, 0, None)
    assert rc == mt.MT_ERR_INVALID, case


def test_gemm_rejects_bad_epilogue():
    ep = mt.EpilogueF32(None, 1, mt.BIAS_COL, 0.0)
    rc = mt.lib().mt_gemm_f32(M(4, 5), M(5, 3), M(4, 3), ctypes.byref(ep), None, 0, None)
    assert rc == mt.MT_ERR_INVALID
    ep = mt.EpilogueF32(0x2000, 1, 7, 0.0)
    rc = mt.lib().mt_gemm_f32(M(4, 5), M(5, 3), M(4, 3), ctypes.byref(ep), None, 0, None)
    assert rc == mt.MT_ERR_INVALID


def test_empty_output_is_a_no_op():
    # M == 0 or N == 0: nothing to launch, success (the reference skips the launch too)
    assert mt.lib().mt_gemm_f32(M(0, 5), M(5, 3), M(0, 3), None, None, 0, None) == mt.MT_OK
    assert mt.lib().mt_gemm_f32(M(4, 5), M(5, 0), M(4, 0), None, None, 0, None) == mt.MT_OK
    # a batch of zero matrices (the reference's bmm loops over no entries)
    assert mt.lib().mt_gemm_f32(M(4, 5, batch=0, bs=20), M(5, 3, batch=0, bs=15),
                                M(4, 3, batch=0, bs=12), None, None, 0, None) == mt.MT_OK
    assert mt.lib().mt_gemm_f32(M(4, 5), M(5, 3), M(4, 3, batch=0, bs=12), None, None, 0,
                                None) == mt.MT_OK
    assert mt.last_config() == "empty"


def test_conv_rejects_invalid_descriptors():
    lib = mt.lib()
    for d in [mt.Conv2dDesc(1, 3, 8, 8, 4, 0, 3, 1, 0),    # kh = 0
              mt.Conv2dDesc(1, 3, 8, 8, 4, 3, 3, 0, 0),    # stride 0
              mt.Conv2dDesc(-1, 3, 8, 8, 4, 3, 3, 1, 0),   # negative batch
              mt.Conv2dDesc(1, 3, 8, 8, 4, 3, 3, 1, -1),   # negative padding
              mt.Conv2dDesc(1, 1 << 31, 8, 8, 4, 3, 3, 1, 1),           # field past 32 bits
              mt.Conv2dDesc(1, 1 << 20, 8, 8, 4, 1 << 11, 1, 1, 1 << 11),  # c_in*kh >= 2^31
              mt.Conv2dDesc(1 << 30, 2, 1 << 30, 1 << 30, 1, 1, 1, 1 << 30, 0),
              # n*c_in*h*w and c_out*kg wrap int64 unless capped
              mt.Conv2dDesc(1 << 30, 1 << 30, 1 << 30, 1 << 30, 1, 1, 1, 1 << 30, 0),
              mt.Conv2dDesc(1, 1 << 15, 1, 1, (1 << 31) - 1, 1 << 15, 1, 1, 1 << 15)]:
        rc = lib.mt_conv2d_fwd_f32(ctypes.byref(d), 0x1000, 0x1000, None, 0x1000, None, 0, None)
        assert rc == mt.MT_ERR_INVALID, (d.n, d.c_in, d.h, d.w, d.c_out, d.kh, d.kw)
        assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) == 0
    # kernel larger than the padded input: the reference's safe_out_size gives 0 -> no work
    d = mt.Conv2dDesc(1, 3, 2, 2, 4, 5, 5, 1, 0)
    assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) == 0
    assert lib.mt_conv2d_fwd_f32(ctypes.byref(d), 0x1000, 0x1000, None, 0x1000, None, 0,
                                 None) == mt.MT_OK
    # a real conv without the im2col workspace is refused
    d = mt.Conv2dDesc(2, 3, 8, 8, 4, 3, 3, 1, 1)
    assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) >= 2 * 27 * 64 * 4
    assert lib.mt_conv2d_fwd_f32(ctypes.byref(d), 0x1000, 0x1000, None, 0x1000, None, 0,
                                 None) == mt.MT_ERR_WORKSPACE


def test_conv_nchw_path_workspace_and_weight_bias_arguments():
    lib = mt.lib()
    # c_in*kh*kw % 4 == 0 with c_in % 16 != 0: the NCHW-view path needs room for
    # an aligned weight copy and is refused without a workspace (before any launch)
    d = mt.Conv2dDesc(2, 4, 8, 8, 6, 3, 3, 1, 1)
    assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) >= 6 * 36 * 4
    assert lib.mt_conv2d_fwd_f32(ctypes.byref(d), 0x1000, 0x1000, None, 0x1000, None, 0,
                                 None) == mt.MT_ERR_WORKSPACE
    # the combined weight + bias gradient validates like the two entries it replaces
    bad = mt.Conv2dDesc(1, 3, 8, 8, 4, 0, 3, 1, 0)
    assert lib.mt_conv2d_bwd_weight_bias_f32(ctypes.byref(bad), 0x1000, 0x1000, 0x1000, 0.0,
                                             0x1000, 0.0, None, 0, None) == mt.MT_ERR_INVALID
    assert lib.mt_conv2d_bwd_weight_bias_f32(None, 0x1000, 0x1000, 0x1000, 0.0, 0x1000, 0.0,
                                             None, 0, None) == mt.MT_ERR_INVALID
    d = mt.Conv2dDesc(2, 16, 8, 8, 6, 3, 3, 1, 1)
    assert lib.mt_conv2d_bwd_weight_bias_f32(ctypes.byref(d), 0x1000, None, 0x1000, 0.0,
                                             0x1000, 0.0, None, 0, None) == mt.MT_ERR_INVALID


def test_linear_rejects_mismatched_shapes():
    lib = mt.lib()
    rc = lib.mt_linear_backward_f32(M(8, 10), M(8, 6), M(11, 6), None, None, 0.0, None, 0, 0.0,
                                    None, 0, None)
    assert rc == mt.MT_ERR_INVALID


def test_linear_backward_rejects_negative_bias_grad_stride():
    lib = mt.lib()
    rc = lib.mt_linear_backward_f32(M(8, 10), M(8, 6), M(10, 6), None, M(10, 6), 0.0, 0x2000, -1,
                                    0.0, None, 0, None)
    assert rc == mt.MT_ERR_INVALID


def test_python_front_end_errors():
    import torch
    with pytest.raises(ValueError):
        mt.matmul(torch.zeros(2, 3), torch.zeros(3, 2))          # CPU tensors: GPU only
    with pytest.raises(ValueError):
        mt.conv2d(torch.zeros(1, 1, 3, 3), torch.zeros(1, 1, 2, 2))


def test_config_counts():
    assert mt.config_count(mt.FAMILY_RS) == 3
    assert mt.config_count(mt.FAMILY_DL) == 8
    assert mt.config_count(mt.FAMILY_KSW) == 9
    assert mt.config_count(mt.FAMILY_SKINNY) == 2
    assert mt.config_count(mt.FAMILY_AUTO) == 0


@pytest.mark.parametrize("family,cfg,splits", [
    (5, 0, 1), (-1, 0, 1), (mt.FAMILY_RS, 3, 1), (mt.FAMILY_DL, 8, 1), (mt.FAMILY_DL, -1, 1),
    (mt.FAMILY_KSW, 9, 1), (mt.FAMILY_KSW, -1, 1), (mt.FAMILY_SKINNY, 2, 1),
    (mt.FAMILY_SKINNY, 0, 65),
    (mt.FAMILY_DL, 0, 0), (mt.FAMILY_DL, 0, 65)])
def test_force_config_rejects_unknown(family, cfg, splits):
    assert mt.lib().mt_gemm_force_config(family, cfg, splits) == mt.MT_ERR_INVALID


def test_forced_split_is_in_the_workspace_query():
    """While a split-K configuration is forced, the workspace query covers its
    partials ([splits][batch][M][N] floats); clearing restores the cost model."""
    a, b, c = M(256, 512), M(512, 256), M(256, 256)
    lib = mt.lib()
    auto = lib.mt_gemm_workspace_f32(a, b, c)
    with mt.forced_config(mt.FAMILY_DL, 2, 8):
        assert lib.mt_gemm_workspace_f32(a, b, c) >= 8 * 256 * 256 * 4
    with mt.forced_config(mt.FAMILY_RS, 0, 1):
        assert lib.mt_gemm_workspace_f32(a, b, c) == auto
    assert lib.mt_gemm_workspace_f32(a, b, c) == auto
    # K = 40 holds three 16-deep chunks: at most three splits.
    a, b = M(256, 40), M(40, 256)
    with mt.forced_config(mt.FAMILY_DL, 1, 16):
        assert lib.mt_gemm_workspace_f32(a, b, c) >= 3 * 256 * 256 * 4


def test_gemv_split_partials_in_the_workspace_query():
    """The workspace query covers the split-K partials of the vector-ALU GEMV
    plan: 1x4096·4096x4096 splits K into 64 ranges on a 256-CU device (four
    workgroups per CU over 16 column groups), 64 x 4096 floats; a forced
    skinny configuration with 16 splits needs 16 x 4096."""
    a, b, c = M(1, 4096), M(4096, 4096), M(1, 4096)
    lib = mt.lib()
    assert lib.mt_gemm_workspace_f32(a, b, c) == 64 * 4096 * 4
    with mt.forced_config(mt.FAMILY_SKINNY, 0, 16):
        assert lib.mt_gemm_workspace_f32(a, b, c) == 16 * 4096 * 4
    # the outer product (rank-k) needs no workspace beyond the MFMA plans'
    assert lib.mt_gemm_workspace_f32(M(4096, 1), M(1, 4096), M(4096, 4096)) == 0


def test_conv_backward_workspace_is_the_paths_need():
    """mt_conv2d_bwd_workspace_f32 reports what the dX and dW (+ db) paths use
    (the larger of the two), not buffers they never touch.  Shapes small
    enough that no GEMM splits K, so every term is a buffer:
    3x3 stride 2, n 1, 16 -> 16 channels, 8x8 -> 4x4:
      dX by the column path (the cost model's pick at this size): column
      buffer 144*16 floats (9216 B) + dY copy 16*16 floats (1024 B);
      forced onto the phased path: dY copy (1024 B) + the phases' sub-kernel
      weights 16*16*9 floats (9216 B) + four compact phase outputs of
      1*16*4*4 floats (4 x 1024 B);
      dW implicit: channels-last x 16*8*8 floats (4096 B), dY read in NCHW;
    1x1 stride 2, n 2, 32 -> 64 channels, 8x8 -> 4x4:
      dX: the per-image product's phase-(0, 0) output 2*32*16 floats (4096 B);
      dW: x's output positions 2*32*16 floats (4096 B) + the per-image
      products and their row sums 2*64*(32 + 1) floats (16896 B)."""
    import ctypes
    lib = mt.lib()
    d = mt.Conv2dDesc(1, 16, 8, 8, 16, 3, 3, 2, 1)
    assert lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d)) == 9216 + 1024
    with mt.forced_config(mt.FAMILY_DL, 1, 1):
        assert lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d)) == 1024 + 9216 + 4 * 1024
    d = mt.Conv2dDesc(2, 32, 8, 8, 64, 1, 1, 2, 0)
    assert lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d)) == 4096 + 16896
    # the benchmark's 5a layer: far below its 57.8 MB column buffer
    d = mt.Conv2dDesc(32, 256, 14, 14, 256, 3, 3, 1, 1)
    need = lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d))
    col = 256 * 9 * 32 * 196 * 4
    xt = 32 * 256 * 196 * 4
    assert xt < need < col, need


def test_pointwise_conv_workspace():
    """1x1, stride 1, n 2, 32 -> 64 channels, 8x8 (K = 64 positions or fewer
    channels: no plan splits K).  Backward: dW's per-image partial products
    and their fused row sums (db), 2 x 64 x (32 + 1) floats (16896 B); dX
    needs nothing.  Forward: the batched
    product needs nothing, the NCHW-view kernel (which takes views whose
    (h, w) do not fold) room for an aligned weight copy, 64 x 32 floats."""
    import ctypes
    lib = mt.lib()
    d = mt.Conv2dDesc(2, 32, 8, 8, 64, 1, 1, 1, 0)
    assert lib.mt_conv2d_bwd_workspace_f32(ctypes.byref(d)) == 16896
    assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) == 8192
    # 7x7 positions (not a multiple of 4): the channels-last path and its copies
    d = mt.Conv2dDesc(2, 32, 7, 7, 64, 1, 1, 1, 0)
    assert lib.mt_conv2d_workspace_f32(ctypes.byref(d)) >= 2 * 32 * 49 * 4


def test_build_refuses_kernels_with_scratch():
    """The build raises on a kernel whose resource remark reports scratch
    (spilled registers): parse of hipcc's -Rpass-analysis=kernel-resource-usage
    lines."""
    from minitensor_amd import build
    out = "\n".join([
        "x.hpp:1:1: remark: Function Name: _ZN3mtk9rankk_f32ILi16EEEvNS_10GemmParamsE "
        "[-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:1:1: remark:     VGPRs: 86 [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:1:1: remark:     ScratchSize [bytes/lane]: 272 [-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:2:1: remark: Function Name: _ZN3mtk9rankk_f32ILi4EEEvNS_10GemmParamsE "
        "[-Rpass-analysis=kernel-resource-usage]",
        "x.hpp:2:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert build._scratch_kernels(out) == [("_ZN3mtk9rankk_f32ILi16EEEvNS_10GemmParamsE", 272)]
    assert build._scratch_kernels("no remarks here") == []
