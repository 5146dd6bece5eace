"""GPU checks of the support kernels around the GEMMs: the strided
copy/accumulate (mt_axpby_f32, the host layer's copy_gpu_strided and gradient
accumulation) and the column sums (Linear bias gradient when not fused)."""
import numpy as np
import pytest
import torch

import minitensor_amd as mt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["dense", "transposed", "offset1", "batch_bcast", "ragged"])
def test_axpby_views(dev, kind):
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    if kind == "dense":               # 16-byte path
        x = torch.rand(37, 64, device=dev, generator=gen)
        y = torch.rand(37, 64, device=dev, generator=gen)
    elif kind == "transposed":        # strided reads
        x = torch.rand(64, 37, device=dev, generator=gen).t()
        y = torch.rand(37, 64, device=dev, generator=gen)
    elif kind == "offset1":           # unaligned rows: scalar path
        x = torch.rand(37 * 64 + 1, device=dev, generator=gen)[1:].view(37, 64)
        y = torch.rand(37 * 64 + 1, device=dev, generator=gen)[1:].view(37, 64)
    elif kind == "batch_bcast":       # x batch 1 broadcast over y's batch
        x = torch.rand(1, 12, 20, device=dev, generator=gen).expand(5, 12, 20)[:1]
        y = torch.rand(5, 12, 20, device=dev, generator=gen)
    else:                             # cols % 4 != 0
        x = torch.rand(9, 31, device=dev, generator=gen)
        y = torch.rand(9, 31, device=dev, generator=gen)
    want = 1.5 * x.double() + 0.25 * y.double()
    mt.axpby(x, y, 1.5, 0.25)
    torch.cuda.synchronize()
    np.testing.assert_allclose(y.cpu().numpy(), want.cpu().numpy(), rtol=1e-6, atol=1e-6)
    mt.axpby(x, y, -2.0, 0.0)             # plain scaled copy: beta = 0 ignores y
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), (-2.0 * x).expand_as(y).cpu().numpy())


@pytest.mark.parametrize("rows,cols,batch,off,bcast", [
    (1024, 2048, 1, 0, False),   # C3's Bᵀ materialised: the tiled 16-byte path
    (67, 45, 1, 0, False),       # ragged extents: the tiled scalar path
    (33, 130, 3, 0, False),      # batched
    (40, 36, 4, 0, True),        # one matrix broadcast over the batch
    (96, 64, 1, 1, False),       # storage offset by one float: unaligned reads
    (31, 200, 1, 0, False),      # rows < 32: the element-wise kernel
])
def test_axpby_transposed_copy_is_exact(dev, rows, cols, batch, off, bcast):
    # y = x for x a transposed view (adjacent rows, strided columns) and y dense:
    # a layout change through LDS tiles, bit for bit the copy
    gen = torch.Generator(device=dev)
    gen.manual_seed(rows * 7 + cols)
    nb = 1 if bcast else batch
    store = torch.rand(nb * cols * rows + off, device=dev, generator=gen)
    x = store[off:].view(nb, cols, rows).transpose(1, 2)          # [nb][rows][cols], row stride 1
    if bcast:
        x = x.expand(batch, rows, cols)
    x = x if batch > 1 else x[0]
    y = torch.full((batch, rows, cols) if batch > 1 else (rows, cols), 7.0, device=dev)
    mt.axpby(x[:1] if bcast else x, y, 1.0, 0.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), x.contiguous().cpu().numpy())
