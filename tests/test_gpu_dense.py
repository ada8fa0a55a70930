"""Dense GEMV (gemv.cu:33-159) and the format-exact matvec_dispatch
(dense.cpp:13-32) on the GPU against fp64 products of the same operands.
Tolerance: max |y - ref| <= 1e-3 * max |ref| (fp32 output)."""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from gpu_util import upload
from helpers import assert_close_out, make_weights

pytestmark = pytest.mark.gpu


def bf16_bits(a):
    return torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(16, 512), (37, 4096), (130, 7168), (8, 8200),
                                       (20000, 64), (5, 100), (3, 7)])
def test_gemv_bf16(rows, cols, rng):
    A = bf16_bits(rng.normal(0, 0.02, (rows, cols)))
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = torch.empty(rows, device="cuda")
    tq.gemv_bf16_to_fp32(A.cuda(), torch.from_numpy(x).cuda(), y, rows, cols)
    torch.cuda.synchronize()
    ref = A.float().double().numpy() @ x.astype(np.float64)
    assert_close_out(y.cpu().numpy().astype(np.float64), ref, "f32")


@pytest.mark.parametrize("rows,cols,batch", [(64, 1024, 1), (33, 257, 1), (16, 4096, 3)])
def test_gemv_fp32(rows, cols, batch, rng):
    A = rng.normal(0, 0.02, (rows * batch, cols)).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = torch.empty(rows * batch, device="cuda")
    Ad, xd = torch.from_numpy(A).cuda(), torch.from_numpy(x).cuda()
    if batch == 1:
        tq.gemv_fp32(Ad, xd, y, rows, cols)
    else:
        tq.gemv_fp32_batched(Ad, xd, y, rows, cols, batch)
    torch.cuda.synchronize()
    assert_close_out(y.cpu().numpy().astype(np.float64), A.astype(np.float64) @ x.astype(np.float64), "f32")


@pytest.mark.parametrize("fmt", ["int4", "int2", "fp4", "nvfp4", "q4k", "q3k", "fp8", "dense_f32", "dense_bf16"])
@pytest.mark.parametrize("lay", [tq.LAYOUT_REF, tq.LAYOUT_TILED])
def test_matvec_dispatch_format_exact(fmt, lay, rng):
    """Each format reaches its own decoder: Q4_K is decoded as Q4_K (the
    reference routes it to the INT4 kernel, dense.cpp:19-24)."""
    rows, cols = 48, 1024
    x = rng.normal(0, 1, cols).astype(np.float32)
    if fmt.startswith("dense"):
        if lay == tq.LAYOUT_TILED:
            pytest.skip("dense weights have no tiled form")
        A = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        if fmt == "dense_bf16":
            t = bf16_bits(A).cuda()
            deq = bf16_bits(A).float().double().numpy()
            W = tq.QWeight(tq.BF16, tq.LAYOUT_REF, rows, cols, t)
        else:
            t = torch.from_numpy(A).cuda()
            deq = A.astype(np.float64)
            W = tq.QWeight(tq.FP32, tq.LAYOUT_REF, rows, cols, t)
    else:
        d = make_weights(fmt, rows, cols, rng, gs=128)
        W = upload(d, lay)
        deq = d["deq"].astype(np.float64)
    y = torch.empty(rows, device="cuda")
    tq.matvec_dispatch(W, torch.from_numpy(x).cuda(), y)
    torch.cuda.synchronize()
    assert_close_out(y.cpu().numpy().astype(np.float64), deq @ x.astype(np.float64), "f32")
