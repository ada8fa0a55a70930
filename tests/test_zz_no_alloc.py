"""GPU test of titan_qgemm_batched_noalloc, the batched dequant-GEMV whose
K-split workspace is the library's static device scratch: called through the
C ABI, its outputs equal titan_qgemm_batched_ws's with a caller workspace bit
for bit, on two calls in a row (the second with a smaller input, which finds
the scratch as the first call left it), and match the oracle's exact
dequantized weights within the GEMV bar (max error <= 1e-3 of max |ref|)."""
import ctypes

import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import assert_close_out, make_weights
from gpu_util import act, to_np, upload

pytestmark = pytest.mark.gpu


def _call_noalloc(Ws, Xs, Ys):
    n = len(Ws)
    arr = (tq.QWeightC * n)(*[w.cstruct() for w in Ws])
    xs = (ctypes.c_void_p * n)(*[tq._ptr(x) for x in Xs])
    ys = (ctypes.c_void_p * n)(*[tq._ptr(y) for y in Ys])
    return tq.lib().titan_qgemm_batched_noalloc(arr, xs, ys, n, tq.dtype_code(Xs[0].dtype),
                                                tq.dtype_code(Ys[0].dtype), Xs[0].shape[0], None)


@pytest.mark.parametrize("fmt,gs", [("int2", 64), ("q3k", 256)])
def test_noalloc_matches_workspace_entry_point(fmt, gs, rng):
    # call 1: two 256 x 8192 problems, 4 tokens; call 2: one smaller
    # 128 x 4096 problem, 2 tokens (both launches hold fewer waves than CUs,
    # so the K split engages in both)
    calls = [([(256, 8192), (256, 8192)], 4), ([(128, 4096)], 2)]
    for shapes, M in calls:
        print(f"noalloc {fmt} shapes={shapes} M={M}", flush=True)
        ds = [make_weights(fmt, r, c, rng, gs=gs) for r, c in shapes]
        Ws = [upload(d, tq.LAYOUT_TILED) for d in ds]
        X = [act(M, c, "f16", rng) for _, c in shapes]
        Xs = [x for x, _ in X]
        Y_na = [torch.full((M, r), float("nan"), device="cuda") for r, _ in shapes]
        Y_ws = [torch.full((M, r), float("nan"), device="cuda") for r, _ in shapes]
        assert _call_noalloc(Ws, Xs, Y_na) == tq.OK
        ws = tq.qgemm_workspace([r for r, _ in shapes], M)
        tq.qgemm_batched(Ws, Xs, Y_ws, workspace=ws)
        torch.cuda.synchronize()
        for d, (_, x64), ya, yw in zip(ds, X, Y_na, Y_ws):
            assert torch.equal(ya, yw), "noalloc must equal the workspace entry point bit for bit"
            assert_close_out(to_np(ya), x64 @ d["deq"].astype(np.float64).T, "f32")


def test_noalloc_rejects_beyond_scratch_and_leaves_outputs(rng):
    d = make_weights("int4", 4096, 1024, rng, gs=128)
    W = upload(d, tq.LAYOUT_TILED)
    M = 32
    rows = (ctypes.c_int * 8)(*([4096] * 8))
    assert tq.lib().titan_qgemm_workspace_bytes(rows, 8, M) > tq.NOALLOC_SCRATCH_BYTES
    x = torch.randn(M, 1024, dtype=torch.float16, device="cuda")
    ys = [torch.zeros(M, 4096, dtype=torch.float16, device="cuda") for _ in range(8)]
    assert _call_noalloc([W] * 8, [x] * 8, ys) == tq.ERR_SCRATCH_LIMIT
    # within the limit the same weights run (split or not) and match
    assert _call_noalloc([W], [x], ys[:1]) == tq.OK
    torch.cuda.synchronize()
    assert all(torch.all(y == 0) for y in ys[1:])
    assert_close_out(to_np(ys[0]), x.double().cpu().numpy() @ d["deq"].astype(np.float64).T, "f16")
