"""GPU parity of the dequant-GEMV with the K range split across workgroups
(titan_qgemm_ws / titan_qgemm_batched_ws, caller workspace).

Same bar as the single-workgroup path: max error normalised by max|ref| <=
1e-3 against the fp64 product of the oracle's exact dequantized weights, one
last-place unit allowed on fp16/bf16 outputs.  The partial sums are added in
a fixed order, so repeated calls must agree bit for bit, and the workspace's
counters must be back at zero after every call (a reused workspace gives the
same results, also after a call of another shape).
"""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import assert_close_out, make_weights
from gpu_util import TDT, act, to_np, upload

pytestmark = pytest.mark.gpu

LAYOUTS = {"ref": tq.LAYOUT_REF, "tiled": tq.LAYOUT_TILED}
# rows x cols small enough that the launch holds few waves: the split engages
# for INT2 and Q3_K; the other formats must run unchanged through the same API
SHAPES = {"int4": (48, 4096, 128), "int2": (48, 4096, 64), "fp4": (32, 2048, 64),
          "nvfp4": (48, 4096, 16), "q4k": (32, 4096, 256), "q3k": (32, 4096, 256),
          "fp8": (32, 2048, 0)}


def lays(fmt):
    return ["tiled"] if fmt == "q3k" else ["ref", "tiled"]


CASES = [(f, l) for f in SHAPES for l in lays(f)]


@pytest.mark.parametrize("fmt,lay", CASES)
@pytest.mark.parametrize("M", [1, 2, 4, 8, 11, 24])
def test_splitk_parity(fmt, lay, M, rng):
    rows, cols, gs = SHAPES[fmt]
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, LAYOUTS[lay])
    ws = tq.qgemm_workspace(rows, M)
    deq64 = d["deq"].astype(np.float64).T
    for xdt, ydt in [("f16", "f16"), ("f32", "f32"), ("bf16", "bf16"), ("f16", "f32")]:
        x, x64 = act(M, cols, xdt, rng)
        y = tq.qgemm(W, x, out_dtype=TDT[ydt], workspace=ws)
        y2 = tq.qgemm(W, x, out_dtype=TDT[ydt], workspace=ws)
        torch.cuda.synchronize()
        assert_close_out(to_np(y), x64 @ deq64, ydt)
        assert torch.equal(y, y2), "split-K results must be deterministic"


@pytest.mark.parametrize("fmt,rows,cols,gs", [("q4k", 4096, 4096, 256), ("int2", 1024, 8192, 64),
                                              ("q3k", 1024, 8192, 256), ("int4", 1024, 4096, 128)])
@pytest.mark.parametrize("M", [1, 4])
def test_splitk_config_shapes(fmt, rows, cols, gs, M, rng):
    """The C1 Q4_K 4096^2 matrix and the 1024-row 70B / 8B shapes, tiled."""
    d = make_weights(fmt, rows, cols, rng, gs=gs)
    W = upload(d, tq.LAYOUT_TILED)
    ws = tq.qgemm_workspace(rows, M)
    x, x64 = act(M, cols, "f16", rng)
    y = tq.qgemm(W, x, out_dtype=torch.float16, workspace=ws)
    base = tq.qgemm(W, x, out_dtype=torch.float16)
    torch.cuda.synchronize()
    ref = x64 @ d["deq"].astype(np.float64).T
    assert_close_out(to_np(y), ref, "f16")
    assert_close_out(to_np(base), ref, "f16")


@pytest.mark.parametrize("fmt,n,k", [("q3k", 28672, 8192), ("int2", 28672, 8192),
                                     ("q3k", 8192, 8192), ("int2", 8192, 28672)])
@pytest.mark.parametrize("M", [1, 4])
def test_workspace_full_size_70b(fmt, n, k, M):
    """The large 70B shapes with a caller workspace, as a caller passes it:
    whichever split the launch heuristics pick, every output row of the first
    and last token matches the oracle's fp32 GEMV of the same REF bytes, and
    the results equal the launch without a workspace within the same bar."""
    import bench
    from oracle import oracle_ctypes as O
    gen = torch.Generator(device="cuda").manual_seed(3 * n + k + M)
    if fmt == "int2":
        (m,) = bench.make_int4_layer(gen, gs=64, bits=2, shapes=[("w", n, k)])
        W = tq.QWeight(tq.INT2, tq.LAYOUT_TILED, n, k, m["tiled"], group_size=64)
        w, s, b = (t.cpu().numpy() for t in m["ref"])
        codes, s16, b16, gs = w.view(np.uint32), s.view(np.uint16), b.view(np.uint16), 64
    else:
        blk = bench.random_kquant(tq.Q3_K, n, k, gen)
        W = tq.QWeight(tq.Q3_K, tq.LAYOUT_TILED, n, k,
                       torch.from_numpy(tq.repack_host(tq.Q3_K, n, k, blk)).cuda())
        codes, s16, b16, gs = blk, None, None, 0
    x = torch.randn(M, k, generator=gen, device="cuda").half()
    ws = tq.qgemm_workspace(n, M)
    y = tq.qgemm(W, x, out_dtype=torch.float32, workspace=ws)
    y2 = tq.qgemm(W, x, out_dtype=torch.float32, workspace=ws)
    base = tq.qgemm(W, x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    for t in sorted({0, M - 1}):
        ref = O.matvec_fmt_mt(fmt, codes, s16, b16, 1.0, gs, x[t].float().cpu().numpy(), n, k, 8)
        assert_close_out(to_np(y[t]), ref.astype(np.float64), "f32")
        assert_close_out(to_np(base[t]), ref.astype(np.float64), "f32")


def test_splitk_workspace_reuse_across_shapes(rng):
    """One workspace serves a large call, a smaller call and the large call
    again: the counters left by each call must be zero for the next."""
    big = make_weights("int4", 256, 4096, rng, gs=128)
    small = make_weights("q4k", 32, 1024, rng)
    Wb, Ws_ = upload(big, tq.LAYOUT_TILED), upload(small, tq.LAYOUT_TILED)
    ws = tq.qgemm_workspace(256, 4)
    xb, xb64 = act(4, 4096, "f16", rng)
    xs, xs64 = act(2, 1024, "f16", rng)
    y1 = tq.qgemm(Wb, xb, out_dtype=torch.float32, workspace=ws)
    y2 = tq.qgemm(Ws_, xs, out_dtype=torch.float32, workspace=ws)
    y3 = tq.qgemm(Wb, xb, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    assert_close_out(to_np(y1), xb64 @ big["deq"].astype(np.float64).T, "f32")
    assert_close_out(to_np(y2), xs64 @ small["deq"].astype(np.float64).T, "f32")
    assert torch.equal(y1, y3)
    # M = 11 in fp32 runs two launches (8 + 3 tokens) on one workspace
    xf, xf64 = act(11, 4096, "f32", rng)
    yf = tq.qgemm(Wb, xf, out_dtype=torch.float32, workspace=tq.qgemm_workspace(256, 11))
    torch.cuda.synchronize()
    assert_close_out(to_np(yf), xf64 @ big["deq"].astype(np.float64).T, "f32")


def test_splitk_workspace_reuse_across_problem_sets(rng):
    """One workspace serves a one-problem call, then a two-problem batched
    call: the second problem's counters must not land on the partial sums the
    first call left (they sit in their own region), so both calls match the
    oracle and a repeat of each gives the same bits."""
    ds = [make_weights("int2", 1024, 8192, rng, gs=64) for _ in range(2)]
    Ws = [upload(d, tq.LAYOUT_TILED) for d in ds]
    ws = tq.qgemm_workspace([1024, 1024], 4)
    for M in (1, 4):
        X = [act(M, 8192, "f16", rng) for _ in range(2)]
        y1 = tq.qgemm(Ws[0], X[0][0], out_dtype=torch.float32, workspace=ws)
        Ys = [torch.zeros(M, 1024, dtype=torch.float32, device="cuda") for _ in range(2)]
        tq.qgemm_batched(Ws, [x for x, _ in X], Ys, workspace=ws)
        y1b = tq.qgemm(Ws[0], X[0][0], out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(y1, y1b)
        assert_close_out(to_np(y1), X[0][1] @ ds[0]["deq"].astype(np.float64).T, "f32")
        for d, (_, x64), Y in zip(ds, X, Ys):
            assert_close_out(to_np(Y), x64 @ d["deq"].astype(np.float64).T, "f32")


@pytest.mark.parametrize("lay", list(LAYOUTS))
def test_splitk_batched(lay, rng):
    shapes = [(64, 4096), (16, 4096), (48, 2048), (32, 1024)]
    ds = [make_weights("int4", r, c, rng, gs=128) for r, c in shapes]
    Ws = [upload(d, LAYOUTS[lay]) for d in ds]
    ws = tq.qgemm_workspace([r for r, _ in shapes], 3)
    for M in (1, 3):
        Xs = [torch.randn(M, c, dtype=torch.float16, device="cuda") for _, c in shapes]
        Ys = [torch.zeros(M, r, dtype=torch.float16, device="cuda") for r, _ in shapes]
        tq.qgemm_batched(Ws, Xs, Ys, workspace=ws)
        torch.cuda.synchronize()
        for d, X, Y in zip(ds, Xs, Ys):
            ref = X.double().cpu().numpy() @ d["deq"].astype(np.float64).T
            assert_close_out(to_np(Y), ref, "f16")


def test_splitk_workspace_errors(rng):
    d = make_weights("int4", 48, 1024, rng, gs=128)
    W = upload(d, tq.LAYOUT_TILED)
    x = torch.randn(1, 1024, dtype=torch.float16, device="cuda")
    y = torch.zeros(1, 48, dtype=torch.float16, device="cuda")
    need = tq.qgemm_workspace_bytes(48, 1)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    L, c = tq.lib(), W.cstruct()
    import ctypes
    args = (ctypes.byref(c), tq._ptr(x), tq.dtype_code(x.dtype), 1024, tq._ptr(y),
            tq.dtype_code(y.dtype), 48, 1)
    assert L.titan_qgemm_ws(*args, tq._ptr(ws), need - 256, None) == tq.ERR_WORKSPACE
    assert L.titan_qgemm_ws(*args, None, need, None) == tq.ERR_INVALID_ARG
    assert L.titan_qgemm_ws(*args, tq._ptr(ws[16:]), need - 16, None) == tq.ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert torch.all(y == 0)
