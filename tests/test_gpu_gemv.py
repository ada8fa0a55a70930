"""GPU parity of the dequant and dequant-GEMV kernels against the CPU oracle.

Dequantized values: bit-exact (memcmp of fp32 bits).  Matmul outputs: max
error normalised by max|ref| <= 1e-3, where ref is the fp64 product of the
oracle's exact dequantized weights and the activations as rounded to their
input dtype; fp16/bf16 outputs may also differ from the rounded reference by
one unit in the last place (helpers.assert_close_out).
"""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import assert_close_out, make_weights, max_rel_err
from gpu_util import FMTS, TDT, act, dev, to_np, upload

from oracle import oracle_ctypes as O

pytestmark = pytest.mark.gpu

LAYOUTS = {"ref": tq.LAYOUT_REF, "tiled": tq.LAYOUT_TILED}
SHAPES = {"int4": (64, 1024, 128), "int2": (48, 2048, 64), "fp4": (32, 1024, 64),
          "nvfp4": (48, 1024, 16), "q4k": (32, 1024, 256), "q3k": (32, 1024, 256),
          "fp8": (32, 512, 0)}


def layouts_for(fmt):
    return ["ref", "tiled"]


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("lay", list(LAYOUTS))
def test_dequant_bit_exact(fmt, lay, rng):
    rows, cols, gs = SHAPES[fmt]
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, LAYOUTS[lay])
    out = tq.qdequant(W, torch.float32)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), d["deq"].view(np.uint32))
    # fp16 / bf16 outputs are the RNE rounding of the exact value
    h = tq.qdequant(W, torch.float16).cpu()
    assert torch.equal(h, torch.from_numpy(d["deq"]).to(torch.float16))
    b = tq.qdequant(W, torch.bfloat16).cpu()
    assert torch.equal(b, torch.from_numpy(d["deq"]).to(torch.bfloat16))


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("lay", list(LAYOUTS))
@pytest.mark.parametrize("M", [1, 2, 4, 8, 11])
def test_qgemm_parity(fmt, lay, M, rng):
    rows, cols, gs = SHAPES[fmt]
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, LAYOUTS[lay])
    for xdt, ydt in [("f16", "f16"), ("f32", "f32"), ("bf16", "bf16"), ("f16", "f32")]:
        x, x64 = act(M, cols, xdt, rng)
        y = tq.qgemm(W, x, out_dtype=TDT[ydt])
        torch.cuda.synchronize()
        ref = x64 @ d["deq"].astype(np.float64).T
        assert_close_out(to_np(y), ref, ydt)


@pytest.mark.parametrize("fmt,lay", [("int2", "ref"), ("int2", "tiled"), ("q3k", "tiled"),
                                     ("q4k", "tiled"), ("int4", "ref")])
@pytest.mark.parametrize("M", [17, 32, 40])
def test_qgemm_many_tokens(fmt, lay, M, rng):
    """More than 16 fp16 tokens on the matrix-core GEMV: 256-column-chunk
    formats (INT2, Q3_K) take 16 tokens a launch (the activation stage of 32
    would not fit in LDS), the others 32."""
    rows, cols, gs = SHAPES[fmt]
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, LAYOUTS[lay])
    x, x64 = act(M, cols, "f16", rng)
    y = tq.qgemm(W, x, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, "f16")


@pytest.mark.parametrize("fmt", ["int4", "int2", "fp4", "nvfp4", "q4k", "fp8"])
def test_ragged_rows_and_strides(fmt, rng):
    # rows not a multiple of 16; x / y with padded row strides
    rows, cols, gs = {"int4": (37, 512, 64), "int2": (21, 512, 64), "fp4": (19, 256, 32),
                      "nvfp4": (45, 512, 16), "q4k": (7, 512, 256), "fp8": (29, 256, 0)}[fmt]
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, tq.LAYOUT_REF)
    xfull = torch.randn(3, cols + 40, dtype=torch.float16, device="cuda")
    x = xfull[:, :cols]
    yfull = torch.zeros(3, rows + 24, dtype=torch.float32, device="cuda")
    y = yfull[:, :rows]
    tq.qgemm(W, x, out=y)
    torch.cuda.synchronize()
    ref = x.double().cpu().numpy() @ d["deq"].astype(np.float64).T
    assert_close_out(to_np(y), ref, "f32")
    assert torch.all(yfull[:, rows:] == 0)


@pytest.mark.parametrize("fmt,rows,cols,gs", [("int4", 24, 136, 8), ("int4", 16, 200, 40),
                                              ("int2", 9, 272, 16), ("fp4", 5, 104, 8),
                                              ("nvfp4", 17, 48, 16), ("q3k", 5, 512, 256)])
def test_generic_path_odd_shapes(fmt, rows, cols, gs, rng):
    """Shapes the reference wrappers accept but the 16-byte-slot kernel does
    not (cols % 32, small groups, Q3_K's 110-byte blocks) take the generic
    kernel; results must still match."""
    d = make_weights(fmt, rows, cols, rng, gs=gs)
    W = upload(d, tq.LAYOUT_REF)
    x, x64 = act(2, cols, "f32", rng)
    y = tq.qgemm(W, x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, "f32")
    out = tq.qdequant(W, torch.float32).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), d["deq"].view(np.uint32))


def test_reference_signature_entry_points(rng):
    """dispatch.h-shaped calls: fp32 in / fp32 out, REF layout."""
    rows, cols = 96, 2048
    x = rng.normal(0, 1, cols).astype(np.float32)
    xd = dev(x)
    y = torch.zeros(rows, dtype=torch.float32, device="cuda")
    # INT4, group 64 (convert_titan.py default) and 128; against the
    # reference-loop CPU GEMV (matmul_avx.cpp restated, bit-exact with it)
    for gs in (64, 128):
        d = make_weights("int4", rows, cols, rng, gs=gs)
        tq.dequant_matvec_int4(dev(d["codes"]), dev(d["scales"]), dev(d["biases"]), xd, y,
                               rows, cols, gs)
        torch.cuda.synchronize()
        ref = O.matvec_int4_cpu(d["codes"], d["scales"], d["biases"], x, rows, cols, gs)
        assert max_rel_err(y.cpu().numpy(), ref) < 1e-5
    d = make_weights("int2", rows, cols, rng, gs=64)
    tq.dequant_matvec_int2(dev(d["codes"]), dev(d["scales"]), dev(d["biases"]), xd, y, rows,
                           cols, 64)
    torch.cuda.synchronize()
    assert max_rel_err(y.cpu().numpy(), O.gemm_f64(d["deq"], x)[0]) < 1e-5
    d = make_weights("fp4", rows, cols, rng, gs=32)
    tq.dequant_matvec_fp4(dev(d["codes"]), dev(d["scales"]), xd, y, rows, cols, 32)
    torch.cuda.synchronize()
    assert max_rel_err(y.cpu().numpy(), O.gemm_f64(d["deq"], x)[0]) < 1e-5
    d = make_weights("nvfp4", rows, cols, rng)
    tq.dequant_matvec_nvfp4(dev(d["codes"]), dev(d["scales"]), d["g"], xd, y, rows, cols)
    torch.cuda.synchronize()
    ref = O.matvec_nvfp4(d["codes"], d["scales"], d["g"], x, rows, cols)  # fp4.cu loop order
    assert max_rel_err(y.cpu().numpy(), ref) < 1e-5


def test_invalid_arguments_launch_nothing():
    L = tq.lib()
    y = torch.zeros(16, device="cuda")
    # cols not a multiple of 8 / of the group size: the reference preconditions
    st = L.titan_dequant_matvec_int4(None, None, None, None, None, 16, 100, 64, None)
    assert st == tq.ERR_INVALID_ARG
    w = torch.zeros(16 * 12, dtype=torch.int32, device="cuda")
    s = torch.zeros(16 * 2, dtype=torch.float16, device="cuda")
    x = torch.zeros(100, device="cuda")
    st = L.titan_dequant_matvec_int4(tq._ptr(w), tq._ptr(s), tq._ptr(s), tq._ptr(x), tq._ptr(y),
                                     16, 100, 64, None)
    assert st == tq.ERR_UNSUPPORTED
    torch.cuda.synchronize()
    assert torch.all(y == 0)


@pytest.mark.parametrize("lay", list(LAYOUTS))
def test_special_cases(lay, rng):
    rows, cols, gs = 32, 512, 64
    # all-zero codes with s = 0, b = 1 -> every weight is 1: y = sum(x)
    codes = np.zeros((rows, cols // 8), np.uint32)
    s = np.zeros((rows, cols // gs), np.uint16)
    b = np.full((rows, cols // gs), 0x3C00, np.uint16)
    d = {"fmt": "int4", "rows": rows, "cols": cols, "gs": gs, "g": 1.0, "codes": codes,
         "scales": s, "biases": b}
    W = upload(d, LAYOUTS[lay])
    x, x64 = act(1, cols, "f32", rng)
    y = to_np(tq.qgemm(W, x, out_dtype=torch.float32))
    assert np.abs(y - x64.sum()).max() < 1e-4
    # one-hot x returns a dequantized column exactly
    d = make_weights("q4k", rows, cols, rng)
    W = upload(d, LAYOUTS[lay])
    for c in (0, 37, 255, 300, 511):
        x = torch.zeros(1, cols, device="cuda")
        x[0, c] = 1.0
        y = tq.qgemm(W, x, out_dtype=torch.float32).cpu().numpy()[0]
        assert np.array_equal(y, d["deq"][:, c])


@pytest.mark.parametrize("lay", list(LAYOUTS))
def test_batched_launch_matches_single(lay, rng):
    shapes = [(64, 1024), (16, 1024), (48, 2048), (32, 512)]
    ds = [make_weights("int4", r, c, rng, gs=128) for r, c in shapes]
    Ws = [upload(d, LAYOUTS[lay]) for d in ds]
    for M in (1, 3):
        Xs = [torch.randn(M, c, dtype=torch.float16, device="cuda") for _, c in shapes]
        Ys = [torch.zeros(M, r, dtype=torch.float16, device="cuda") for r, _ in shapes]
        tq.qgemm_batched(Ws, Xs, Ys)
        torch.cuda.synchronize()
        for d, X, Y in zip(ds, Xs, Ys):
            ref = X.double().cpu().numpy() @ d["deq"].astype(np.float64).T
            assert_close_out(to_np(Y), ref, "f16")


@pytest.mark.parametrize("M", [5, 6, 8, 16, 24, 32, 50, 64, 100])
@pytest.mark.parametrize("rows,cols,gs", [(64, 512, 128), (80, 384, 32), (208, 1024, 64),
                                          (128, 768, 256)])
def test_int4_token_tiled_parity(M, rows, cols, gs, rng):
    """INT4 tiled with M >= 5 runs the token-tiled dequant-GEMM (up to 8 tokens its
    branch-free loop; partial row blocks, every group size class, one and several 16-token
    tiles, 64-token tiles)."""
    d = make_weights("int4", rows, cols, rng, gs=gs)
    W = upload(d, tq.LAYOUT_TILED)
    for xdt, ydt in [("f16", "f16"), ("bf16", "f32"), ("f32", "bf16")]:
        x, x64 = act(M, cols, xdt, rng)
        y = tq.qgemm(W, x, out_dtype=TDT[ydt])
        torch.cuda.synchronize()
        assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, ydt)


def test_int4_token_tiled_batched_strided(rng):
    """Batched problems of different shapes share one launch; padded strides."""
    shapes = [(64, 512), (16, 512), (112, 1024)]
    ds = [make_weights("int4", r, c, rng, gs=128) for r, c in shapes]
    Ws = [upload(d, tq.LAYOUT_TILED) for d in ds]
    M = 40
    Xs = [act(M, c, "f16", rng) for _, c in shapes]
    Ys = [torch.empty(M, r, dtype=torch.float16, device="cuda") for r, _ in shapes]
    tq.qgemm_batched(Ws, [x for x, _ in Xs], Ys)
    torch.cuda.synchronize()
    for d, (x, x64), y in zip(ds, Xs, Ys):
        assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, "f16")
    d = ds[0]
    xfull = torch.randn(M, 512 + 56, dtype=torch.float16, device="cuda")
    yfull = torch.zeros(M, 64 + 8, dtype=torch.float32, device="cuda")
    tq.qgemm(Ws[0], xfull[:, :512], out=yfull[:, :64])
    torch.cuda.synchronize()
    ref = xfull[:, :512].double().cpu().numpy() @ d["deq"].astype(np.float64).T
    assert_close_out(to_np(yfull[:, :64]), ref, "f32")
    assert torch.all(yfull[:, 64:] == 0)


@pytest.mark.parametrize("rows,cols,gs,nact", [(64, 512, 128, 17), (40, 1000, 40, 40), (96, 256, 64, 0)])
def test_sparse_dequant_matvec_int4(rows, cols, gs, nact, rng):
    """sparse.cu:142-205: only the listed rows are written (REF INT4, fp32)."""
    d = make_weights("int4", rows, cols, rng, gs=gs)
    active = np.sort(rng.choice(rows, size=nact, replace=False)).astype(np.int32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = torch.full((rows,), 7.5, device="cuda")
    tq.sparse_dequant_matvec_int4(dev(d["codes"]), dev(d["scales"]), dev(d["biases"]), dev(x), y,
                                  dev(active) if nact else torch.zeros(0, dtype=torch.int32, device="cuda"),
                                  cols, gs)
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    ref = d["deq"].astype(np.float64) @ x.astype(np.float64)
    mask = np.zeros(rows, bool)
    mask[active] = True
    assert np.all(got[~mask] == 7.5)
    if nact:
        assert_close_out(got[mask], ref[mask], "f32")


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("fmt,rows,cols,gs", [("int4", 32, 1024, 256), ("int4", 16, 640, 128),
                                              ("int4", 48, 512, 32), ("int4", 64, 14336, 128),
                                              ("int2", 16, 1024, 512), ("int2", 32, 768, 128)])
def test_scale_cells_and_k_split(fmt, rows, cols, gs, M, rng):
    """Tiled INT4 / INT2 scales in 16-byte cells (groups over several chunks,
    padded cells, several groups per chunk) and long rows whose chunks are
    split between the waves of a workgroup."""
    d = make_weights(fmt, rows, cols, rng, gs=gs)
    W = upload(d, tq.LAYOUT_TILED)
    x, x64 = act(M, cols, "f16", rng)
    y = tq.qgemm(W, x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, "f32")


@pytest.mark.parametrize("M", [1, 8, 32])
def test_llama8b_layer_full_size(M):
    """The headline workload at its real size: the seven INT4 g128 matrices of
    a Llama-3-8B layer in one batched launch against the oracle's fp32 GEMV
    (dequant.cu:23-104 semantics) on every output, for a sample of tokens."""
    import bench
    gen = torch.Generator(device="cuda").manual_seed(11 + M)
    layer = bench.make_int4_layer(gen)
    Ws = [tq.QWeight(m["fmt"], tq.LAYOUT_TILED, m["rows"], m["cols"], m["tiled"], group_size=128)
          for m in layer]
    X = {k: torch.randn(M, k, generator=gen, device="cuda").half() for k in (4096, 14336)}
    Xs = [X[m["cols"]] for m in layer]
    Ys = [torch.empty(M, m["rows"], device="cuda", dtype=torch.float32) for m in layer]
    tq.qgemm_batched(Ws, Xs, Ys)
    torch.cuda.synchronize()
    toks = sorted({0, M - 1, M // 2})
    for m, y in zip(layer, Ys):
        w, s, b = (t.cpu().numpy() for t in m["ref"])
        s16, b16 = s.view(np.uint16), b.view(np.uint16)
        for t in toks:
            x32 = X[m["cols"]][t].float().cpu().numpy()
            ref = O.matvec_fmt_mt("int4", w.view(np.uint32), s16, b16, 1.0, 128, x32, m["rows"], m["cols"], 8)
            assert_close_out(to_np(y[t]), ref.astype(np.float64), "f32")


@pytest.mark.parametrize("fmt,n,k", [("q4k", 4096, 4096),
                                     ("q3k", 8192, 8192), ("q3k", 1024, 8192), ("q3k", 28672, 8192),
                                     ("q3k", 8192, 28672), ("int2", 8192, 8192), ("int2", 1024, 8192),
                                     ("int2", 28672, 8192), ("int2", 8192, 28672)])
@pytest.mark.parametrize("M", [1, 4])
def test_kquant_int2_full_size(fmt, n, k, M):
    """The Q4_K 4096^2 and Llama-3-70B Q3_K / INT2 g64 benchmark shapes (tiled
    layout, fp16 tokens) against the oracle's fp32 GEMV of the same REF bytes
    (ggml block formats; dequant.cu:110-172 for INT2) for every output row."""
    import bench
    gen = torch.Generator(device="cuda").manual_seed(n + k + M)
    if fmt == "int2":
        (m,) = bench.make_int4_layer(gen, gs=64, bits=2, shapes=[("w", n, k)])
        W = tq.QWeight(tq.INT2, tq.LAYOUT_TILED, n, k, m["tiled"], group_size=64)
        w, s, b = (t.cpu().numpy() for t in m["ref"])
        codes, s16, b16, gs = w.view(np.uint32), s.view(np.uint16), b.view(np.uint16), 64
    else:
        f = tq.Q4_K if fmt == "q4k" else tq.Q3_K
        blk = bench.random_kquant(f, n, k, gen)
        W = tq.QWeight(f, tq.LAYOUT_TILED, n, k, torch.from_numpy(tq.repack_host(f, n, k, blk)).cuda())
        codes, s16, b16, gs = blk, None, None, 0
    x = torch.randn(M, k, generator=gen, device="cuda").half()
    y = tq.qgemm(W, x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for t in sorted({0, M - 1}):
        ref = O.matvec_fmt_mt(fmt, codes, s16, b16, 1.0, gs, x[t].float().cpu().numpy(), n, k, 8)
        assert_close_out(to_np(y[t]), ref.astype(np.float64), "f32")


@pytest.mark.parametrize("fmt", ["q4k", "q3k"])
@pytest.mark.parametrize("M", [1, 4])
def test_kquant_llama8b_layer_full_size(fmt, M):
    """The Llama-3-8B layer in Q4_K / Q3_K (bench's synthetic K-quant layer,
    one batched launch): the 14336-column rows run with the per-format K split
    the launch heuristics pick at this shape; every output of the first and
    last token against the oracle's fp32 GEMV of the same ggml bytes."""
    import bench
    f = tq.Q4_K if fmt == "q4k" else tq.Q3_K
    gen = torch.Generator(device="cuda").manual_seed(21 + M + f)
    blks = [bench.random_kquant(f, n, k, gen) for _, n, k in bench.LLAMA8B]
    Ws = [tq.QWeight(f, tq.LAYOUT_TILED, n, k, torch.from_numpy(tq.repack_host(f, n, k, b)).cuda())
          for (_, n, k), b in zip(bench.LLAMA8B, blks)]
    X = {k: torch.randn(M, k, generator=gen, device="cuda").half() for k in (4096, 14336)}
    Xs = [X[k] for _, _, k in bench.LLAMA8B]
    Ys = [torch.empty(M, n, device="cuda", dtype=torch.float32) for _, n, _ in bench.LLAMA8B]
    tq.qgemm_batched(Ws, Xs, Ys)
    torch.cuda.synchronize()
    for (_, n, k), b, y in zip(bench.LLAMA8B, blks, Ys):
        for t in sorted({0, M - 1}):
            ref = O.matvec_fmt_mt(fmt, b, None, None, 1.0, 0, X[k][t].float().cpu().numpy(), n, k, 8)
            assert_close_out(to_np(y[t]), ref.astype(np.float64), "f32")


# chunk counts that end inside a group of 4 chunks (ragged), rows long enough
# to need two activation phases at one token, and the doubled stage of small
# multi-phase launches
RAGGED = {"int4": [(48, 640, 128), (48, 17024, 128)], "int2": [(48, 1280, 64), (32, 17152, 64)],
          "fp4": [(32, 640, 64)], "nvfp4": [(48, 640, 16), (32, 16512, 16)],
          "q4k": [(32, 768, 256), (32, 16640, 256)], "q3k": [(32, 1280, 256), (16, 16640, 256)],
          "fp8": [(32, 320, 0)]}


@pytest.mark.parametrize("fmt,rows,cols,gs", [(f, r, c, g) for f, v in RAGGED.items() for r, c, g in v])
@pytest.mark.parametrize("M", [1, 3, 8])
def test_tiled_ragged_and_multi_phase(fmt, rows, cols, gs, M, rng):
    """Rows whose chunks end inside a group (the loads past the row read zeros
    through the code plane's range check and their results are discarded) and
    rows folded in several activation phases, every tiled format, against the
    fp64 product of the oracle's exact dequantized weights."""
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    W = upload(d, tq.LAYOUT_TILED)
    x, x64 = act(M, cols, "f16", rng)
    y = tq.qgemm(W, x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close_out(to_np(y), x64 @ d["deq"].astype(np.float64).T, "f32")


@pytest.mark.parametrize("M", [1, 4])
def test_batched_exact_and_ragged_mix(M, rng):
    """One batched launch whose problems are partly whole groups and partly
    ragged (the launch takes the general kernel), with different K."""
    shapes = [(64, 4096), (48, 640), (32, 2048), (16, 896)]
    ds = [make_weights("int4", r, c, rng, gs=128) for r, c in shapes]
    Ws = [upload(d, tq.LAYOUT_TILED) for d in ds]
    X = [act(M, c, "f16", rng) for _, c in shapes]
    Ys = [torch.zeros(M, r, dtype=torch.float32, device="cuda") for r, _ in shapes]
    tq.qgemm_batched(Ws, [x for x, _ in X], Ys)
    torch.cuda.synchronize()
    for d, (_, x64), Y in zip(ds, X, Ys):
        assert_close_out(to_np(Y), x64 @ d["deq"].astype(np.float64).T, "f32")


@pytest.mark.parametrize("fmt,M", [("int2", 1), ("int2", 4), ("q3k", 1)])
def test_tail_split_eight_problem_batch(fmt, M):
    """Eight 2304 x 8192 problems in one launch: each takes a two-wave K split
    (72 workgroups, 576 in all), so the last 64 workgroups, the tail of the
    last problem, are re-split into one-tile workgroups and that problem into
    two (nine problems in the launch).  Every output of the first and last
    token against the oracle's fp32 GEMV of the same bytes."""
    import bench
    n, k = 2304, 8192
    gen = torch.Generator(device="cuda").manual_seed(77 + M)
    Ws, refs = [], []
    for _ in range(8):
        if fmt == "int2":
            (m,) = bench.make_int4_layer(gen, gs=64, bits=2, shapes=[("w", n, k)])
            Ws.append(tq.QWeight(tq.INT2, tq.LAYOUT_TILED, n, k, m["tiled"], group_size=64))
            w, s, b = (t.cpu().numpy() for t in m["ref"])
            refs.append((w.view(np.uint32), s.view(np.uint16), b.view(np.uint16), 64))
        else:
            blk = bench.random_kquant(tq.Q3_K, n, k, gen)
            Ws.append(tq.QWeight(tq.Q3_K, tq.LAYOUT_TILED, n, k,
                                 torch.from_numpy(tq.repack_host(tq.Q3_K, n, k, blk)).cuda()))
            refs.append((blk, None, None, 0))
    X = [torch.randn(M, k, generator=gen, device="cuda").half() for _ in range(8)]
    Ys = [torch.empty(M, n, device="cuda", dtype=torch.float32) for _ in range(8)]
    tq.qgemm_batched(Ws, X, Ys)
    torch.cuda.synchronize()
    for (codes, s16, b16, gs), x, y in zip(refs, X, Ys):
        for t in sorted({0, M - 1}):
            ref = O.matvec_fmt_mt(fmt, codes, s16, b16, 1.0, gs, x[t].float().cpu().numpy(), n, k, 8)
            assert_close_out(to_np(y[t]), ref.astype(np.float64), "f32")
