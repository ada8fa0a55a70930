"""GPU parity of the FP8 prefill path and the MoE routing / epilogue kernels."""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from helpers import assert_close_out, max_rel_err
from gpu_util import dev, to_np

from oracle import oracle_ctypes as O

pytestmark = pytest.mark.gpu


def bf16_bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M,K", [(1, 256), (7, 4096), (64, 1000), (5, 1003)])
def test_fp8_quantize_rows_bit_exact(M, K, dt):
    # bf16 values are exact in fp16 (|x| > 2^-14 here) and fp32, so every
    # input dtype has the same answer; K = 1003 takes the unvectorised path
    g = torch.Generator().manual_seed(M * 7 + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    x[x.abs() < 2 ** -12] = 0
    x[0, :5] = 0  # partial zeros; an all-zero row below
    if M > 2:
        x[2] = 0
    xd = x.to({"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]).cuda()
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(M, dtype=torch.float32, device="cuda")
    tq.fp8_quantize_rows(xd, xq, xs)
    torch.cuda.synchronize()
    q, s = O.quantize_act_fp8(bf16_bits(x))
    assert np.array_equal(xq.cpu().numpy(), q)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), s.view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(128, 128, 128), (256, 384, 512), (128, 256, 1024)])
def test_fp8_gemm_parity(M, N, K, rng):
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    wq, sw = O.quantize_fp8_rows(W)
    x = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float32)).to(torch.bfloat16)
    aq, sa = O.quantize_act_fp8(bf16_bits(x))
    ref = O.gemm_fp8(aq, sa, wq, sw).astype(np.float64)
    t = O.e4m3_ref_table().astype(np.float64)
    ref64 = (t[aq] @ t[wq].T) * sa[:, None].astype(np.float64) * sw[None, :]
    assert max_rel_err(ref, ref64) < 1e-5
    for odt, tdt in [("bf16", torch.bfloat16), ("f32", torch.float32)]:
        out = torch.empty(M, N, dtype=tdt, device="cuda")
        tq.fp8_gemm(dev(aq), dev(sa), dev(wq), dev(sw), out)
        torch.cuda.synchronize()
        assert_close_out(to_np(out), ref64, odt)


def test_fp8_gemm_rejects_untiled_shapes():
    L = tq.lib()
    a = torch.zeros(100, 128, dtype=torch.uint8, device="cuda")
    s = torch.ones(128, device="cuda")
    o = torch.zeros(100, 128, device="cuda")
    st = L.titan_fp8_gemm(tq._ptr(a), tq._ptr(s), tq._ptr(a), tq._ptr(s), tq._ptr(o), tq.FP32,
                          100, 128, 128, None)
    assert st == tq.ERR_UNSUPPORTED


def test_moe_gate_and_topk(rng):
    E, hd, k = 256, 7168, 8
    h = rng.normal(0, 1, hd).astype(np.float32)
    G = rng.normal(0, 0.02, (E, hd)).astype(np.float32)
    logits = torch.empty(E, device="cuda")
    tq.moe_gate(dev(h), dev(G), logits)
    torch.cuda.synchronize()
    ref = O.gemm_f64(G, h)[0]
    assert max_rel_err(logits.cpu().numpy(), ref) < 1e-5
    lg = logits.cpu().numpy()
    w = torch.empty(k, device="cuda")
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    tq.moe_topk(logits, w, idx, k)
    torch.cuda.synchronize()
    w_ref, i_ref = O.moe_topk(lg, k)
    assert idx.cpu().numpy().tolist() == i_ref.tolist()
    assert np.allclose(w.cpu().numpy(), w_ref, rtol=1e-5, atol=0)


def test_moe_topk_batched_and_ties(rng):
    T, E, k = 64, 256, 8
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    logits[0, :] = 0.0           # all tied: lowest indices win
    logits[1, [5, 9, 200]] = 7.0  # exact ties at the top
    ld = dev(logits)
    w = torch.empty(T, k, device="cuda")
    idx = torch.empty(T, k, dtype=torch.int32, device="cuda")
    tq.moe_topk_batched(ld, w, idx, k)
    torch.cuda.synchronize()
    wi, ii = w.cpu().numpy(), idx.cpu().numpy()
    for t in range(T):
        w_ref, i_ref = O.moe_topk(logits[t], k)
        assert ii[t].tolist() == i_ref.tolist(), t
        assert np.allclose(wi[t], w_ref, rtol=1e-5)
    assert ii[0].tolist() == list(range(8))
    assert ii[1, :3].tolist() == [5, 9, 200]


def test_swiglu_and_combine_bit_exact(rng):
    n = 5000
    g = rng.normal(0, 2, n).astype(np.float32)
    u = rng.normal(0, 1, n).astype(np.float32)
    out = torch.empty(n, device="cuda")
    tq.swiglu(out, dev(g), dev(u))
    torch.cuda.synchronize()
    assert max_rel_err(out.cpu().numpy(), O.swiglu(g, u)) < 1e-6
    dim, na = 7168, 8
    res = rng.normal(0, 1, dim).astype(np.float32)
    eo = rng.normal(0, 1, (na, dim)).astype(np.float32)
    wts = rng.uniform(0, 1, na).astype(np.float32)
    sh = rng.normal(0, 1, dim).astype(np.float32)
    for shared in (None, sh):
        rd = dev(res)
        o = torch.empty(dim, device="cuda")
        tq.fused_moe_combine_norm(o, rd, dev(eo), dev(wts), None if shared is None else dev(shared),
                                  1.0, dim, na)
        torch.cuda.synchronize()
        o_ref, r_ref = O.moe_combine(res, eo, wts, shared, 1.0)
        assert np.array_equal(o.cpu().numpy(), o_ref)
        assert np.array_equal(rd.cpu().numpy(), r_ref)


def test_quantize_fp4_bit_exact(rng):
    numel, gs = 64 * 256, 64
    v = rng.normal(0, 1, numel).astype(np.float32)
    v[:gs] = 0  # a zero group takes the 1e-10 floor
    out = torch.zeros(numel // 8, dtype=torch.int32, device="cuda")
    sc = torch.zeros(numel // gs, dtype=torch.float16, device="cuda")
    tq.quantize_fp4(dev(v), out, sc, numel, gs)
    torch.cuda.synchronize()
    w_ref, s_ref = O.quantize_fp4(v.reshape(1, -1), gs)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), w_ref.ravel())
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), s_ref.ravel())


@pytest.mark.parametrize("M,N,K", [(2048, 14336, 4096), (2048, 4096, 14336), (512, 2048, 1024)])
def test_fp8_gemm_full_size(M, N, K):
    """The benchmark shapes (256x256 and 256x128 tiles; the small one takes
    128x128 tiles): every output against a GPU fp32 product of the same e4m3
    operands, and 8 sampled rows against the oracle (dequant.cu FP8 semantics,
    fp32 accumulation).  Tolerance: max |out - ref| <= 1e-3 * max |ref| (bf16)."""
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    W = torch.randn(N, K, generator=g, device="cuda") * 0.02
    sw = (W.abs().amax(1) / 448.0).float()
    wq = (W / sw[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    sa = torch.empty(M, device="cuda")
    tq.fp8_quantize_rows(x, xq, sa)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    tq.fp8_gemm(xq, sa, wq, sw, out)
    torch.cuda.synchronize()
    table = torch.from_numpy(O.e4m3_ref_table()).cuda()
    a32 = table[xq.long()] * sa[:, None]
    w32 = table[wq.long()] * sw[:, None]
    ref = (a32 @ w32.T).double()
    assert_close_out(out.float().double().cpu().numpy(), ref.cpu().numpy(), "bf16")
    rows = np.random.default_rng(0).choice(M, 8, replace=False)
    o8 = O.gemm_fp8(xq.cpu().numpy()[rows], sa.cpu().numpy()[rows], wq.cpu().numpy(), sw.cpu().numpy())
    assert_close_out(out.float().double().cpu().numpy()[rows], o8.astype(np.float64), "bf16")


def e4m3_conversion_cases():
    """fp32 values that pin an e4m3 conversion: every finite code value, every
    midpoint between neighbours (ties to even) and the fp32 values one ulp
    either side, the subnormal range, signed zeros, a NaN, random values."""
    vals = O.e4m3_ref_table()
    pos = np.unique(vals[np.isfinite(vals) & (vals >= 0) & (vals <= 448)])
    mids = (pos[:-1].astype(np.float64) + pos[1:]) / 2
    mids = mids.astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    dn = np.nextafter(mids, np.float32(-np.inf))
    rnd = np.random.default_rng(5).uniform(0, 448, 4000).astype(np.float32)
    tiny = np.array([2.0 ** -10, 2.0 ** -10 * 1.0000001, 2.0 ** -11, 2.0 ** -30, 0.0], np.float32)
    p = np.concatenate([pos, mids, up, dn, rnd, tiny]).astype(np.float32)
    out = np.concatenate([p, -p, np.array([np.nan, -0.0], np.float32)])
    return out[(out <= 448) | np.isnan(out)]


def test_fp8_quantize_rows_conversion_exhaustive():
    """titan_fp8_quantize_rows on fp32 rows whose largest magnitude is 448
    (scale exactly 1): every other element is converted as it is, and must
    give the oracle's RNE e4m3 code (fp4.cu-style saturation, NaN -> 0x7F)."""
    v = e4m3_conversion_cases()
    K = 1024
    rows = -(-len(v) // (K - 1))
    x = np.zeros((rows, K), np.float32)
    flat = np.concatenate([v, np.zeros(rows * (K - 1) - len(v), np.float32)])
    x[:, 1:] = flat.reshape(rows, K - 1)
    x[:, 0] = 448.0
    xd = torch.from_numpy(x).cuda()
    xq = torch.empty(rows, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(rows, dtype=torch.float32, device="cuda")
    tq.fp8_quantize_rows(xd, xq, xs)
    torch.cuda.synchronize()
    assert np.all(xs.cpu().numpy() == 1.0)
    want = O.f32_to_e4m3(x.reshape(-1)).reshape(rows, K)
    got = xq.cpu().numpy()
    bad = np.nonzero(got != want)
    assert bad[0].size == 0, [(float(x[i, j]), int(got[i, j]), int(want[i, j])) for i, j in zip(*bad)][:10]
