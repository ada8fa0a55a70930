"""Pins of the CPU oracle (oracle/qmm_oracle.c) -- CPU only.

Each check is chosen so that a plausible mistake in the oracle (wrong shift,
swapped nibble, transposed index, dropped term) fails it: independent
implementations (numpy/torch conversions, the reference's own compiled CPU
GEMV in oracle/_ref), known-answer blocks packed by an independent packer
written here from the ggml block layout, brute force in fp64, and
quantize->dequantize error bounds.
"""
import struct

import numpy as np
import pytest
import torch

from oracle import oracle_ctypes as O

L = O.lib()


# ---------------------------------------------------------------- conversions
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def test_f32_to_f16_rne(rng):
    v = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 1e-5, 2000),
                        rng.normal(0, 3e4, 2000), [65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8,
                                                   2.98e-8, 2.99e-8, -0.0]]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    got = np.array([L.or_f32_to_f16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_roundtrip_matches_torch(rng):
    v = np.concatenate([rng.normal(0, 1, 4000), rng.normal(0, 1e30, 100)]).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.or_f32_to_bf16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([L.or_bf16_to_f32(int(x)) for x in ref], np.float32)
    assert np.array_equal(back, torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_e4m3_decode_matches_torch_and_nan_rule():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_ref_table()
    nan = (codes & 0x7F) == 0x7F
    assert np.array_equal(got[~nan], ref[~nan])
    # fp4.cu:174: the two NaN codes decode to 0 in the reference decoder
    assert np.all(got[nan] == 0.0)
    ocp = np.array([L.or_e4m3_ocp_to_f32(int(c)) for c in codes], np.float32)
    assert np.all(np.isnan(ocp[nan])) and np.array_equal(ocp[~nan], ref[~nan])


def test_e4m3_encode_nearest_even(rng):
    # brute force: nearest representable finite e4m3 value, ties to even code
    table = O.e4m3_ref_table()
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F])
    v = np.concatenate([rng.normal(0, 1, 3000), rng.normal(0, 100, 1000), rng.normal(0, 0.01, 1000),
                        table[finite] + 1e-7, (table[finite[:-1]] + table[finite[1:]]) / 2,
                        [448.0, 464.0, 500.0, -1e9]]).astype(np.float32)
    got = O.f32_to_e4m3(v)
    for x, c in zip(v, got):
        a = min(abs(float(x)), 448.0)
        mags = table[:0x7F]
        d = np.abs(mags.astype(np.float64) - a)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
        assert (c & 0x7F) == want, (x, c, want)
    # agrees with torch's RNE conversion inside the finite range
    inr = np.abs(v) < 448
    t = torch.from_numpy(v[inr]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got[inr], t)


def test_fp4_lut_known_values():
    # fp4.cu:23-26
    want = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    got = [L.or_fp4_e2m1_to_f32(i) for i in range(16)]
    assert got == want
    assert struct.pack("<f", got[8]) == struct.pack("<f", -0.0)


# ---------------------------------------------------------------- INT4 / INT2
def test_int4_gemv_bit_exact_with_reference_cpu_build(rng):
    R = O.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    for rows, cols, gs in [(64, 1024, 64), (33, 512, 128), (8, 4096, 128), (5, 136, 8)]:
        W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
        w, s, b = O.quantize_int4(W, gs)
        x = rng.normal(0, 1, cols).astype(np.float32)
        y1 = O.matvec_int4_cpu(w, s, b, x, rows, cols, gs)
        y2 = O.ref_matvec_int4(w, s, b, x, rows, cols, gs)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_int4_dequant_equals_reference_one_hot(rng):
    """The reference GEMV with a one-hot x returns one dequantized column
    (acc = fma(w, 1, 0) = w exactly): pins or_dequant_int4 bit for bit."""
    R = O.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built")
    rows, cols, gs = 16, 256, 64
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    w, s, b = O.quantize_int4(W, gs)
    D = O.dequant_int4(w, s, b, rows, cols, gs)
    for c in [0, 1, 7, 8, 63, 64, 129, 255]:
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        col = O.ref_matvec_int4(w, s, b, x, rows, cols, gs)
        assert np.array_equal(col.view(np.uint32), D[:, c].view(np.uint32))


def test_int4_known_answer():
    # one row, 16 columns, group 8: word 0 = 0x76543210 (col n -> q n), word 1
    # = 0xFEDCBA98; group 0 scale 0.5 bias -1, group 1 scale 2 bias 0.25
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    s = np.array([[0x3800, 0x4000]], np.uint16)
    b = np.array([[0xBC00, 0x3400]], np.uint16)
    D = O.dequant_int4(w, s, b, 1, 16, 8)[0]
    want = [0.5 * q - 1 for q in range(8)] + [2.0 * q + 0.25 for q in range(8, 16)]
    assert D.tolist() == want


def test_int2_known_answer():
    w = np.array([[0b11100100 | (0b00011011 << 8) | (0xFF << 16)]], np.uint32)
    s = np.array([[0x3C00]], np.uint16)  # 1.0
    b = np.array([[0xC000]], np.uint16)  # -2.0
    D = O.dequant_int2(w, s, b, 1, 16, 16)[0]
    codes = [0, 1, 2, 3, 3, 2, 1, 0, 3, 3, 3, 3, 0, 0, 0, 0]
    assert D.tolist() == [c - 2.0 for c in codes]


def test_affine_quantize_error_bound(rng):
    W = rng.normal(0, 0.02, (32, 1024)).astype(np.float32)
    for fn, deq, levels in [(O.quantize_int4, O.dequant_int4, 15), (O.quantize_int2, O.dequant_int2, 3)]:
        w, s, b = fn(W, 64)
        D = deq(w, s, b, 32, 1024, 64)
        G = W.reshape(32, -1, 64)
        step = (G.max(-1) - G.min(-1)) / levels
        err = np.abs(D - W).reshape(32, -1, 64).max(-1)
        # half a step, plus the fp16 rounding of scale (x levels) and bias
        bound = step / 2 + levels * step * 2 ** -11 + np.abs(G.min(-1)) * 2 ** -11 + 1e-7
        assert np.all(err <= bound * 1.01)


# ---------------------------------------------------------------- FP4 / NVFP4
def test_nvfp4_known_answer():
    # byte 0x2F: low nibble 0xF (-6) is column 0, high nibble 0x2 (1.0) column 1
    # (fp4.cu:219-220); scale bytes 0x38 (1.0) for cols 0-15 and 0x40 (2.0) for
    # 16-31, global scale 0.5; the NaN scale code 0x7F reads as 0.
    w = np.zeros((1, 24), np.uint8)
    w[0, 0] = 0x2F
    w[0, 8] = 0x71      # cols 16, 17: lut 0.5 and 6.0 under scale 2 x 0.5
    w[0, 16] = 0x55     # cols 32, 33 under scale 0x7F
    s = np.array([[0x38, 0x40, 0x7F]], np.uint8)
    D = O.dequant_nvfp4(w, s, 0.5, 1, 48)[0]
    assert D[0] == -3.0 and D[1] == 0.5
    assert D[16] == 0.5 and D[17] == 6.0
    assert D[32] == 0.0 and D[33] == 0.0


def test_nvfp4_gemv_matches_fp64(rng):
    rows, cols = 16, 512
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    g = float(np.abs(W).max() / (6 * 448))
    w, s = O.quantize_nvfp4(W, g)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y = O.matvec_nvfp4(w, s, g, x, rows, cols)
    ref = O.gemm_f64(O.dequant_nvfp4(w, s, g, rows, cols), x)[0]
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # quantisation is faithful: within one e2m1 step of the block scale
    D = O.dequant_nvfp4(w, s, g, rows, cols)
    assert np.abs(D - W).max() < 0.35 * np.abs(W).max()


def test_fp4_quantizer_thresholds():
    # fp4.cu:118-135: amax/6 scale; thresholds .25/.75/1.25/1.75/2.5/3.5/5
    v = np.array([[6.0, 0.2, 0.3, -0.8, 1.3, 1.8, 2.6, 3.6]], np.float32)
    w, s = O.quantize_fp4(v, 8)
    assert O.f16_bits_to_f32(s)[0, 0] == 1.0
    codes = [(int(w[0, 0]) >> (4 * n)) & 0xF for n in range(8)]
    assert codes == [7, 0, 1, 8 | 2, 3, 4, 5, 6]


# ---------------------------------------------------------------- Q4_K / Q3_K
def pack_q4k_block(d, dmin, sc, mn, q):
    """Independent Q4_K packer from the ggml block layout: {f16 d, f16 dmin,
    u8 scales[12], u8 qs[128]}; sub-block j < 4 keeps its 6-bit scale/min in
    the low 6 bits of bytes j / j+4; j >= 4 keeps the low 4 bits in byte j+4
    (scale low nibble, min high nibble) and the top 2 bits in the top bits of
    bytes j-4 (scale) and j (min)."""
    sb = bytearray(12)
    for j in range(8):
        if j < 4:
            sb[j] |= sc[j] & 63
            sb[j + 4] |= mn[j] & 63
        else:
            sb[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
            sb[j - 4] |= (sc[j] >> 4) << 6
            sb[j] |= (mn[j] >> 4) << 6
    qs = bytearray(128)
    for e in range(256):
        c, r = divmod(e, 64)
        if r < 32:
            qs[32 * c + r] |= q[e]
        else:
            qs[32 * c + r - 32] |= q[e] << 4
    return (np.float16(d).tobytes() + np.float16(dmin).tobytes() + bytes(sb) + bytes(qs))


def q4k_expected(d, dmin, sc, mn, q):
    d32, m32 = np.float32(np.float16(d)), np.float32(np.float16(dmin))
    out = np.zeros(256, np.float32)
    for e in range(256):
        j = e // 32
        out[e] = np.float32(d32 * np.float32(sc[j])) * np.float32(q[e]) - np.float32(m32 * np.float32(mn[j]))
    return out


def test_q4k_known_answer_blocks(rng):
    cases = [
        (1.0, 0.0, list(range(1, 9)), [0] * 8, [e % 16 for e in range(256)]),
        (0.5, 0.25, [63, 1, 17, 32, 48, 5, 60, 33], [7, 63, 0, 40, 16, 49, 3, 62],
         list(rng.integers(0, 16, 256))),
        (2.0 ** -10, 3.0, [int(v) for v in rng.integers(0, 64, 8)],
         [int(v) for v in rng.integers(0, 64, 8)], list(rng.integers(0, 16, 256))),
    ]
    for d, dmin, sc, mn, q in cases:
        blk = np.frombuffer(pack_q4k_block(d, dmin, sc, mn, q), np.uint8)
        got = O.dequant_q4k(blk.reshape(1, 144), 1, 256)[0]
        assert np.array_equal(got, q4k_expected(d, dmin, sc, mn, q))


def test_q4k_every_scale_position():
    """Each sub-block's (scale, min) reaches exactly its own 32 elements."""
    for j in range(8):
        for val in (1, 15, 16, 48, 63):
            sc = [0] * 8
            mn = [0] * 8
            sc[j] = val
            blk = np.frombuffer(pack_q4k_block(1.0, 1.0, sc, mn, [1] * 256), np.uint8)
            got = O.dequant_q4k(blk.reshape(1, 144), 1, 256)[0]
            want = np.zeros(256, np.float32)
            want[32 * j:32 * j + 32] = val
            assert np.array_equal(got, want), (j, val)
            sc = [0] * 8
            mn[j] = val
            blk = np.frombuffer(pack_q4k_block(1.0, 1.0, sc, mn, [1] * 256), np.uint8)
            got = O.dequant_q4k(blk.reshape(1, 144), 1, 256)[0]
            want = np.zeros(256, np.float32)
            want[32 * j:32 * j + 32] = -val
            assert np.array_equal(got, want), (j, val)


def pack_q3k_block(d, sc, q):
    """Independent Q3_K packer: {u8 hmask[32], u8 qs[64], u8 scales[12], f16 d}.
    Element 128h + 32j + l: low 2 bits of (q + 4) at bits 2j of qs[32h + l],
    bit 2 of (q + 4) at bit 4h + j of hmask[l]; sub-block k = e // 16 uses
    6-bit scale sc[k] + 32 whose low nibble is in scales[k] (k < 8) or the
    high nibble of scales[k - 8], and whose top 2 bits are at bits 2*(k // 4)
    of scales[8 + k % 4]."""
    hm = bytearray(32)
    qs = bytearray(64)
    sb = bytearray(12)
    for e in range(256):
        h, r = divmod(e, 128)
        j, l = divmod(r, 32)
        u = q[e] + 4
        qs[32 * h + l] |= (u & 3) << (2 * j)
        if u & 4:
            hm[l] |= 1 << (4 * h + j)
    for k in range(16):
        u = sc[k] + 32
        if k < 8:
            sb[k] |= u & 15
        else:
            sb[k - 8] |= (u & 15) << 4
        sb[8 + k % 4] |= (u >> 4) << (2 * (k // 4))
    return bytes(hm) + bytes(qs) + bytes(sb) + np.float16(d).tobytes()


def test_q3k_known_answer_blocks(rng):
    for d in (1.0, 0.03125, 2.0 ** -12):
        sc = [int(v) for v in rng.integers(-32, 32, 16)]
        q = [int(v) for v in rng.integers(-4, 4, 256)]
        blk = np.frombuffer(pack_q3k_block(d, sc, q), np.uint8)
        got = O.dequant_q3k(blk.reshape(1, 110), 1, 256)[0]
        d32 = np.float32(np.float16(d))
        want = np.array([np.float32(d32 * np.float32(sc[e // 16])) * np.float32(q[e])
                         for e in range(256)], np.float32)
        assert np.array_equal(got, want)


def test_q3k_every_scale_position():
    for k in range(16):
        for val in (-32, -1, 1, 15, 16, 31):
            sc = [0] * 16
            sc[k] = val
            blk = np.frombuffer(pack_q3k_block(1.0, sc, [1] * 256), np.uint8)
            got = O.dequant_q3k(blk.reshape(1, 110), 1, 256)[0]
            want = np.zeros(256, np.float32)
            want[16 * k:16 * k + 16] = val
            assert np.array_equal(got, want), (k, val)


def test_kquant_quantize_error_bound(rng):
    W = rng.normal(0, 0.02, (8, 1024)).astype(np.float32)
    D4 = O.dequant_q4k(O.quantize_q4k(W), 8, 1024)
    D3 = O.dequant_q3k(O.quantize_q3k(W), 8, 1024)
    rng_w = np.abs(W).max()
    assert np.abs(D4 - W).max() < 0.12 * rng_w
    assert np.abs(D3 - W).max() < 0.35 * rng_w
    assert np.corrcoef(D4.ravel(), W.ravel())[0, 1] > 0.99
    assert np.corrcoef(D3.ravel(), W.ravel())[0, 1] > 0.95


# ---------------------------------------------------------------- FP8
def test_fp8_rows_and_act_quant(rng):
    W = rng.normal(0, 0.02, (8, 256)).astype(np.float32)
    w, s = O.quantize_fp8_rows(W)
    assert np.allclose(s, np.abs(W).max(1) / 448, rtol=0, atol=0)
    t = torch.from_numpy((W / s[:, None]).astype(np.float32)).to(torch.float8_e4m3fn)
    assert np.array_equal(w, t.view(torch.uint8).numpy())
    x = torch.randn(4, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    q, xs = O.quantize_act_fp8(xb)
    xf = x.float().numpy()
    assert np.array_equal(xs, (np.abs(xf).max(1) / np.float32(448)).astype(np.float32))
    want = torch.from_numpy((xf / xs[:, None]).astype(np.float32)).to(torch.float8_e4m3fn)
    assert np.array_equal(q, want.view(torch.uint8).numpy())


def test_fp8_gemm_reference_matches_fp64(rng):
    A = rng.integers(0, 256, (8, 128)).astype(np.uint8)
    A[(A & 0x7F) == 0x7F] = 0
    Wq = rng.integers(0, 256, (16, 128)).astype(np.uint8)
    Wq[(Wq & 0x7F) == 0x7F] = 0
    sa = rng.uniform(0.5, 2, 8).astype(np.float32)
    sw = rng.uniform(0.5, 2, 16).astype(np.float32)
    out = O.gemm_fp8(A, sa, Wq, sw)
    t = O.e4m3_ref_table().astype(np.float64)
    ref = (t[A] @ t[Wq].T) * sa[:, None] * sw[None, :]
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


# ---------------------------------------------------------------- dense / MoE
def test_gemm_f32_vs_f64(rng):
    W = rng.normal(0, 1, (16, 300)).astype(np.float32)
    X = rng.normal(0, 1, (3, 300)).astype(np.float32)
    a = O.gemm_f32(W, X)
    b = O.gemm_f64(W, X)
    assert np.abs(a - b).max() < 1e-4
    assert np.allclose(b, X.astype(np.float64) @ W.astype(np.float64).T, rtol=1e-12, atol=1e-12)


def test_moe_topk_semantics():
    # hand-computed: softmax over all E, top-k with the lowest index on ties
    logits = np.array([0.0, 2.0, 1.0, 2.0, -1.0], np.float32)
    w, idx = O.moe_topk(logits, 3)
    assert idx.tolist() == [1, 3, 2]
    e = np.exp(logits - 2.0)
    p = e / (e.sum() + 1e-8)
    sel = p[[1, 3, 2]]
    assert np.allclose(w, sel / (sel.sum() + 1e-8), rtol=1e-6)
    # k = E returns every expert
    w, idx = O.moe_topk(logits, 5)
    assert sorted(idx.tolist()) == [0, 1, 2, 3, 4]
    assert abs(float(w.sum()) - 1.0) < 1e-6


def test_swiglu_and_combine():
    g = np.array([-2.0, 0.0, 1.0, 3.0], np.float32)
    u = np.array([1.0, 5.0, 2.0, -1.0], np.float32)
    out = O.swiglu(g, u)
    assert np.allclose(out, g / (1 + np.exp(-g)) * u, rtol=1e-6)
    res = np.array([1.0, 2.0], np.float32)
    eo = np.array([[1.0, 1.0], [2.0, -1.0]], np.float32)
    o, r = O.moe_combine(res, eo, np.array([0.25, 0.5], np.float32),
                         np.array([4.0, 8.0], np.float32), 1.0)
    assert o.tolist() == [1.0 + 0.25 + 1.0 + 4.0, 2.0 + 0.25 - 0.5 + 8.0]
    assert np.array_equal(o, r)


# ---------------------------------------------------------------- FP4 (fp16 group scale)
FP4_VALUES = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]


def test_fp4_known_answer_words_and_groups():
    """fp4.cu:28-84 by hand: nibble n of word p is column 8p+n, and the whole
    word takes the scale of group (8p) // group_size of its own row."""
    # row 0: word 0 = codes 0..7 ascending, word 1 = 15..8 descending,
    # word 2 = 0x7 in every nibble, word 3 = 0x9 (-0.5) in every nibble;
    # row 1: the same words rotated by one.
    words = [0x76543210, 0x89ABCDEF, 0x77777777, 0x99999999]
    w = np.array([words, words[1:] + words[:1]], np.uint32)
    # group 16 -> groups {word 0, word 1} and {word 2, word 3}: scales per row
    s = np.array([[0x3C00, 0x4000],     # 1.0, 2.0
                  [0x3800, 0x4400]],    # 0.5, 4.0
                 np.uint16)
    D = O.dequant_fp4(w, s, 2, 32, 16)
    want0 = ([FP4_VALUES[n] for n in range(8)] + [FP4_VALUES[15 - n] for n in range(8)]
             + [12.0] * 8 + [-1.0] * 8)
    want1 = ([0.5 * FP4_VALUES[15 - n] for n in range(8)] + [0.5 * 6.0] * 8
             + [-2.0] * 8 + [4.0 * FP4_VALUES[n] for n in range(8)])
    assert D[0].tolist() == want0
    assert D[1].tolist() == want1
    w = w[:, :3]
    want0 = want0[:24]
    # group 8 (one scale per word) and group 24 (all three words share one)
    s8 = np.array([[0x3C00, 0x4000, 0x3400]] * 2, np.uint16)   # 1, 2, 0.25
    D8 = O.dequant_fp4(w[:1], s8[:1], 1, 24, 8)[0]
    assert D8[:8].tolist() == want0[:8]
    assert D8[8:16].tolist() == [2.0 * FP4_VALUES[15 - n] for n in range(8)]
    assert D8[16:].tolist() == [1.5] * 8
    D24 = O.dequant_fp4(w[:1], np.array([[0x4000]], np.uint16), 1, 24, 24)[0]
    assert D24.tolist() == [2.0 * v for v in want0[:16]] + [12.0] * 8
    # a group size that is not a multiple of 8: word p uses group (8p) // 12,
    # so word 1 (columns 8..15) still takes group 0's scale
    s12 = np.array([[0x3C00, 0x4000]], np.uint16)
    D12 = O.dequant_fp4(w[:1], s12, 1, 24, 12)[0]
    assert D12[:16].tolist() == want0[:16]
    assert D12[16:].tolist() == [12.0] * 8
    # signed zero of code 8 survives the scale
    assert struct.pack("<f", float(D[0][8 + 7])) == struct.pack("<f", -0.0)


def test_fp4_quantize_dequantize_round_trip(rng):
    """Values on the E2M1 grid times a power-of-two group scale come back
    exactly through or_quantize_fp4 -> or_dequant_fp4 (scale = amax/6 is then
    exact in fp16); random values come back within one grid step."""
    rows, cols, gs = 8, 256, 32
    q = rng.integers(0, 16, (rows, cols))
    q[:, ::gs] = 7                                  # every group holds +6 -> amax = 6s
    scale = 2.0 ** rng.integers(-12, 3, (rows, cols // gs))
    W = (np.array(FP4_VALUES, np.float64)[q] * np.repeat(scale, gs, 1)).astype(np.float32)
    w, s = O.quantize_fp4(W, gs)
    D = O.dequant_fp4(w, s, rows, cols, gs)
    assert np.array_equal(D, W)
    Wr = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    w, s = O.quantize_fp4(Wr, gs)
    D = O.dequant_fp4(w, s, rows, cols, gs)
    sc = O.f16_bits_to_f32(s).astype(np.float64)
    amax = np.abs(Wr.reshape(rows, -1, gs)).max(-1)
    # the widest E2M1 gap is 2 (4 -> 6): half of it in units of the scale, plus
    # the fp16 rounding of the scale times the largest code
    bound = sc * 1.0 + 6 * np.abs(sc - amax / 6) + 1e-9
    err = np.abs(D - Wr).reshape(rows, -1, gs).max(-1)
    assert np.all(err <= bound)


# ---------------------------------------------------------------- per-format row GEMV
def _fmt_operands(fmt, rng, rows, cols):
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    z16 = np.zeros(1, np.uint16)
    if fmt == "int4":
        w, s, b = O.quantize_int4(W, 128)
        return (w, s, b, 1.0, 128), O.dequant_int4(w, s, b, rows, cols, 128)
    if fmt == "int2":
        w, s, b = O.quantize_int2(W, 64)
        return (w, s, b, 1.0, 64), O.dequant_int2(w, s, b, rows, cols, 64)
    if fmt == "nvfp4":
        g = float(np.abs(W).max() / (6 * 448))
        w, s = O.quantize_nvfp4(W, g)
        return (w, s, z16, g, 16), O.dequant_nvfp4(w, s, g, rows, cols)
    if fmt == "q4k":
        blk = O.quantize_q4k(W)
        return (blk, z16, z16, 1.0, 256), O.dequant_q4k(blk, rows, cols)
    if fmt == "q3k":
        blk = O.quantize_q3k(W)
        return (blk, z16, z16, 1.0, 256), O.dequant_q3k(blk, rows, cols)
    w, cs = O.quantize_fp8_rows(W)
    return (w, cs, z16, 1.0, 1), O.dequant_fp8(w, cs, rows, cols)


@pytest.mark.parametrize("fmt", ["int4", "int2", "nvfp4", "q4k", "q3k", "fp8"])
def test_matvec_fmt_mt_matches_fp64(fmt, rng):
    """or_matvec_fmt_mt (the reference for the full-size GPU GEMV tests) is
    the fp64 product of the exact dequantized matrix up to fp32 accumulation
    error; every row reads its own codes and scales (rows differ, so a wrong
    row stride fails), and the thread split does not change a bit."""
    rows, cols = 37, 1536
    (codes, s, b, g, gs), D = _fmt_operands(fmt, rng, rows, cols)
    x = rng.normal(0, 1, cols).astype(np.float32)
    y1 = O.matvec_fmt_mt(fmt, codes, s, b, g, gs, x, rows, cols, 1)
    ref = O.gemm_f64(D, x)[0]
    # fp32 accumulation of `cols` terms: |err| <= cols * 2^-24 * sum |w x|
    bound = cols * 2.0 ** -24 * (np.abs(D.astype(np.float64)) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y1 - ref) <= bound)
    assert np.abs(y1 - ref).max() <= 1e-5 * np.abs(ref).max()
    y5 = O.matvec_fmt_mt(fmt, codes, s, b, g, gs, x, rows, cols, 5)
    assert np.array_equal(y1.view(np.uint32), y5.view(np.uint32))
    # one-hot x returns one dequantized column exactly (fma(w, 1, 0) = w)
    for c in (0, 255, 256, cols - 1):
        e = np.zeros(cols, np.float32)
        e[c] = 1.0
        col = O.matvec_fmt_mt(fmt, codes, s, b, g, gs, e, rows, cols, 3)
        assert np.array_equal(col, D[:, c]), (fmt, c)
