"""Shared test helpers: synthetic weights per format and tolerance checks."""
import numpy as np

from oracle import oracle_ctypes as O

# tolerance of the north star: max relative error 1e-3, normalised by max|ref|,
# for fp32-accumulated outputs; outputs rounded to fp16/bf16 may in addition
# differ from the rounded reference by one unit in the last place.
REL_TOL = 1e-3


def ulp(v, dtype):
    a = np.abs(np.asarray(v, np.float64))
    if dtype == "f32":
        m, emin = 24, -126
    elif dtype == "f16":
        m, emin = 11, -14
    else:
        m, emin = 8, -126
    e = np.floor(np.log2(np.maximum(a, 2.0 ** emin)))
    return 2.0 ** (e - (m - 1))


def round_to(v, dtype):
    v = np.asarray(v, np.float64)
    if dtype == "f32":
        return v.astype(np.float32).astype(np.float64)
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float64)
    import torch
    return torch.from_numpy(v.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def max_rel_err(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-30)
    return float(np.abs(y - ref).max() / scale)


def assert_close_out(y, ref, out_dtype, tol=REL_TOL):
    """y (GPU result in out_dtype) against ref (fp64 or fp32 exact-ish)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    r = round_to(ref, out_dtype)
    scale = max(np.abs(ref).max(), 1e-30)
    allowed = np.maximum(tol * scale, ulp(ref, out_dtype) * 1.0001)
    bad = np.abs(y - r) > allowed
    assert not bad.any(), (
        f"{bad.sum()} / {bad.size} outside tolerance; max rel err "
        f"{np.abs(y - r).max() / scale:.3e} (tol {tol})")
    return float(np.abs(y - ref).max() / scale)


def make_weights(fmt, rows, cols, rng, gs=128, sigma=0.02):
    """Quantize N(0, sigma) weights with the oracle's producer.  Returns a dict
    of REF-layout numpy arrays plus the exact dequantized matrix."""
    W = rng.normal(0.0, sigma, (rows, cols)).astype(np.float32)
    d = {"fmt": fmt, "rows": rows, "cols": cols, "gs": gs, "g": 1.0,
         "codes": None, "scales": None, "biases": None}
    if fmt == "int4":
        w, s, b = O.quantize_int4(W, gs)
        d.update(codes=w, scales=s, biases=b, deq=O.dequant_int4(w, s, b, rows, cols, gs))
    elif fmt == "int2":
        w, s, b = O.quantize_int2(W, gs)
        d.update(codes=w, scales=s, biases=b, deq=O.dequant_int2(w, s, b, rows, cols, gs))
    elif fmt == "fp4":
        w, s = O.quantize_fp4(W, gs)
        d.update(codes=w, scales=s, deq=O.dequant_fp4(w, s, rows, cols, gs))
    elif fmt == "nvfp4":
        g = float(np.abs(W).max() / (6.0 * 448.0))
        w, s = O.quantize_nvfp4(W, g)
        d.update(codes=w, scales=s, g=g, gs=16, deq=O.dequant_nvfp4(w, s, g, rows, cols))
    elif fmt == "q4k":
        blk = O.quantize_q4k(W)
        d.update(codes=blk, gs=256, deq=O.dequant_q4k(blk, rows, cols))
    elif fmt == "q3k":
        blk = O.quantize_q3k(W)
        d.update(codes=blk, gs=256, deq=O.dequant_q3k(blk, rows, cols))
    elif fmt == "fp8":
        w, s = O.quantize_fp8_rows(W)
        d.update(codes=w, scales=s, gs=0, deq=O.dequant_fp8(w, s, rows, cols))
    else:
        raise ValueError(fmt)
    d["W"] = W
    return d
