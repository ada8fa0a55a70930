"""Golden fixtures (tests/golden/*.npz, written by tests/golden/gen_golden.py).

CPU: the oracle reproduces every fixture bit for bit (producer, dequantizer,
and for INT4 the reference's own CPU GEMV output).  GPU: the HIP library,
through its C ABI, dequantizes every fixture bit-exactly in both layouts and
its GEMV matches the fixture's fp64 product within the north-star tolerance.
"""
import glob
import os

import numpy as np
import pytest

from oracle import oracle_ctypes as O
import helpers

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def as_weights(f):
    fmt = str(f["fmt"])
    return {"fmt": fmt, "rows": int(f["rows"]), "cols": int(f["cols"]), "gs": int(f["gs"]),
            "g": float(f["g"]), "codes": f["codes"], "scales": f.get("scales"),
            "biases": f.get("biases")}


def oracle_deq(d):
    fmt, r, c, gs = d["fmt"], d["rows"], d["cols"], d["gs"]
    if fmt == "int4":
        return O.dequant_int4(d["codes"], d["scales"], d["biases"], r, c, gs)
    if fmt == "int2":
        return O.dequant_int2(d["codes"], d["scales"], d["biases"], r, c, gs)
    if fmt == "fp4":
        return O.dequant_fp4(d["codes"], d["scales"], r, c, gs)
    if fmt == "nvfp4":
        return O.dequant_nvfp4(d["codes"], d["scales"], d["g"], r, c)
    if fmt == "q4k":
        return O.dequant_q4k(d["codes"], r, c)
    if fmt == "q3k":
        return O.dequant_q3k(d["codes"], r, c)
    return O.dequant_fp8(d["codes"], d["scales"], r, c)


def test_fixtures_present():
    fmts = {os.path.basename(p).split("_")[0] for p in FIXTURES}
    assert fmts == {"int4", "int2", "fp4", "nvfp4", "q4k", "q3k", "fp8"}


@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_oracle_reproduces_fixture(path):
    f = load(path)
    d = as_weights(f)
    deq = np.asarray(oracle_deq(d), np.float32).reshape(d["rows"], d["cols"])
    assert np.array_equal(deq.view(np.uint32), f["deq_bits"])
    if "W" in f:  # the producer is deterministic
        again = helpers.make_weights(d["fmt"], d["rows"], d["cols"],
                                     np.random.default_rng(int(f["seed"])), gs=d["gs"] or 128)
        assert np.array_equal(np.asarray(again["codes"]), f["codes"])
    if d["fmt"] == "int4":
        y = O.matvec_int4_cpu(d["codes"], d["scales"], d["biases"], f["x"][0], d["rows"],
                              d["cols"], d["gs"])
        assert np.array_equal(np.asarray(y, np.float32).view(np.uint32), f["y_cpu_ref_bits"])
    # the fp64 product is the dequantized matrix times the activations
    y64 = f["x"].astype(np.float64) @ deq.astype(np.float64).T
    np.testing.assert_allclose(y64, f["y_f64"], rtol=0, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=[os.path.basename(p) for p in FIXTURES])
def test_gpu_matches_fixture(path):
    import torch
    import titan_qmm as tq
    import gpu_util as G
    f = load(path)
    d = as_weights(f)
    layouts = [tq.LAYOUT_REF]
    if tq.tiled_bytes(G.FMTS[d["fmt"]], d["rows"], d["cols"], d["gs"]):
        layouts.append(tq.LAYOUT_TILED)
    for layout in layouts:
        W = G.upload(d, layout)
        deq = tq.qdequant(W).cpu().numpy()
        assert np.array_equal(deq.view(np.uint32), f["deq_bits"]), f"layout {layout}"
        x = torch.from_numpy(f["x"]).half().cuda()
        for odt in ("f32", "f16", "bf16"):
            y = tq.qgemm(W, x, out_dtype=G.TDT[odt])
            helpers.assert_close_out(G.to_np(y), f["y_f64"], odt)
