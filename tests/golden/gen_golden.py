"""Writes the committed golden fixtures tests/golden/<fmt>_<rows>x<cols>.npz.

Each fixture holds, for one format and shape: the packed REF-layout weights
(codes / scales / biases / global scale) made by the oracle's producer from
seeded N(0, 0.02) weights, the exact dequantized matrix as fp32 bit patterns,
two fp16-valued activation rows and their fp64 product with the dequantized
matrix.  For INT4 it also holds the output of the reference's own CPU GEMV
(matmul_avx.cpp:54-100, built from the reference sources into oracle/_ref),
which at generation time must equal the oracle's restatement bit for bit.

Run from the repository root:  python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import oracle_ctypes as O  # noqa: E402
import helpers  # noqa: E402

FORMATS = ["int4", "int2", "fp4", "nvfp4", "q4k", "q3k", "fp8"]
SHAPES = [(4, 512), (16, 1024)]
GS = {"int4": 128, "int2": 64, "fp4": 64}


def fixture(fmt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    d = helpers.make_weights(fmt, rows, cols, rng, gs=GS.get(fmt, 128))
    x = rng.normal(0, 1, (2, cols)).astype(np.float16).astype(np.float32)
    deq = np.asarray(d["deq"], np.float32).reshape(rows, cols)
    out = dict(fmt=np.array(fmt), rows=np.int32(rows), cols=np.int32(cols),
               gs=np.int32(d["gs"]), g=np.float32(d["g"]), seed=np.int64(seed),
               codes=np.ascontiguousarray(d["codes"]),
               deq_bits=deq.view(np.uint32), x=x,
               y_f64=x.astype(np.float64) @ deq.astype(np.float64).T)
    if d["scales"] is not None:
        out["scales"] = np.ascontiguousarray(d["scales"])
    if d["biases"] is not None:
        out["biases"] = np.ascontiguousarray(d["biases"])
    if rows * cols <= 4 * 512:
        out["W"] = d["W"]
    if fmt == "int4":
        y_or = O.matvec_int4_cpu(d["codes"], d["scales"], d["biases"], x[0], rows, cols, d["gs"])
        if O.ref_lib() is not None:
            y_ref = O.ref_matvec_int4(d["codes"], d["scales"], d["biases"], x[0], rows, cols,
                                      d["gs"])
            assert np.array_equal(np.asarray(y_ref, np.float32).view(np.uint32),
                                  np.asarray(y_or, np.float32).view(np.uint32)), \
                "oracle INT4 CPU GEMV differs from the reference build"
        out["y_cpu_ref_bits"] = np.asarray(y_or, np.float32).view(np.uint32)
    return out


def main():
    O.build()
    for i, fmt in enumerate(FORMATS):
        for j, (r, c) in enumerate(SHAPES):
            f = fixture(fmt, r, c, seed=1000 + 10 * i + j)
            path = os.path.join(HERE, f"{fmt}_{r}x{c}.npz")
            np.savez_compressed(path, **f)
            print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
