"""GPU-side helpers for the parity tests: upload oracle-made weights in either
layout and run the library through its C ABI."""
import numpy as np
import torch

import titan_qmm as tq

FMTS = {"int4": tq.INT4, "int2": tq.INT2, "fp4": tq.FP4, "nvfp4": tq.NVFP4,
        "q4k": tq.Q4_K, "q3k": tq.Q3_K, "fp8": tq.FP8_E4M3}
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def upload(d, layout):
    """Weight dict from helpers.make_weights -> tq.QWeight on cuda:0."""
    f = FMTS[d["fmt"]]
    rows, cols = d["rows"], d["cols"]
    gs = d["gs"] if d["fmt"] in ("int4", "int2", "fp4") else 0
    if layout == tq.LAYOUT_REF:
        return tq.QWeight(f, layout, rows, cols, dev(d["codes"]),
                          None if d["scales"] is None else dev(d["scales"]),
                          None if d["biases"] is None else dev(d["biases"]),
                          group_size=gs, global_scale=d["g"])
    scales = None if d["fmt"] == "fp8" else d["scales"]
    t = tq.repack_host(f, rows, cols, d["codes"], scales, d["biases"], gs)
    return tq.QWeight(f, layout, rows, cols, dev(t),
                      dev(d["scales"]) if d["fmt"] == "fp8" else None, None,
                      group_size=gs, global_scale=d["g"])


def act(M, K, dt, rng):
    """x ~ N(0, 1) rounded to dtype dt; returns (torch cuda tensor, exact fp64 numpy)."""
    x = torch.from_numpy(rng.normal(0, 1, (M, K)).astype(np.float32)).to(TDT[dt])
    return x.cuda(), x.double().numpy()


def to_np(t):
    return t.float().cpu().numpy().astype(np.float64)
