"""Weights read from checkpoint files and repacked at load time
(titan_ckpt_load_tiled) feed the GPU kernels: the products match the oracle's
restatement of the reference kernel for each stored format (NVFP4 from
safetensors, fp4.cu:187-252; Q4_K / Q3_K from GGUF; INT4 from titan-v1 blobs,
dequant.cu:23-104).  Tolerance: max |y - ref| <= 1e-3 * max |ref|."""
import numpy as np
import pytest
import torch

import titan_qmm as tq
from ckpt_files import int4_blob, write_gguf, write_safetensors, write_titan_v1
from helpers import assert_close_out
from oracle import oracle_ctypes as O

pytestmark = pytest.mark.gpu


def gemv(W, x32):
    x = torch.from_numpy(x32).cuda().half()
    y = tq.qgemm(W, x.unsqueeze(0), out_dtype=torch.float32)
    torch.cuda.synchronize()
    return y.cpu().numpy()[0].astype(np.float64), x.float().cpu().numpy().astype(np.float64)


def test_nvfp4_from_safetensors(tmp_path, rng):
    rows, cols = 256, 1024
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    g = float(np.abs(W).max() / (6.0 * 448.0))
    w, s = O.quantize_nvfp4(W, g)
    p = "model.layers.1.mlp.experts.7.down_proj"
    write_safetensors(tmp_path / "m.safetensors", {p + ".weight": ("U8", w.shape, w.tobytes()),
                                                  p + ".weight_scale": ("F8_E4M3", s.shape, s.tobytes()),
                                                  p + ".weight_scale_2": ("F32", [], np.float32(g).tobytes())})
    with tq.Checkpoint(tmp_path / "m.safetensors") as ck:
        Wd = ck.load_weight(p)
    x32 = rng.normal(0, 1, cols).astype(np.float32)
    y, x16 = gemv(Wd, x32)
    assert_close_out(y, O.dequant_nvfp4(w, s, g, rows, cols).astype(np.float64) @ x16, "f32")
    assert_close_out(y, O.matvec_nvfp4(w, s, g, x16.astype(np.float32), rows, cols).astype(np.float64), "f32")


@pytest.mark.parametrize("typ", [12, 11])
def test_kquant_from_gguf(tmp_path, rng, typ):
    rows, cols = 64, 2048
    Wf = rng.normal(0, 0.02, (rows, cols))
    blocks = O.quantize_q4k(Wf) if typ == 12 else O.quantize_q3k(Wf)
    write_gguf(tmp_path / "m.gguf", [("blk.3.ffn_up.weight", typ, [cols, rows], blocks.tobytes())],
               [("general.alignment", 4, 64)], alignment=64)
    with tq.Checkpoint(tmp_path / "m.gguf") as ck:
        Wd = ck.load_weight("blk.3.ffn_up.weight")
    deq = O.dequant_q4k(blocks, rows, cols) if typ == 12 else O.dequant_q3k(blocks, rows, cols)
    y, x16 = gemv(Wd, rng.normal(0, 1, cols).astype(np.float32))
    assert_close_out(y, deq.astype(np.float64) @ x16, "f32")


def test_int4_from_titan_v1(tmp_path, rng):
    rows, cols, gs = 128, 4096, 128
    w, s, b = O.quantize_int4(rng.normal(0, 0.02, (rows, cols)), gs)
    name = "model.layers.0.self_attn.o_proj.weight"
    write_titan_v1(tmp_path, {"files": {"attention": ("attention.bin", [
        (name, "int4", (rows, cols), int4_blob(w, s, b), gs)])}})
    with tq.Checkpoint(tmp_path) as ck:
        Wd = ck.load_weight(name)
    y, x16 = gemv(Wd, rng.normal(0, 1, cols).astype(np.float32))
    assert_close_out(y, O.dequant_int4(w, s, b, rows, cols, gs).astype(np.float64) @ x16, "f32")
    ref = O.matvec_int4_cpu(w, s, b, x16.astype(np.float32), rows, cols, gs)   # matmul_avx.cpp:54-100 order
    assert_close_out(y, ref.astype(np.float64), "f32")
