"""CPU tests of the checkpoint readers and the load-time repack
(include/titan_ckpt.h; reference readers loader.cpp:36-472,
gguf_loader.cpp:60-342, moe.cpp:613-724, convert_titan.py:146-235).

Every quantized weight is checked byte-exactly: the TILED buffer that
titan_ckpt_load_tiled writes unpacks (titan_unpack_host) to exactly the bytes
stored in the file.  Plain tensors read back byte-exactly, and for the
standard dtypes the files written by the safetensors library itself are read
too."""
import json
import os
import struct

import numpy as np
import pytest

import titan_qmm as tq
from ckpt_files import (GGUF_ARR, GGUF_F32, GGUF_STR, GGUF_U32, GGUF_U64, int4_blob,
                        write_gguf, write_safetensors, write_titan_v1)
from oracle import oracle_ctypes as O


def nvfp4_parts(rows, cols, rng):
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    g = float(np.abs(W).max() / (6.0 * 448.0))
    w, s = O.quantize_nvfp4(W, g)
    return w, s, g


def check_tiled_roundtrip(ck, name, fmt, rows, cols, codes, scales=None, biases=None, gs=0):
    buf, info = ck.load_tiled(name)
    assert (info["fmt"], info["rows"], info["cols"]) == (fmt, rows, cols)
    assert info["tiled_bytes"] == tq.tiled_bytes(fmt, rows, cols, gs) == buf.nbytes
    c2, s2, b2 = tq.unpack_host(fmt, rows, cols, buf, codes, scales, biases, gs)
    assert np.array_equal(c2, codes)
    if scales is not None:
        assert np.array_equal(s2, scales)
    if biases is not None:
        assert np.array_equal(b2, biases)
    return info


def test_safetensors_nvfp4_experts(tmp_path, rng):
    base = "model.layers.0.mlp.experts.{}.{}_proj"
    parts, tensors = {}, {}
    for e, (proj, gmode) in enumerate([("gate", "f32"), ("up", "bf16"), ("down", "none")]):
        rows, cols = (256, 512) if proj != "down" else (512, 256)
        w, s, g = nvfp4_parts(rows, cols, rng)
        name = base.format(e, proj)
        parts[name] = (w, s, g, gmode, rows, cols)
        tensors[name + ".weight"] = ("U8", w.shape, w.tobytes())
        tensors[name + ".weight_scale"] = ("F8_E4M3", s.shape, s.tobytes())
        if gmode == "f32":
            tensors[name + ".weight_scale_2"] = ("F32", [], np.float32(g).tobytes())
        elif gmode == "bf16":
            tensors[name + ".weight_scale_2"] = ("BF16", [], O.f32_to_bf16_bits([g]).tobytes())
        tensors[name + ".input_scale"] = ("F32", [], np.float32(1.0).tobytes())
    dense = rng.normal(0, 1, (8, 64)).astype(np.float16)
    tensors["model.norm.weight"] = ("F16", dense.shape, dense.tobytes())
    path = tmp_path / "model.safetensors"
    write_safetensors(path, tensors, metadata={"format": "pt", "note": "a \"quoted\" \\ value"},
                      pad_header=5)
    with tq.Checkpoint(path) as ck:
        assert len(ck) == len(tensors)
        t = ck.tensor(ck.find("model.norm.weight"))
        assert (t["dtype"], t["shape"], t["nbytes"]) == (tq.CK_F16, (8, 64), dense.nbytes)
        assert np.array_equal(ck.read("model.norm.weight").view(np.float16).reshape(8, 64), dense)
        for name, (w, s, g, gmode, rows, cols) in parts.items():
            info = check_tiled_roundtrip(ck, name, tq.NVFP4, rows, cols, w, s)
            # weight_scale_2: F32 exact, BF16 widened, absent -> 1.0 (moe.cpp:670-699)
            want = {"f32": np.float32(g),
                    "bf16": np.uint32(O.f32_to_bf16_bits([g])[0]).astype(np.uint32) << 16,
                    "none": np.float32(1.0)}[gmode]
            if gmode == "bf16":
                want = np.array([want], np.uint32).view(np.float32)[0]
            assert np.float32(info["global_scale"]) == want


def test_safetensors_written_by_the_library(tmp_path, rng):
    st = pytest.importorskip("safetensors.numpy")
    arrs = {"a": rng.normal(0, 1, (3, 5)).astype(np.float32),
            "b": rng.normal(0, 1, (7,)).astype(np.float16),
            "c": rng.integers(0, 255, (4, 6), dtype=np.uint8),
            "d": rng.integers(-5, 5, (2, 2, 2), dtype=np.int64)}
    path = tmp_path / "lib.safetensors"
    st.save_file(arrs, str(path), metadata={"k": "v"})
    codes = {np.float32: tq.CK_F32, np.float16: tq.CK_F16, np.uint8: tq.CK_U8, np.int64: tq.CK_I64}
    with tq.Checkpoint(path) as ck:
        assert len(ck) == 4
        for k, a in arrs.items():
            t = ck.tensor(ck.find(k))
            assert t["shape"] == a.shape and t["dtype"] == codes[a.dtype.type]
            assert ck.read(k).tobytes() == a.tobytes()


def test_safetensors_sharded_directory(tmp_path, rng):
    w0 = rng.integers(0, 255, (16, 32), dtype=np.uint8)
    w1 = rng.normal(0, 1, (4,)).astype(np.float32)
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors", {"x.weight": ("U8", w0.shape, w0.tobytes())})
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors", {"y.bias": ("F32", w1.shape, w1.tobytes())})
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": {"x.weight": "model-00001-of-00002.safetensors",
                                                  "y.bias": "model-00002-of-00002.safetensors"}}, f)
    with tq.Checkpoint(tmp_path) as ck:
        assert sorted(t["name"] for t in ck.tensors()) == ["x.weight", "y.bias"]
        assert ck.read("x.weight").tobytes() == w0.tobytes()
        assert ck.read("y.bias").tobytes() == w1.tobytes()


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_kquants(tmp_path, rng, alignment):
    rows, cols = 32, 512
    q4 = O.quantize_q4k(rng.normal(0, 0.02, (rows, cols)))
    q3 = O.quantize_q3k(rng.normal(0, 0.02, (rows, cols)))
    f32 = rng.normal(0, 1, (3, 4)).astype(np.float32)
    kvs = [("general.architecture", GGUF_STR, "llama"),
           ("general.alignment", GGUF_U32, alignment),
           ("llama.block_count", GGUF_U64, 2),
           ("llama.rope.freq_base", GGUF_F32, 10000.0),
           ("tokenizer.ggml.tokens", GGUF_ARR, (GGUF_STR, ["<s>", "</s>", "a"])),
           ("tokenizer.ggml.scores", GGUF_ARR, (GGUF_F32, [0.0, 0.5, 1.0]))]
    tensors = [("blk.0.ffn_gate.weight", 12, [cols, rows], q4.tobytes()),
               ("blk.0.ffn_down.weight", 11, [cols, rows], q3.tobytes()),
               ("blk.0.attn_norm.weight", 0, [4, 3], f32.tobytes())]
    path = tmp_path / "m.gguf"
    write_gguf(path, tensors, kvs, alignment=alignment)
    with tq.Checkpoint(path) as ck:
        assert len(ck) == 3
        t = ck.tensor(ck.find("blk.0.ffn_gate.weight"))
        assert (t["dtype"], t["ggml_type"], t["shape"], t["nbytes"]) == (tq.CK_GGML, 12, (rows, cols), q4.nbytes)
        t = ck.tensor(ck.find("blk.0.attn_norm.weight"))
        assert (t["dtype"], t["shape"]) == (tq.CK_F32, (3, 4))
        assert np.array_equal(ck.read("blk.0.attn_norm.weight").view(np.float32).reshape(3, 4), f32)
        check_tiled_roundtrip(ck, "blk.0.ffn_gate.weight", tq.Q4_K, rows, cols, q4)
        check_tiled_roundtrip(ck, "blk.0.ffn_down.weight", tq.Q3_K, rows, cols, q3)
        with pytest.raises(tq.TitanError, match="status -2"):   # a plain f32 tensor is no quantized weight
            ck.load_tiled("blk.0.attn_norm.weight")


def test_titan_v1_int4(tmp_path, rng):
    rows, cols, gs = 64, 1024, 128
    w, s, b = O.quantize_int4(rng.normal(0, 0.02, (rows, cols)), gs)
    w2, s2, b2 = O.quantize_int4(rng.normal(0, 0.02, (32, 512)), 64)
    emb = rng.normal(0, 1, (10, 16)).astype(np.float16)
    write_titan_v1(tmp_path, {
        "files": {"attention": ("attention.bin", [
            ("model.layers.0.self_attn.q_proj.weight", "int4", (rows, cols), int4_blob(w, s, b), gs)]),
            "embedding": ("embedding.bin", [("model.embed_tokens.weight", "fp16", emb.shape, emb.tobytes(), 0)])},
        "expert_index": {"0": ("experts/layer_00.bin", [
            ("model.layers.0.mlp.experts.0.up_proj.weight", "int4", (32, 512), int4_blob(w2, s2, b2), 64)])}})
    with tq.Checkpoint(tmp_path) as ck:
        assert len(ck) == 3
        t = ck.tensor(ck.find("model.layers.0.self_attn.q_proj.weight"))
        assert (t["dtype"], t["shape"], t["group_size"]) == (tq.CK_INT4_AFFINE, (rows, cols), gs)
        check_tiled_roundtrip(ck, "model.layers.0.self_attn.q_proj.weight", tq.INT4, rows, cols, w, s, b, gs)
        check_tiled_roundtrip(ck, "model.layers.0.mlp.experts.0.up_proj.weight", tq.INT4, 32, 512,
                              w2, s2, b2, 64)
        assert ck.read("model.embed_tokens.weight").tobytes() == emb.tobytes()


def test_errors(tmp_path, rng):
    with pytest.raises(tq.TitanError, match="status -5"):
        tq.Checkpoint(tmp_path / "missing.safetensors")
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(tq.TitanError, match="status -5"):
        tq.Checkpoint(bad)
    trunc = tmp_path / "trunc.safetensors"
    write_safetensors(trunc, {"a": ("F32", [4], np.zeros(4, np.float32).tobytes())})
    trunc.write_bytes(trunc.read_bytes()[:-4])                 # data shorter than data_offsets
    with pytest.raises(tq.TitanError, match="status -5"):
        tq.Checkpoint(trunc)
    gg = tmp_path / "v1.gguf"
    write_gguf(gg, [], [], version=1)
    with pytest.raises(tq.TitanError, match="status -2"):
        tq.Checkpoint(gg)
    ok = tmp_path / "ok.safetensors"
    w, s, g = nvfp4_parts(16, 128, rng)
    write_safetensors(ok, {"p.weight": ("U8", w.shape, w.tobytes()), "p.weight_scale": ("F8_E4M3", s.shape, s.tobytes())})
    with tq.Checkpoint(ok) as ck:
        with pytest.raises(tq.TitanError, match="status -6"):
            ck.load_tiled("q")
        info = ck.weight_info("p")
        small = np.empty(info["tiled_bytes"] - 1, np.uint8)
        st = tq.lib().titan_ckpt_load_tiled(ck._h, b"p", small.ctypes.data_as(tq._P), small.nbytes, None)
        assert st == tq.ERR_INVALID_ARG
