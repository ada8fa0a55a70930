"""Writers of small checkpoint files for the loader tests.

safetensors: 8-byte little-endian header length, JSON header
({name: {dtype, shape, data_offsets}}, optional __metadata__), data.
GGUF v3: magic, version, tensor and key/value counts, key/values, tensor
infos (dims innermost first), data at the next `general.alignment` boundary.
titan-v1: manifest.json + .bin files as tools/convert_titan.py:146-235 writes
them (an int4 entry is int32 codes | fp16 scales | fp16 biases).
These follow the published formats; they are test fixtures, not product code.
"""
import json
import os
import struct

import numpy as np


def write_safetensors(path, tensors, metadata=None, pad_header=0):
    """tensors: {name: (dtype_str, shape, raw bytes)} in file order."""
    header, off, blobs = {}, 0, []
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dt, shape, raw) in tensors.items():
        raw = bytes(raw)
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode() + b" " * pad_header
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _gstr(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


GGUF_U32, GGUF_F32, GGUF_STR, GGUF_ARR, GGUF_U64 = 4, 6, 8, 9, 10


def _gval(t, v):
    if t == GGUF_U32:
        return struct.pack("<I", v)
    if t == GGUF_U64:
        return struct.pack("<Q", v)
    if t == GGUF_F32:
        return struct.pack("<f", v)
    if t == GGUF_STR:
        return _gstr(v)
    if t == GGUF_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_gval(et, x) for x in items)
    raise ValueError(t)


def write_gguf(path, tensors, kvs=(), alignment=32, version=3):
    """tensors: [(name, ggml_type, dims innermost first, raw bytes)];
    kvs: [(key, gguf type, value)] (a 'general.alignment' entry sets the
    alignment the writer pads to)."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _gstr(k) + struct.pack("<I", t) + _gval(t, v)
    off, datas = 0, []
    for name, typ, dims, raw in tensors:
        off = (off + alignment - 1) // alignment * alignment
        out += _gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", typ, off)
        datas.append((off, bytes(raw)))
        off += len(raw)
    pad = (-len(out)) % alignment
    out += b"\0" * pad
    base = len(out)
    for o, raw in datas:
        out += b"\0" * (base + o - len(out))
        out += raw
    with open(path, "wb") as f:
        f.write(out)


def write_titan_v1(dirname, groups):
    """groups: {section: {key: (file name, [(name, dtype, shape, raw, group_size)])}}
    with section 'files' or 'expert_index'."""
    manifest = {"format": "titan-v1", "model_config": {}, "quantization": "int4",
                "group_size": 128, "files": {}, "expert_index": {}}
    for sec, entries in groups.items():
        for key, (fname, tensors) in entries.items():
            os.makedirs(os.path.dirname(os.path.join(dirname, fname)) or dirname, exist_ok=True)
            ents, off = [], 0
            with open(os.path.join(dirname, fname), "wb") as f:
                for name, dt, shape, raw, gs in tensors:
                    e = {"name": name, "offset": off, "size": len(raw), "dtype": dt, "shape": list(shape)}
                    if dt == "int4":
                        e["group_size"] = gs
                    f.write(raw)
                    ents.append(e)
                    off += len(raw)
            manifest[sec][key] = {"file": fname, "tensors": ents}
    with open(os.path.join(dirname, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)


def int4_blob(w, s, b):
    """convert_titan.py:168-171: weights | scales | biases."""
    return np.ascontiguousarray(w).tobytes() + np.ascontiguousarray(s).tobytes() + \
        np.ascontiguousarray(b).tobytes()
