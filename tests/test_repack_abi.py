"""CPU tests of the product library: it loads, exports every symbol that
include/*.h declares, and its host-side loader repack is an exact byte
permutation with an exact inverse (no GPU needed for any of these)."""
import os
import re

import numpy as np
import pytest

import titan_qmm as tq
from helpers import make_weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FMTS = {"int4": tq.INT4, "int2": tq.INT2, "fp4": tq.FP4, "nvfp4": tq.NVFP4,
        "q4k": tq.Q4_K, "q3k": tq.Q3_K, "fp8": tq.FP8_E4M3}


def declared_functions():
    names = []
    inc = os.path.join(ROOT, "include")
    for f in sorted(os.listdir(inc)):
        if not f.endswith(".h"):
            continue
        text = open(os.path.join(inc, f)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(titan_\w+)\s*\(", text, flags=re.M)
    return names


def test_library_exports_every_declared_symbol():
    L = tq.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert L.titan_version().startswith(b"titan-qmm")
    assert L.titan_status_string(-2) == b"unsupported shape/format/layout"


def ref_parts(d):
    return d["codes"], d["scales"], d["biases"]


@pytest.mark.parametrize("fmt", list(FMTS))
@pytest.mark.parametrize("rows,cols", [(16, 512), (48, 1024), (32, 2048)])
def test_repack_roundtrip_bytes(fmt, rows, cols, rng):
    gs = 64 if fmt in ("int4", "int2", "fp4") else 0
    d = make_weights(fmt, rows, cols, rng, gs=gs or 128)
    f = FMTS[fmt]
    codes, scales, biases = ref_parts(d)
    if fmt == "fp8":
        scales = None  # per-row fp32 scales are not part of the tiled buffer
    n = tq.tiled_bytes(f, rows, cols, gs)
    ref_bytes = sum(a.nbytes for a in (codes, scales, biases) if a is not None)
    assert n == ref_bytes, "tiled layout must be a permutation of the REF bytes"
    t = tq.repack_host(f, rows, cols, codes, scales, biases, gs)
    c2, s2, b2 = tq.unpack_host(f, rows, cols, t, codes, scales, biases, gs)
    assert np.array_equal(c2, codes)
    if scales is not None:
        assert np.array_equal(s2, scales)
    if biases is not None:
        assert np.array_equal(b2, biases)
    # a permutation: the multiset of bytes is unchanged -- except Q3_K, whose
    # tiled hmask words permute bits (the decoder's order): there the bit
    # count is unchanged, and so is the multiset of the other bytes
    allref = np.concatenate([np.ascontiguousarray(a).view(np.uint8).ravel()
                             for a in (codes, scales, biases) if a is not None])
    if fmt != "q3k":
        assert np.array_equal(np.sort(allref), np.sort(t))
    else:
        blk = allref.reshape(-1, 110)
        plane = rows * cols // 4  # the tiled code plane, then the hmask plane
        hm = t[plane:plane + rows * (cols // 256) * 32]
        assert np.unpackbits(hm).sum() == np.unpackbits(blk[:, :32]).sum()
        rest = np.concatenate([t[:plane], t[plane + hm.size:]])
        assert np.array_equal(np.sort(blk[:, 32:].ravel()), np.sort(rest))


def test_q3k_tiled_hmask_bit_order(rng):
    """Tiled Q3_K hmask word: ggml bit 4h + jj of byte k (half h, level jj)
    at bit (2jj + 2 + (k & 1) + 16 (k >> 1) + 8h) mod 32, so that the decoder
    finds the high bit of level jj of bytes 0 and 2 at bits 2jj + 2 and
    2jj + 18 (bytes 1, 3 one higher; h = 1 rotated by 8).  One hand-placed
    bit per (k, h, jj) through a one-block matrix."""
    rows, cols = 16, 256
    d = make_weights("q3k", rows, cols, rng)
    codes = d["codes"].copy()
    plane = rows * cols // 4
    for k in range(4):
        for h in range(2):
            for jj in range(4):
                blk = codes.view(np.uint8).reshape(rows, 110)
                blk[:, :32] = 0
                blk[0, 4 + k] = 1 << (4 * h + jj)  # hmask word 1 (j = 1), byte k
                t = tq.repack_host(FMTS["q3k"], rows, cols, codes)
                # row 0, block 0, plane entry j = 1, first word of the pair
                off = plane + ((0 * 1 + 0) * 4 + 1) * 16 * 8
                w = int(np.frombuffer(t[off:off + 4].tobytes(), np.uint32)[0])
                assert w == 1 << ((2 * jj + 2 + (k & 1) + 16 * (k >> 1) + 8 * h) % 32), (k, h, jj)


def test_repack_code_plane_is_lane_major(rng):
    """Chunk c of a 16-row tile is 1 KiB in lane order (lane = 16*j + r); lane
    (r, j) holds words j, 4+j, 8+j, 12+j of row r's 64-byte chunk."""
    d = make_weights("int4", 16, 256, rng, gs=64)
    t = tq.repack_host(tq.INT4, 16, 256, d["codes"], d["scales"], d["biases"], 64)
    words = d["codes"].reshape(16, 32)  # row -> 32 words (two chunks of 16)
    tw = t[:16 * 128].view(np.uint32)
    for c in range(2):
        for j in range(4):
            for r in range(16):
                lane = 16 * j + r
                got = tw[c * 256 + lane * 4: c * 256 + lane * 4 + 4]
                assert got.tolist() == [int(words[r, 16 * c + 4 * i + j]) for i in range(4)]


def test_repack_rejects_untileable_shapes():
    assert tq.tiled_bytes(tq.INT4, 15, 256, 64) == 0       # rows % 16
    assert tq.tiled_bytes(tq.INT4, 16, 96, 32) == 0        # 48-byte rows
    assert tq.tiled_bytes(tq.INT4, 16, 256, 16) == 0       # group inside a 32-col slot
    assert tq.tiled_bytes(tq.Q4_K, 16, 384, 0) == 0
    assert tq.tiled_bytes(tq.NVFP4, 16, 128, 0) == 16 * 64 + 16 * 8
    assert tq.tiled_bytes(tq.NVFP4, 16, 64, 0) == 0         # NVFP4 tiles whole 128-column chunks
    with pytest.raises(tq.TitanError):
        tq.repack_host(tq.INT4, 15, 256, np.zeros((15, 32), np.uint32),
                       np.zeros((15, 4), np.uint16), np.zeros((15, 4), np.uint16), 64)


@pytest.mark.parametrize("fmt,rows,cols,gs", [("int4", 32, 1024, 256),   # a group over two chunks
                                              ("int4", 16, 640, 128),    # five groups: padded scale cell
                                              ("int4", 16, 512, 32),     # four groups per chunk
                                              ("int2", 16, 1024, 512),   # two chunks per group
                                              ("int2", 32, 768, 128)])   # three chunks: padded cell
def test_repack_roundtrip_scale_cells(fmt, rows, cols, gs, rng):
    """INT4 / INT2 scales sit in 16-byte cells (repeated for groups longer
    than a chunk, padded to whole cells); the round trip stays exact."""
    d = make_weights(fmt, rows, cols, rng, gs=gs)
    f = FMTS[fmt]
    n = tq.tiled_bytes(f, rows, cols, gs)
    assert n > 0
    t = tq.repack_host(f, rows, cols, d["codes"], d["scales"], d["biases"], gs)
    c2, s2, b2 = tq.unpack_host(f, rows, cols, t, d["codes"], d["scales"], d["biases"], gs)
    assert np.array_equal(c2, d["codes"]) and np.array_equal(s2, d["scales"]) and np.array_equal(b2, d["biases"])


SHIM_PROBE = r"""
#include "titan_qmm_shim.hpp"
#include <cstdio>
static int seen = 0;
static void on_status(int st, const char*) { if (st == TITAN_ERR_INVALID_ARG) seen++; }
int main() {
    namespace tc = titan::cuda;
    tc::set_status_handler(on_status);
    tc::init_cublas();
    // argument checks only: every call below is rejected before any HIP call
    tc::swiglu(nullptr, nullptr, nullptr, 0, nullptr);
    tc::gemv_fp32(nullptr, nullptr, nullptr, 4, 4, nullptr);
    tc::gemv_fp32_batched(nullptr, nullptr, nullptr, 4, 4, 0, nullptr);
    tc::gemv_bf16_to_fp32(nullptr, nullptr, nullptr, 4, 4, nullptr);
    tc::dequant_matvec_int4(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 128, 128, nullptr);
    tc::dequant_matvec_int2(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 128, 128, nullptr);
    tc::dequant_matvec_fp4(nullptr, nullptr, nullptr, nullptr, 4, 128, 32, nullptr);
    tc::dequant_matvec_nvfp4(nullptr, nullptr, 1.0f, nullptr, nullptr, 4, 128, nullptr);
    tc::sparse_dequant_matvec_int4(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 128, 128, nullptr);
    tc::destroy_cublas();
    std::printf("%d %d\n", seen, tc::last_status());
    return 0;
}
"""


def test_cpp_shim_compiles_and_forwards(tmp_path):
    """include/titan_qmm_shim.hpp restores the reference's titan::cuda names
    (src/compute/dispatch.h:30-130) over the C ABI; the probe links the
    product library and sees each call's status through the shim."""
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no host C++ compiler")
    tq.lib()
    src = tmp_path / "probe.cpp"
    src.write_text(SHIM_PROBE)
    exe = tmp_path / "probe"
    libdir = os.path.dirname(tq.LIB_PATH)
    subprocess.run([gxx, "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include", str(src),
                    "-L", libdir, "-ltitan_qmm", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["9", str(tq.ERR_INVALID_ARG)]


def test_every_entry_point_rejects_bad_arguments():
    """Null pointers and non-positive sizes return TITAN_ERR_INVALID_ARG before
    any device work (so this runs without a GPU); the reference checks
    nothing and returns void (dispatch.h:30-130)."""
    import ctypes
    L = tq.lib()
    E = tq.ERR_INVALID_ARG
    N = None
    W = tq.QWeightC()
    calls = {
        "titan_dequant_matvec_int4": (N, N, N, N, N, 16, 128, 128, N),
        "titan_dequant_matvec_int2": (N, N, N, N, N, 16, 128, 64, N),
        "titan_dequant_matvec_fp4": (N, N, N, N, 16, 128, 32, N),
        "titan_dequant_matvec_nvfp4": (N, N, ctypes.c_float(1.0), N, N, 16, 128, N),
        "titan_sparse_dequant_matvec_int4": (N, N, N, N, N, N, 1, 128, 128, N),
        "titan_quantize_fp4": (N, N, N, 128, 32, N),
        "titan_qgemm": (N, N, tq.FP16, 128, N, tq.FP16, 16, 1, N),
        "titan_qgemm_batched": (ctypes.byref(W), N, N, 0, tq.FP16, tq.FP16, 1, N),
        "titan_qgemm_ws": (N, N, tq.FP16, 128, N, tq.FP16, 16, 1, N, ctypes.c_size_t(0), N),
        "titan_qgemm_batched_ws": (ctypes.byref(W), N, N, 0, tq.FP16, tq.FP16, 1, N,
                                   ctypes.c_size_t(0), N),
        "titan_qgemm_batched_noalloc": (ctypes.byref(W), N, N, 0, tq.FP16, tq.FP16, 1, N),
        "titan_qdequant": (N, N, tq.FP32, N),
        "titan_fp8_quantize_rows": (N, tq.BF16, 1, 128, N, N, N),
        "titan_fp8_gemm": (N, N, N, N, N, tq.BF16, 128, 128, 128, N),
        "titan_moe_gate": (N, N, N, 128, 8, N),
        "titan_moe_topk": (N, N, N, 8, 2, N),
        "titan_moe_topk_batched": (N, N, N, 1, 8, 2, N),
        "titan_swiglu": (N, N, N, 16, N),
        "titan_fused_moe_combine_norm": (N, N, N, N, N, ctypes.c_float(0.0), N, 16, 1,
                                         ctypes.c_float(1e-6), N),
        "titan_moe_nvfp4_forward": (N, 8, 512, 512, N, tq.BF16, 1, N, N, 2, N, N,
                                    ctypes.c_float(0.0), N, tq.BF16, N, ctypes.c_size_t(0), N),
        "titan_gemv_bf16_to_fp32": (N, N, N, 16, 16, N),
        "titan_gemv_fp32": (N, N, N, 16, 16, N),
        "titan_gemv_fp32_batched": (N, N, N, 16, 16, 2, N),
        "titan_matvec_dispatch": (N, N, N, N),
    }
    for name, args in calls.items():
        assert getattr(L, name)(*args) == E, name
    # sizes: zero or negative rows / cols / tokens
    x = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(x, ctypes.c_void_p)
    assert L.titan_gemv_fp32(p, p, p, 0, 16, N) == E
    assert L.titan_gemv_fp32(p, p, p, 16, -1, N) == E
    assert L.titan_fp8_quantize_rows(p, tq.BF16, 0, 128, p, p, N) == E
    assert L.titan_swiglu(p, p, p, 0, N) == E
    # K-split workspace: one fixed 8 KiB counter region (2048 tile groups),
    # then 16 parts of fp32 partials per token (at most 32 tokens a launch)
    # for every problem, rows rounded up to whole 16-row tiles
    rows = (ctypes.c_int * 2)(4096, 1000)
    one = L.titan_qgemm_workspace_bytes(rows, 1, 1)
    assert one == 8192 + 16 * 4096 * 4
    assert L.titan_qgemm_workspace_bytes(rows, 2, 1) == one + 16 * 1008 * 4
    assert L.titan_qgemm_workspace_bytes(rows, 1, 64) == 8192 + 32 * 16 * 4096 * 4
    assert L.titan_qgemm_workspace_bytes(rows, 0, 1) == 0
    assert L.titan_qgemm_workspace_bytes(N, 1, 1) == 0


def test_noalloc_rejects_beyond_static_scratch():
    """titan_qgemm_batched_noalloc refuses, before any device work (so this
    runs without a GPU), a call whose K-split workspace would exceed the
    library's static scratch, with its own status."""
    import ctypes
    L = tq.lib()
    rows = (ctypes.c_int * 8)(*([4096] * 8))
    assert L.titan_qgemm_workspace_bytes(rows, 8, 32) > tq.NOALLOC_SCRATCH_BYTES
    assert L.titan_qgemm_workspace_bytes(rows, 1, 32) <= tq.NOALLOC_SCRATCH_BYTES
    Ws = (tq.QWeightC * 8)()
    for w in Ws:
        w.format, w.layout, w.rows, w.cols, w.group_size = tq.INT4, tq.LAYOUT_TILED, 4096, 1024, 128
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    xs = (ctypes.c_void_p * 8)(*([p] * 8))
    assert L.titan_qgemm_batched_noalloc(Ws, xs, xs, 8, tq.FP16, tq.FP16, 32, None) == tq.ERR_SCRATCH_LIMIT
    assert L.titan_status_string(tq.ERR_SCRATCH_LIMIT).startswith(b"problem needs more than the static scratch")
    assert L.titan_qgemm_batched_noalloc(Ws, xs, xs, 8, tq.FP16, tq.FP16, 0, None) == tq.ERR_INVALID_ARG
