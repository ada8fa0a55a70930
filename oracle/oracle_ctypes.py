"""numpy bindings for the CPU oracle (liboracle.so) and oracle/_ref.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the measured or
shipped path.  The product library (titan-engine_amd/) never imports this.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


def build():
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
        L = _LIB
        L.or_f16_to_f32.restype = _F
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [_F]
        L.or_bf16_to_f32.restype = _F
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [_F]
        L.or_e4m3_ref_to_f32.restype = _F
        L.or_e4m3_ref_to_f32.argtypes = [ctypes.c_uint8]
        L.or_e4m3_ocp_to_f32.restype = _F
        L.or_e4m3_ocp_to_f32.argtypes = [ctypes.c_uint8]
        L.or_f32_to_e4m3.restype = ctypes.c_uint8
        L.or_f32_to_e4m3.argtypes = [_F]
        L.or_fp4_e2m1_to_f32.restype = _F
        L.or_fp4_e2m1_to_f32.argtypes = [ctypes.c_uint8]
        for fn in ["or_dequant_int4", "or_dequant_int2", "or_dequant_fp4", "or_dequant_nvfp4",
                   "or_dequant_q4k", "or_dequant_q3k", "or_dequant_fp8", "or_gemm_f32",
                   "or_gemm_f64", "or_matvec_int4_cpu", "or_matvec_int4_cpu_mt",
                   "or_matvec_nvfp4", "or_matvec_fmt_mt", "or_quantize_int4",
                   "or_quantize_int2", "or_quantize_fp4", "or_quantize_nvfp4",
                   "or_quantize_q4k", "or_quantize_q3k", "or_quantize_fp8_rows",
                   "or_quantize_act_fp8", "or_gemm_fp8", "or_moe_topk", "or_swiglu",
                   "or_moe_combine"]:
            getattr(L, fn).restype = None
    return _LIB


def _p(a):
    return a.ctypes.data_as(_P) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- scalar helpers (vectorised through numpy where exact) -------------------

def f16_bits_to_f32(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def e4m3_ref_table():
    L = lib()
    return np.array([L.or_e4m3_ref_to_f32(i) for i in range(256)], dtype=np.float32)


def f32_to_e4m3(v):
    L = lib()
    v = np.asarray(v, dtype=np.float32).ravel()
    return np.array([L.or_f32_to_e4m3(float(x)) for x in v], dtype=np.uint8)


def f32_to_bf16_bits(v):
    L = lib()
    v = np.asarray(v, dtype=np.float32).ravel()
    return np.array([L.or_f32_to_bf16(float(x)) for x in v], dtype=np.uint16)


# ---- quantizers ---------------------------------------------------------------

def quantize_int4(W, gs):
    W = _c(W, np.float32)
    rows, cols = W.shape
    w = np.zeros((rows, cols // 8), np.uint32)
    s = np.zeros((rows, cols // gs), np.uint16)
    b = np.zeros((rows, cols // gs), np.uint16)
    lib().or_quantize_int4(_p(W), _I(rows), _I(cols), _I(gs), _p(w), _p(s), _p(b))
    return w, s, b


def quantize_int2(W, gs):
    W = _c(W, np.float32)
    rows, cols = W.shape
    w = np.zeros((rows, cols // 16), np.uint32)
    s = np.zeros((rows, cols // gs), np.uint16)
    b = np.zeros((rows, cols // gs), np.uint16)
    lib().or_quantize_int2(_p(W), _I(rows), _I(cols), _I(gs), _p(w), _p(s), _p(b))
    return w, s, b


def quantize_fp4(W, gs):
    W = _c(W, np.float32)
    rows, cols = W.shape
    w = np.zeros((rows, cols // 8), np.uint32)
    s = np.zeros((rows, cols // gs), np.uint16)
    lib().or_quantize_fp4(_p(W), _I(rows * cols), _I(gs), _p(w), _p(s))
    return w, s


def quantize_nvfp4(W, g):
    W = _c(W, np.float32)
    rows, cols = W.shape
    w = np.zeros((rows, cols // 2), np.uint8)
    s = np.zeros((rows, cols // 16), np.uint8)
    lib().or_quantize_nvfp4(_p(W), _I(rows), _I(cols), _F(g), _p(w), _p(s))
    return w, s


def quantize_q4k(W):
    W = _c(W, np.float32)
    rows, cols = W.shape
    out = np.zeros((rows, cols // 256 * 144), np.uint8)
    lib().or_quantize_q4k(_p(W), _I(rows), _I(cols), _p(out))
    return out


def quantize_q3k(W):
    W = _c(W, np.float32)
    rows, cols = W.shape
    out = np.zeros((rows, cols // 256 * 110), np.uint8)
    lib().or_quantize_q3k(_p(W), _I(rows), _I(cols), _p(out))
    return out


def quantize_fp8_rows(W):
    W = _c(W, np.float32)
    rows, cols = W.shape
    w = np.zeros((rows, cols), np.uint8)
    s = np.zeros(rows, np.float32)
    lib().or_quantize_fp8_rows(_p(W), _I(rows), _I(cols), _p(w), _p(s))
    return w, s


def quantize_act_fp8(x_bf16_bits):
    x = _c(x_bf16_bits, np.uint16)
    M, K = x.shape
    q = np.zeros((M, K), np.uint8)
    s = np.zeros(M, np.float32)
    lib().or_quantize_act_fp8(_p(x), _I(M), _I(K), _p(q), _p(s))
    return q, s


# ---- dequantizers -------------------------------------------------------------

def dequant_int4(w, s, b, rows, cols, gs):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_int4(_p(_c(w, np.uint32)), _p(_c(s, np.uint16)), _p(_c(b, np.uint16)),
                          _I(rows), _I(cols), _I(gs), _p(out))
    return out


def dequant_int2(w, s, b, rows, cols, gs):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_int2(_p(_c(w, np.uint32)), _p(_c(s, np.uint16)), _p(_c(b, np.uint16)),
                          _I(rows), _I(cols), _I(gs), _p(out))
    return out


def dequant_fp4(w, s, rows, cols, gs):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_fp4(_p(_c(w, np.uint32)), _p(_c(s, np.uint16)), _I(rows), _I(cols),
                         _I(gs), _p(out))
    return out


def dequant_nvfp4(w, s, g, rows, cols):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_nvfp4(_p(_c(w, np.uint8)), _p(_c(s, np.uint8)), _F(g), _I(rows),
                           _I(cols), _p(out))
    return out


def dequant_q4k(blocks, rows, cols):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_q4k(_p(_c(blocks, np.uint8)), _I(rows), _I(cols), _p(out))
    return out


def dequant_q3k(blocks, rows, cols):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_q3k(_p(_c(blocks, np.uint8)), _I(rows), _I(cols), _p(out))
    return out


def dequant_fp8(w, cs, rows, cols):
    out = np.zeros((rows, cols), np.float32)
    lib().or_dequant_fp8(_p(_c(w, np.uint8)), _p(_c(cs, np.float32)), _I(rows), _I(cols),
                         _p(out))
    return out


# ---- dense / GEMV references -----------------------------------------------------

def gemm_f32(W, X):
    W = _c(W, np.float32)
    X = _c(np.atleast_2d(X), np.float32)
    N, K = W.shape
    M = X.shape[0]
    Y = np.zeros((M, N), np.float32)
    lib().or_gemm_f32(_p(W), _p(X), _I(M), _I(N), _I(K), _p(Y))
    return Y


def gemm_f64(W, X):
    W = _c(W, np.float32)
    X = _c(np.atleast_2d(X), np.float32)
    N, K = W.shape
    M = X.shape[0]
    Y = np.zeros((M, N), np.float64)
    lib().or_gemm_f64(_p(W), _p(X), _I(M), _I(N), _I(K), _p(Y))
    return Y


def matvec_int4_cpu(w, s, b, x, rows, cols, gs):
    y = np.zeros(rows, np.float32)
    lib().or_matvec_int4_cpu(_p(_c(w, np.uint32)), _p(_c(s, np.uint16)), _p(_c(b, np.uint16)),
                             _p(_c(x, np.float32)), _p(y), _I(rows), _I(cols), _I(gs))
    return y


FMT_CODES = {"int4": 0, "int2": 1, "nvfp4": 2, "q4k": 3, "q3k": 4, "fp8": 5}


def matvec_fmt_mt(fmt, codes, s, b, g, gs, x, rows, cols, nthreads):
    y = np.zeros(rows, np.float32)
    lib().or_matvec_fmt_mt(_I(FMT_CODES[fmt]), _p(codes), _p(s), _p(b), _F(g), _I(gs),
                           _p(_c(x, np.float32)), _p(y), _I(rows), _I(cols), _I(nthreads))
    return y


def matvec_nvfp4(w, s, g, x, rows, cols):
    y = np.zeros(rows, np.float32)
    lib().or_matvec_nvfp4(_p(_c(w, np.uint8)), _p(_c(s, np.uint8)), _F(g),
                          _p(_c(x, np.float32)), _p(y), _I(rows), _I(cols))
    return y


def gemm_fp8(A, sa, W, sw):
    A = _c(A, np.uint8)
    W = _c(W, np.uint8)
    M, K = A.shape
    N = W.shape[0]
    out = np.zeros((M, N), np.float32)
    lib().or_gemm_fp8(_p(A), _p(_c(sa, np.float32)), _p(W), _p(_c(sw, np.float32)),
                      _I(M), _I(N), _I(K), _p(out))
    return out


def moe_topk(logits, k):
    logits = _c(logits, np.float32)
    E = logits.shape[0]
    w = np.zeros(k, np.float32)
    idx = np.zeros(k, np.int32)
    lib().or_moe_topk(_p(logits), _I(E), _I(k), _p(w), _p(idx))
    return w, idx


def swiglu(gate, up):
    gate = _c(gate, np.float32)
    up = _c(up, np.float32)
    out = np.zeros_like(gate)
    lib().or_swiglu(_p(out), _p(gate), _p(up), _I(gate.size))
    return out


def moe_combine(residual, expert_out, w, shared=None, shared_w=0.0):
    residual = _c(residual, np.float32).copy()
    expert_out = _c(expert_out, np.float32)
    out = np.zeros_like(residual)
    na = expert_out.shape[0]
    lib().or_moe_combine(_p(out), _p(residual), _p(expert_out), _p(_c(w, np.float32)),
                         _p(_c(shared, np.float32)) if shared is not None else None,
                         _F(shared_w), _I(residual.size), _I(na))
    return out, residual


# ---- the reference's own CPU expert path (oracle/_ref) ----------------------------

def _cpu_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return all(t in flags for t in ("avx512f", "avx512bw", "avx512vl", "f16c", " fma"))
    except OSError:
        return False


_REF = None


def ref_lib():
    """The reference's matmul_avx.cpp/expert_cpu.cpp built into oracle/_ref, or None.

    The AVX-512 build is used where the host supports it (the reference's
    TITAN_HAS_AVX512 configuration), else the reference's scalar fallback."""
    global _REF
    if _REF is None:
        name = "libtitan_ref_cpu_avx512.so" if _cpu_has_avx512() else "libtitan_ref_cpu_scalar.so"
        path = os.path.join(HERE, "_ref", name)
        if not os.path.exists(path):
            return None
        _REF = ctypes.CDLL(path)
        _REF.ref_dequant_matvec_int4.restype = None
        _REF.variant = "avx512" if "avx512" in name else "scalar"
    return _REF


def ref_matvec_int4(w, s, b, x, rows, cols, gs):
    L = ref_lib()
    y = np.zeros(rows, np.float32)
    L.ref_dequant_matvec_int4(_p(_c(w, np.uint32)), _p(_c(s, np.uint16)), _p(_c(b, np.uint16)),
                              _p(_c(x, np.float32)), _p(y), _I(rows), _I(cols), _I(gs))
    return y
