"""Python host bindings of the gfx950 quantized matrix-product library.

Loads ``libtitan_qmm.so`` (built in-tree by ``make -C titan-engine_amd``) and
exposes its C ABI (include/titan_qmm.h).  Device buffers are passed as torch
tensors (torch is used for device memory and streams only); host-side repack
functions take numpy arrays.  There is no fallback: every entry point raises
if the native library is missing or a call returns a non-zero status.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtitan_qmm.so")

# status / enums (include/titan_qmm.h)
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_LAUNCH, ERR_WORKSPACE = 0, -1, -2, -3, -4
ERR_SCRATCH_LIMIT = -7
NOALLOC_SCRATCH_BYTES = 32 << 20
ERR_IO, ERR_NOT_FOUND = -5, -6
FP32, FP16, BF16 = 0, 1, 2
FP8_E4M3, FP4, INT4, INT2, Q4_K, Q3_K, NVFP4 = 3, 5, 7, 8, 9, 10, 32
LAYOUT_REF, LAYOUT_TILED = 0, 1
MAX_BATCH = 8

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t


class QWeightC(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int32), ("layout", ctypes.c_int32),
                ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("group_size", ctypes.c_int32), ("global_scale", ctypes.c_float),
                ("codes", _P), ("scales", _P), ("biases", _P)]


class TitanError(RuntimeError):
    pass


# checkpoint reader (include/titan_ckpt.h)
CK_F32, CK_F16, CK_BF16, CK_F64, CK_I8, CK_U8, CK_I16, CK_I32, CK_I64, CK_BOOL = range(10)
CK_F8_E4M3, CK_F8_E5M2, CK_GGML, CK_INT4_AFFINE = 10, 11, 100, 200


class CkTensorC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int), ("ggml_type", ctypes.c_int),
                ("ndim", ctypes.c_int), ("shape", ctypes.c_int64 * 8), ("nbytes", ctypes.c_uint64),
                ("group_size", ctypes.c_int)]


class CkWeightC(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int), ("rows", ctypes.c_int), ("cols", ctypes.c_int),
                ("group_size", ctypes.c_int), ("global_scale", ctypes.c_float),
                ("tiled_bytes", ctypes.c_size_t)]


_LIB = None

# every function the header declares, with its ctypes argument list
_SIGS = {
    "titan_dequant_matvec_int4": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "titan_dequant_matvec_int2": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "titan_dequant_matvec_fp4": [_P, _P, _P, _P, _I, _I, _I, _P],
    "titan_dequant_matvec_nvfp4": [_P, _P, _F, _P, _P, _I, _I, _P],
    "titan_quantize_fp4": [_P, _P, _P, _I, _I, _P],
    "titan_sparse_dequant_matvec_int4": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "titan_qgemm": [ctypes.POINTER(QWeightC), _P, _I, _I64, _P, _I, _I64, _I, _P],
    "titan_qgemm_batched": [ctypes.POINTER(QWeightC), ctypes.POINTER(_P), ctypes.POINTER(_P),
                            _I, _I, _I, _I, _P],
    "titan_qgemm_workspace_bytes": [ctypes.POINTER(_I), _I, _I],
    "titan_qgemm_ws": [ctypes.POINTER(QWeightC), _P, _I, _I64, _P, _I, _I64, _I, _P, _SZ, _P],
    "titan_qgemm_batched_noalloc": [ctypes.POINTER(QWeightC), ctypes.POINTER(_P), ctypes.POINTER(_P),
                                    _I, _I, _I, _I, _P],
    "titan_qgemm_batched_ws": [ctypes.POINTER(QWeightC), ctypes.POINTER(_P), ctypes.POINTER(_P),
                               _I, _I, _I, _I, _P, _SZ, _P],
    "titan_qdequant": [ctypes.POINTER(QWeightC), _P, _I, _P],
    "titan_tiled_bytes": [_I, _I, _I, _I],
    "titan_repack_host": [_I, _I, _I, _I, _P, _P, _P, _P, _SZ],
    "titan_unpack_host": [_I, _I, _I, _I, _P, _P, _P, _P],
    "titan_fp8_quantize_rows": [_P, _I, _I, _I, _P, _P, _P],
    "titan_fp8_gemm": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "titan_moe_gate": [_P, _P, _P, _I, _I, _P],
    "titan_moe_topk": [_P, _P, _P, _I, _I, _P],
    "titan_moe_topk_batched": [_P, _P, _P, _I, _I, _I, _P],
    "titan_swiglu": [_P, _P, _P, _I, _P],
    "titan_fused_moe_combine_norm": [_P, _P, _P, _P, _P, _F, _P, _I, _I, _F, _P],
    "titan_moe_nvfp4_workspace_bytes": [_I, _I, _I, _I, _I],
    "titan_moe_nvfp4_forward": [_P, _I, _I, _I, _P, _I, _I, _P, _P, _I, _P, _P, _F, _P, _I,
                                _P, _SZ, _P],
    "titan_ckpt_open": [ctypes.c_char_p, ctypes.POINTER(_P)],
    "titan_ckpt_count": [_P],
    "titan_ckpt_tensor_at": [_P, _I, ctypes.POINTER(CkTensorC)],
    "titan_ckpt_find": [_P, ctypes.c_char_p],
    "titan_ckpt_read": [_P, _I, _P, _SZ],
    "titan_ckpt_weight_info": [_P, ctypes.c_char_p, ctypes.POINTER(CkWeightC)],
    "titan_ckpt_load_tiled": [_P, ctypes.c_char_p, _P, _SZ, ctypes.POINTER(CkWeightC)],
    "titan_gemv_bf16_to_fp32": [_P, _P, _P, _I, _I, _P],
    "titan_gemv_fp32": [_P, _P, _P, _I, _I, _P],
    "titan_gemv_fp32_batched": [_P, _P, _P, _I, _I, _I, _P],
    "titan_matvec_dispatch": [ctypes.POINTER(QWeightC), _P, _P, _P],
    "titan_version": [],
    "titan_status_string": [_I],
}


def lib():
    """The loaded native library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise TitanError(f"{LIB_PATH} is missing: build it with `make -C titan-engine_amd`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _I
        L.titan_ckpt_close.argtypes = [_P]
        L.titan_ckpt_close.restype = None
        L.titan_tiled_bytes.restype = _SZ
        L.titan_moe_nvfp4_workspace_bytes.restype = _SZ
        L.titan_qgemm_workspace_bytes.restype = _SZ
        L.titan_version.restype = ctypes.c_char_p
        L.titan_status_string.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


def _check(st, what):
    if st != OK:
        raise TitanError(f"{what}: status {st} ({lib().titan_status_string(st).decode()})")


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, np.ndarray):
        return t.ctypes.data_as(_P)
    return _P(t.data_ptr())


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return _P(s.cuda_stream)


_TORCH_DT = {}


def dtype_code(torch_dtype):
    import torch
    return {torch.float32: FP32, torch.float16: FP16, torch.bfloat16: BF16}[torch_dtype]


# ---------------------------------------------------------------------------
# weights
# ---------------------------------------------------------------------------
class QWeight:
    """A quantized matrix on the device: format, layout, shape and buffers.

    REF layout: ``codes`` / ``scales`` / ``biases`` as the reference stores
    them.  TILED layout: ``codes`` is the tiled buffer (FP8 keeps its fp32
    per-row ``scales``).  Tensors are kept alive by this object."""

    def __init__(self, fmt, layout, rows, cols, codes, scales=None, biases=None,
                 group_size=0, global_scale=1.0):
        self.fmt, self.layout, self.rows, self.cols = fmt, layout, rows, cols
        self.codes, self.scales, self.biases = codes, scales, biases
        self.group_size, self.global_scale = group_size, float(global_scale)

    def cstruct(self):
        return QWeightC(self.fmt, self.layout, self.rows, self.cols, self.group_size,
                        self.global_scale, _ptr(self.codes), _ptr(self.scales),
                        _ptr(self.biases))

    def nbytes(self):
        n = 0
        for t in (self.codes, self.scales, self.biases):
            if t is not None:
                n += t.numel() * t.element_size()
        return n


def tiled_bytes(fmt, rows, cols, group_size=0):
    return int(lib().titan_tiled_bytes(fmt, rows, cols, group_size))


def repack_host(fmt, rows, cols, codes, scales=None, biases=None, group_size=0):
    """REF numpy parts -> TILED numpy uint8 buffer (exact byte permutation)."""
    n = tiled_bytes(fmt, rows, cols, group_size)
    if n == 0:
        raise TitanError("format/shape has no tiled form")
    out = np.zeros(n, np.uint8)
    c = np.ascontiguousarray(codes)
    s = None if scales is None else np.ascontiguousarray(scales)
    b = None if biases is None else np.ascontiguousarray(biases)
    _check(lib().titan_repack_host(fmt, rows, cols, group_size, _ptr(c), _ptr(s), _ptr(b),
                                   _ptr(out), n), "titan_repack_host")
    return out


def unpack_host(fmt, rows, cols, tiled, codes_like, scales_like=None, biases_like=None,
                group_size=0):
    """TILED numpy buffer -> REF parts shaped like the given templates."""
    codes = np.zeros_like(codes_like)
    scales = None if scales_like is None else np.zeros_like(scales_like)
    biases = None if biases_like is None else np.zeros_like(biases_like)
    t = np.ascontiguousarray(tiled)
    _check(lib().titan_unpack_host(fmt, rows, cols, group_size, _ptr(t), _ptr(codes),
                                   _ptr(scales), _ptr(biases)), "titan_unpack_host")
    return codes, scales, biases


# ---------------------------------------------------------------------------
# compute
# ---------------------------------------------------------------------------
def qgemm_workspace_bytes(rows, M):
    """Bytes of the K-split workspace for problems with these row counts."""
    rows = [int(r) for r in (rows if isinstance(rows, (list, tuple)) else [rows])]
    arr = (_I * len(rows))(*rows)
    return int(lib().titan_qgemm_workspace_bytes(arr, len(rows), int(M)))


def qgemm_workspace(rows, M, device="cuda"):
    """A zero-filled workspace for qgemm(..., workspace=) / qgemm_batched."""
    import torch
    return torch.zeros(qgemm_workspace_bytes(rows, M), dtype=torch.uint8, device=device)


def _ws_args(workspace):
    return _ptr(workspace), workspace.numel() * workspace.element_size()


def qgemm(W, X, out_dtype=None, out=None, stream=None, workspace=None):
    """Y[m] = W @ X[m] for X of shape [M, cols] (fp32/fp16/bf16 on the GPU).
    With `workspace` (from qgemm_workspace) small problems split K across
    workgroups (titan_qgemm_ws)."""
    import torch
    X2 = X if X.dim() == 2 else X.view(1, -1)
    M = X2.shape[0]
    if out is None:
        out = torch.empty((M, W.rows), dtype=out_dtype or X.dtype, device=X.device)
    ws = W.cstruct()
    if workspace is None:
        _check(lib().titan_qgemm(ctypes.byref(ws), _ptr(X2), dtype_code(X2.dtype), X2.stride(0),
                                 _ptr(out), dtype_code(out.dtype), out.stride(0), M,
                                 _stream(stream)), "titan_qgemm")
    else:
        _check(lib().titan_qgemm_ws(ctypes.byref(ws), _ptr(X2), dtype_code(X2.dtype),
                                    X2.stride(0), _ptr(out), dtype_code(out.dtype),
                                    out.stride(0), M, *_ws_args(workspace), _stream(stream)),
               "titan_qgemm_ws")
    return out


def qgemm_batched(Ws, Xs, Ys, stream=None, workspace=None):
    n = len(Ws)
    arr = (QWeightC * n)(*[w.cstruct() for w in Ws])
    xs = (_P * n)(*[_ptr(x) for x in Xs])
    ys = (_P * n)(*[_ptr(y) for y in Ys])
    M = Xs[0].shape[0] if Xs[0].dim() == 2 else 1
    if workspace is None:
        _check(lib().titan_qgemm_batched(arr, xs, ys, n, dtype_code(Xs[0].dtype),
                                         dtype_code(Ys[0].dtype), M, _stream(stream)),
               "titan_qgemm_batched")
    else:
        _check(lib().titan_qgemm_batched_ws(arr, xs, ys, n, dtype_code(Xs[0].dtype),
                                            dtype_code(Ys[0].dtype), M, *_ws_args(workspace),
                                            _stream(stream)), "titan_qgemm_batched_ws")


def qgemm_batched_noalloc(Ws, Xs, Ys, stream=None):
    """qgemm_batched with the K-split workspace in the library's static device
    scratch (titan_qgemm_batched_noalloc): allocates nothing."""
    n = len(Ws)
    arr = (QWeightC * n)(*[w.cstruct() for w in Ws])
    xs = (_P * n)(*[_ptr(x) for x in Xs])
    ys = (_P * n)(*[_ptr(y) for y in Ys])
    M = Xs[0].shape[0] if Xs[0].dim() == 2 else 1
    _check(lib().titan_qgemm_batched_noalloc(arr, xs, ys, n, dtype_code(Xs[0].dtype),
                                             dtype_code(Ys[0].dtype), M, _stream(stream)),
           "titan_qgemm_batched_noalloc")


class PreparedBatch:
    """qgemm_batched with its C arguments built once: calling it issues one
    titan_qgemm_batched on the stream given at preparation (for replaying the
    same weights/activations/outputs in a decode loop)."""

    def __init__(self, Ws, Xs, Ys, stream=None, workspace=None):
        n = len(Ws)
        self._keep = (Ws, Xs, Ys, workspace)
        args = ((QWeightC * n)(*[w.cstruct() for w in Ws]),
                (_P * n)(*[_ptr(x) for x in Xs]), (_P * n)(*[_ptr(y) for y in Ys]), n,
                dtype_code(Xs[0].dtype), dtype_code(Ys[0].dtype),
                Xs[0].shape[0] if Xs[0].dim() == 2 else 1)
        if workspace is None:
            self._args = args + (_stream(stream),)
            self._fn = lib().titan_qgemm_batched
        else:
            self._args = args + _ws_args(workspace) + (_stream(stream),)
            self._fn = lib().titan_qgemm_batched_ws

    def __call__(self):
        st = self._fn(*self._args)
        if st:
            _check(st, self._fn.__name__)


def qdequant(W, out_dtype=None, stream=None):
    import torch
    out = torch.empty((W.rows, W.cols), dtype=out_dtype or torch.float32, device="cuda")
    ws = W.cstruct()
    _check(lib().titan_qdequant(ctypes.byref(ws), _ptr(out), dtype_code(out.dtype),
                                _stream(stream)), "titan_qdequant")
    return out


def dequant_matvec_int4(w, s, b, x, y, rows, cols, gs, stream=None):
    _check(lib().titan_dequant_matvec_int4(_ptr(w), _ptr(s), _ptr(b), _ptr(x), _ptr(y), rows,
                                           cols, gs, _stream(stream)), "dequant_matvec_int4")


def dequant_matvec_int2(w, s, b, x, y, rows, cols, gs, stream=None):
    _check(lib().titan_dequant_matvec_int2(_ptr(w), _ptr(s), _ptr(b), _ptr(x), _ptr(y), rows,
                                           cols, gs, _stream(stream)), "dequant_matvec_int2")


def dequant_matvec_fp4(w, s, x, y, rows, cols, gs, stream=None):
    _check(lib().titan_dequant_matvec_fp4(_ptr(w), _ptr(s), _ptr(x), _ptr(y), rows, cols, gs,
                                          _stream(stream)), "dequant_matvec_fp4")


def dequant_matvec_nvfp4(w, s, g, x, y, rows, cols, stream=None):
    _check(lib().titan_dequant_matvec_nvfp4(_ptr(w), _ptr(s), float(g), _ptr(x), _ptr(y), rows,
                                            cols, _stream(stream)), "dequant_matvec_nvfp4")


def gemv_bf16_to_fp32(A, x, y, rows, cols, stream=None):
    """gemv.cu:103-159: y = bf16(A) @ x, fp32 x / y (A passed as a bf16 or int16 tensor)."""
    _check(lib().titan_gemv_bf16_to_fp32(_ptr(A), _ptr(x), _ptr(y), rows, cols, _stream(stream)),
           "gemv_bf16_to_fp32")


def gemv_fp32(A, x, y, rows, cols, stream=None):
    _check(lib().titan_gemv_fp32(_ptr(A), _ptr(x), _ptr(y), rows, cols, _stream(stream)), "gemv_fp32")


def gemv_fp32_batched(A, x, y, rows, cols, batch, stream=None):
    _check(lib().titan_gemv_fp32_batched(_ptr(A), _ptr(x), _ptr(y), rows, cols, batch,
                                         _stream(stream)), "gemv_fp32_batched")


def matvec_dispatch(W, x, y, stream=None):
    """dense.cpp:13-32, format-exact: W is a QWeight (quantized, or fmt FP32 /
    BF16 with the dense matrix in ``codes``); fp32 x [cols] -> fp32 y [rows]."""
    c = W.cstruct()
    _check(lib().titan_matvec_dispatch(ctypes.byref(c), _ptr(x), _ptr(y), _stream(stream)),
           "matvec_dispatch")


def sparse_dequant_matvec_int4(w, s, b, x, y, active, cols, gs, stream=None):
    _check(lib().titan_sparse_dequant_matvec_int4(_ptr(w), _ptr(s), _ptr(b), _ptr(x), _ptr(y),
                                                  _ptr(active), active.numel(), cols, gs,
                                                  _stream(stream)), "sparse_dequant_matvec_int4")


def quantize_fp4(x, out, scales, numel, gs, stream=None):
    _check(lib().titan_quantize_fp4(_ptr(x), _ptr(out), _ptr(scales), numel, gs,
                                    _stream(stream)), "quantize_fp4")


def fp8_quantize_rows(x, xq, xs, stream=None):
    M, K = x.shape
    _check(lib().titan_fp8_quantize_rows(_ptr(x), dtype_code(x.dtype), M, K, _ptr(xq), _ptr(xs),
                                         _stream(stream)), "fp8_quantize_rows")


def fp8_gemm(A, sa, W, sw, out, stream=None):
    M, K = A.shape
    N = W.shape[0]
    _check(lib().titan_fp8_gemm(_ptr(A), _ptr(sa), _ptr(W), _ptr(sw), _ptr(out),
                                dtype_code(out.dtype), M, N, K, _stream(stream)), "fp8_gemm")


def moe_gate(h, G, logits, stream=None):
    E, hd = G.shape
    _check(lib().titan_moe_gate(_ptr(h), _ptr(G), _ptr(logits), hd, E, _stream(stream)),
           "moe_gate")


def moe_topk(logits, w, idx, k, stream=None):
    _check(lib().titan_moe_topk(_ptr(logits), _ptr(w), _ptr(idx), logits.numel(), k,
                                _stream(stream)), "moe_topk")


def moe_topk_batched(logits, w, idx, k, stream=None):
    T, E = logits.shape
    _check(lib().titan_moe_topk_batched(_ptr(logits), _ptr(w), _ptr(idx), T, E, k,
                                        _stream(stream)), "moe_topk_batched")


def swiglu(out, gate, up, stream=None):
    _check(lib().titan_swiglu(_ptr(out), _ptr(gate), _ptr(up), out.numel(), _stream(stream)),
           "swiglu")


def fused_moe_combine_norm(out, residual, expert_out, w, shared, shared_w, dim, na,
                           stream=None):
    _check(lib().titan_fused_moe_combine_norm(_ptr(out), _ptr(residual), _ptr(expert_out),
                                              _ptr(w), _ptr(shared), float(shared_w), None, dim,
                                              na, 1e-5, _stream(stream)),
           "fused_moe_combine_norm")


class NvExpertC(ctypes.Structure):
    """titan_nvfp4_expert: device pointers to the three TILED NVFP4 matrices
    and their fp32 global scales."""
    _fields_ = [("gate", _P), ("up", _P), ("down", _P), ("gate_scale", ctypes.c_float),
                ("up_scale", ctypes.c_float), ("down_scale", ctypes.c_float)]


def nvfp4_expert_table(experts):
    """[(gate_dev, up_dev, down_dev, gs_gate, gs_up, gs_down)] -> device uint8
    tensor holding the titan_nvfp4_expert array (keep the weight tensors alive)."""
    import torch
    arr = (NvExpertC * len(experts))(*[NvExpertC(_ptr(g), _ptr(u), _ptr(d), float(a), float(b),
                                                 float(c)) for g, u, d, a, b, c in experts])
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.cuda()


def moe_nvfp4_workspace_bytes(tokens, k, E, hidden, inter):
    return int(lib().titan_moe_nvfp4_workspace_bytes(tokens, k, E, hidden, inter))


def moe_nvfp4_forward(table, E, hidden, inter, x, indices, weights, out, workspace,
                      residual=None, shared=None, shared_weight=0.0, stream=None):
    T, k = indices.shape
    _check(lib().titan_moe_nvfp4_forward(_ptr(table), E, hidden, inter, _ptr(x),
                                         dtype_code(x.dtype), T, _ptr(indices), _ptr(weights), k,
                                         _ptr(residual), _ptr(shared), float(shared_weight),
                                         _ptr(out), dtype_code(out.dtype), _ptr(workspace),
                                         workspace.numel() * workspace.element_size(),
                                         _stream(stream)), "moe_nvfp4_forward")


# ---------------------------------------------------------------------------
# checkpoints: safetensors / GGUF / titan-v1 reads and load-time repack
# ---------------------------------------------------------------------------
class Checkpoint:
    """A checkpoint opened through titan_ckpt_open (a .safetensors or .gguf
    file, or a directory of safetensors shards or a titan-v1 manifest).

    ``load_tiled(name)`` returns the TILED host buffer of a quantized weight
    (GGUF Q4_K / Q3_K, titan-v1 int4, or an NVFP4 projection given by its base
    name) and its description; ``load_weight(name)`` uploads it as a QWeight."""

    def __init__(self, path):
        h = _P()
        _check(lib().titan_ckpt_open(os.fsencode(str(path)), ctypes.byref(h)), f"open {path}")
        self._h = h

    def close(self):
        if self._h:
            lib().titan_ckpt_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return int(lib().titan_ckpt_count(self._h))

    def tensor(self, index):
        t = CkTensorC()
        _check(lib().titan_ckpt_tensor_at(self._h, int(index), ctypes.byref(t)), "tensor_at")
        return dict(name=t.name.decode(), dtype=t.dtype, ggml_type=t.ggml_type,
                    shape=tuple(t.shape[d] for d in range(t.ndim)), nbytes=int(t.nbytes),
                    group_size=t.group_size)

    def tensors(self):
        return [self.tensor(i) for i in range(len(self))]

    def find(self, name):
        return int(lib().titan_ckpt_find(self._h, name.encode()))

    def read(self, name_or_index):
        i = name_or_index if isinstance(name_or_index, int) else self.find(name_or_index)
        if i < 0:
            raise TitanError(f"{name_or_index}: status {ERR_NOT_FOUND} (tensor not found)")
        out = np.empty(self.tensor(i)["nbytes"], np.uint8)
        _check(lib().titan_ckpt_read(self._h, i, _ptr(out), out.nbytes), "read")
        return out

    def weight_info(self, name):
        w = CkWeightC()
        _check(lib().titan_ckpt_weight_info(self._h, name.encode(), ctypes.byref(w)), f"weight {name}")
        return dict(fmt=w.format, rows=w.rows, cols=w.cols, group_size=w.group_size,
                    global_scale=w.global_scale, tiled_bytes=int(w.tiled_bytes))

    def load_tiled(self, name):
        info = self.weight_info(name)
        out = np.empty(info["tiled_bytes"], np.uint8)
        w = CkWeightC()
        _check(lib().titan_ckpt_load_tiled(self._h, name.encode(), _ptr(out), out.nbytes,
                                           ctypes.byref(w)), f"load {name}")
        return out, info

    def load_weight(self, name, device="cuda"):
        import torch
        buf, info = self.load_tiled(name)
        dev = torch.from_numpy(buf).to(device)
        return QWeight(info["fmt"], LAYOUT_TILED, info["rows"], info["cols"], dev,
                       group_size=info["group_size"], global_scale=info["global_scale"])
