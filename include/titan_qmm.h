/*
 * titan_qmm.h -- C ABI of the MI355X (gfx950) quantized matrix-product path.
 *
 * Drop-in boundary for Titan Engine's src/compute kernel entry points.  Every
 * function is extern "C", takes caller-owned device pointers, plain sizes and
 * a hipStream_t, allocates no device memory, and returns an int status
 * (TITAN_OK == 0).  Preconditions are validated on the host before any
 * launch; a failed check launches nothing.
 *
 * Reference interfaces replaced (paths into the titan-engine tree):
 *   titan_dequant_matvec_int4   src/compute/dispatch.h:32-34  (dequant.cu:227-240)
 *   titan_dequant_matvec_int2   src/compute/dispatch.h:35-37  (dequant.cu:242-255)
 *   titan_dequant_matvec_fp4    src/compute/dispatch.h:107-109 (fp4.cu:147-159)
 *   titan_dequant_matvec_nvfp4  src/compute/dispatch.h:110-112 (fp4.cu:240-252)
 *   titan_quantize_fp4          src/compute/dispatch.h:113-114 (fp4.cu:254-266)
 *   titan_sparse_dequant_matvec_int4 src/compute/dispatch.h:127-130 (sparse.cu:142-205)
 *   titan_moe_gate              src/compute/dispatch.h:82-83   (moe.cu:197-205)
 *   titan_moe_topk              src/compute/dispatch.h:84-85   (moe.cu:207-214)
 *   titan_swiglu                src/compute/dispatch.h:47-48   (activation.cu:145-151)
 *   titan_fused_moe_combine_norm src/compute/dispatch.h:59-63  (activation.cu:171-185)
 * The remaining entry points are the north-star extensions of those calls:
 * fp16/bf16 activations and outputs, M > 1 tokens, the gfx950 tiled weight
 * layout and its loader-side repack (hook point: loader.cpp:434-472,
 * gguf_loader.cpp:321-342, moe.cpp:613-724), Q4_K / Q3_K decoders
 * (gguf_loader.h:62-100 block geometry; types.h:27-28), the FP8 prefill GEMM
 * and the NVFP4 MoE grouped-expert path (moe.cpp:874-1005).
 */
#ifndef TITAN_QMM_H
#define TITAN_QMM_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
enum {
    TITAN_OK = 0,
    TITAN_ERR_INVALID_ARG = -1,   /* null pointer, non-positive size, bad enum */
    TITAN_ERR_UNSUPPORTED = -2,   /* shape / format / layout combination */
    TITAN_ERR_LAUNCH = -3,        /* hipGetLastError() after the launch */
    TITAN_ERR_WORKSPACE = -4,     /* workspace missing or too small */
    TITAN_ERR_IO = -5,            /* checkpoint file missing, unreadable or malformed */
    TITAN_ERR_NOT_FOUND = -6,     /* no such tensor in the checkpoint */
    TITAN_ERR_SCRATCH_LIMIT = -7  /* needs more than the static scratch (TITAN_NOALLOC_SCRATCH_BYTES) */
};

/* ---- element / weight formats --------------------------------------------
 * Values 0..14 are titan::DType (types.h:17-33); NVFP4 has no DType in the
 * reference (moe.cpp detects it from U8 tensors) and gets its own value. */
enum {
    TITAN_FP32 = 0,
    TITAN_FP16 = 1,
    TITAN_BF16 = 2,
    TITAN_FP8_E4M3 = 3,  /* weights: e4m3 codes [rows][cols] + fp32 per-row scale */
    TITAN_FP4 = 5,       /* fp4.cu:28-84: u32 [rows][cols/8] + fp16 group scale */
    TITAN_INT4 = 7,      /* dequant.cu:23-104: u32 [rows][cols/8] + fp16 scale, bias */
    TITAN_INT2 = 8,      /* dequant.cu:110-172: u32 [rows][cols/16] + fp16 scale, bias */
    TITAN_Q4_K = 9,      /* ggml block of 256: 144 bytes */
    TITAN_Q3_K = 10,     /* ggml block of 256: 110 bytes */
    TITAN_NVFP4 = 32     /* fp4.cu:162-170: u8 [rows][cols/2] + e4m3 [rows][cols/16] + fp32 */
};

/* ---- weight layouts -------------------------------------------------------
 * TITAN_LAYOUT_REF   : bytes exactly as the reference / GGUF stores them
 *                      (codes, scales, biases as separate row-major arrays;
 *                      K-quants as arrays of blocks).
 * TITAN_LAYOUT_TILED : the gfx950 layout written by titan_repack_host(): one
 *                      buffer of planes, 16-row tiles, each 64-byte column
 *                      chunk of 16 rows stored as 1 KiB in wave-lane order so
 *                      that one wave's 64 x 16-byte loads are contiguous.  A
 *                      byte permutation of the REF bytes (same size), except
 *                      that Q3_K's hmask words also have their bits re-ordered
 *                      for the decoder; titan_unpack_host inverts it exactly. */
enum { TITAN_LAYOUT_REF = 0, TITAN_LAYOUT_TILED = 1 };

/* A quantized weight matrix W [rows][cols] (rows = output features). */
typedef struct titan_qweight {
    int32_t format;       /* TITAN_INT4 ... TITAN_NVFP4 */
    int32_t layout;       /* TITAN_LAYOUT_* */
    int32_t rows;
    int32_t cols;
    int32_t group_size;   /* INT4 / INT2 / FP4: elements per scale group */
    float global_scale;   /* NVFP4: per-tensor fp32 scale (weight_scale_2) */
    const void* codes;    /* REF: packed codes or K-quant blocks; TILED: the tiled buffer */
    const void* scales;   /* REF: group scales (fp16 / e4m3); FP8 (both layouts): fp32 [rows] */
    const void* biases;   /* REF INT4/INT2: fp16 biases; otherwise NULL */
} titan_qweight;

/* ======================================================================== */
/* Reference-signature entry points (fp32 activations in, fp32 out, REF     */
/* layout).  y[r] = sum_c W[r][c] * x[c], W dequantized exactly as the      */
/* reference kernels do, fp32 accumulation.                                  */
/* ======================================================================== */
int titan_dequant_matvec_int4(const void* weights, const void* scales, const void* biases,
                              const float* input, float* output, int rows, int cols,
                              int group_size, hipStream_t stream);
int titan_dequant_matvec_int2(const void* weights, const void* scales, const void* biases,
                              const float* input, float* output, int rows, int cols,
                              int group_size, hipStream_t stream);
int titan_dequant_matvec_fp4(const void* weights, const void* scales, const float* input,
                             float* output, int rows, int cols, int group_size,
                             hipStream_t stream);
int titan_dequant_matvec_nvfp4(const void* weights, const void* scales, float global_scale,
                               const float* input, float* output, int rows, int cols,
                               hipStream_t stream);
/* sparse.cu:142-205 (dispatch.h:127-130): output[active_indices[i]] =
 * dot(W[row], input) for the listed rows only (REF INT4 layout, fp32 in and
 * out); other outputs are left untouched.  Indices must be valid rows. */
int titan_sparse_dequant_matvec_int4(const void* weights, const void* scales, const void* biases,
                                     const float* input, float* output,
                                     const int* active_indices, int num_active, int cols,
                                     int group_size, hipStream_t stream);
/* fp4.cu:90-141: per group amax/6 scale (fp16), nearest-E2M1 by threshold. */
int titan_quantize_fp4(const float* input, void* output, void* scales, int numel,
                       int group_size, hipStream_t stream);

/* ======================================================================== */
/* General quantized matmul.                                                 */
/* ======================================================================== */
/* Y[m][r] = sum_c W[r][c] * X[m][c] for m < M tokens.  X: M rows of x_dtype
 * (FP32/FP16/BF16) with row stride ldx elements; Y: M rows of y_dtype with
 * row stride ldy elements.  fp32 accumulation.  Any M >= 1. */
int titan_qgemm(const titan_qweight* W, const void* X, int x_dtype, int64_t ldx,
                void* Y, int y_dtype, int64_t ldy, int M, hipStream_t stream);

/* Up to TITAN_MAX_BATCH independent problems of one format and layout in a
 * single launch (e.g. the q/k/v/o/gate/up/down matrices of one layer).  Xs[i]
 * and Ys[i] are the i-th problem's activations / outputs (dense, M rows). */
#define TITAN_MAX_BATCH 8
int titan_qgemm_batched(const titan_qweight* Ws, const void* const* Xs, void* const* Ys,
                        int n, int x_dtype, int y_dtype, int M, hipStream_t stream);

/* The same products with the K (column) range of small problems split across
 * workgroups (no counterpart in the reference: its GEMV launches one block
 * per row, dequant.cu:227-240).  Used for the 256-column-chunk formats
 * (Q3_K; INT2 from two tokens) when the launch would otherwise hold fewer
 * waves than the GPU has CUs (matrices of fewer than about 1024 rows), where
 * it measured faster; every other case runs exactly as titan_qgemm /
 * titan_qgemm_batched.
 * `workspace` is a caller-owned device buffer of at least
 * titan_qgemm_workspace_bytes() bytes, 256-byte aligned, zero-filled once
 * before its first use; every call leaves its counters at zero again, and the
 * counters of every call sit in one fixed region at the start of the
 * workspace that no partial sum overlaps, so a workspace can be reused by any
 * later call (other problem sets, other token counts) ordered after it on a
 * stream, provided it is large enough for that call.  Calls that share one
 * workspace must not overlap.  Results are deterministic (the
 * partial sums are added in a fixed order). */
size_t titan_qgemm_workspace_bytes(const int* rows, int n, int M);
int titan_qgemm_ws(const titan_qweight* W, const void* X, int x_dtype, int64_t ldx,
                   void* Y, int y_dtype, int64_t ldy, int M, void* workspace,
                   size_t workspace_bytes, hipStream_t stream);
int titan_qgemm_batched_ws(const titan_qweight* Ws, const void* const* Xs, void* const* Ys,
                           int n, int x_dtype, int y_dtype, int M, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* titan_qgemm_batched_ws with the workspace in a static device array that the
 * library holds on every GPU it runs on until the process ends, so the call
 * allocates nothing (no hipMalloc, no library allocation).  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Returns TITAN_ERR_SCRATCH_LIMIT, before any device work, when
 * titan_qgemm_workspace_bytes(rows, n, M) exceeds TITAN_NOALLOC_SCRATCH_BYTES
 * (32 MiB: e.g. 4096 rows at 32 tokens, or 28672 rows at 16 tokens).  Every
 * call on one GPU shares that GPU's array (the first call on a device clears
 * its counters with a kernel on `stream`; every call leaves them at zero):
 * calls on one GPU must be ordered (one stream, or synchronised); calls that
 * overlap on one GPU race.  Results equal titan_qgemm_batched_ws bit for bit. */
#define TITAN_NOALLOC_SCRATCH_BYTES (32u << 20)
int titan_qgemm_batched_noalloc(const titan_qweight* Ws, const void* const* Xs, void* const* Ys,
                                int n, int x_dtype, int y_dtype, int M, hipStream_t stream);

/* Exact dequantization: out[r][c] (out_dtype FP32 is bit-exact with the
 * reference's dequantized value; FP16/BF16 round it to nearest-even). */
int titan_qdequant(const titan_qweight* W, void* out, int out_dtype, hipStream_t stream);

/* ======================================================================== */
/* Loader repack (host, no GPU needed).                                      */
/* ======================================================================== */
/* Bytes of the TITAN_LAYOUT_TILED buffer for a format/shape (0 if the
 * format/shape has no tiled form: rows % 16 or the 64-byte chunking fails). */
size_t titan_tiled_bytes(int format, int rows, int cols, int group_size);
/* REF parts (codes / scales / biases as in titan_qweight) -> tiled buffer. */
int titan_repack_host(int format, int rows, int cols, int group_size, const void* codes,
                      const void* scales, const void* biases, void* tiled, size_t tiled_bytes);
/* Exact inverse of titan_repack_host. */
int titan_unpack_host(int format, int rows, int cols, int group_size, const void* tiled,
                      void* codes, void* scales, void* biases);

/* ======================================================================== */
/* FP8 prefill GEMM.                                                         */
/* ======================================================================== */
/* Per-token activation quantization: scale[m] = amax_m / 448 (1 for an
 * all-zero row), xq[m][k] = e4m3_rne_saturate(x[m][k] / scale[m]). */
int titan_fp8_quantize_rows(const void* x, int x_dtype, int M, int K, uint8_t* xq,
                            float* x_scale, hipStream_t stream);
/* out[m][n] = (sum_k e4m3(A[m][k]) * e4m3(W[n][k])) * sa[m] * sw[n], fp32
 * accumulation on MFMA, out_dtype FP32/FP16/BF16. */
int titan_fp8_gemm(const uint8_t* A, const float* sa, const uint8_t* W, const float* sw,
                   void* out, int out_dtype, int M, int N, int K, hipStream_t stream);

/* ======================================================================== */
/* MoE routing / epilogues (fp32, reference semantics).                      */
/* ======================================================================== */
int titan_moe_gate(const float* hidden, const float* gate_weight, float* logits,
                   int hidden_dim, int num_experts, hipStream_t stream);
int titan_moe_topk(const float* logits, float* weights, int* indices, int num_experts,
                   int k, hipStream_t stream);
/* One top-k per token: logits [tokens][num_experts] -> weights / indices
 * [tokens][k], each row with the titan_moe_topk semantics. */
int titan_moe_topk_batched(const float* logits, float* weights, int* indices, int tokens,
                           int num_experts, int k, hipStream_t stream);
int titan_swiglu(float* output, const float* gate, const float* up, int dim,
                 hipStream_t stream);
int titan_fused_moe_combine_norm(float* output, float* residual, const float* expert_outputs,
                                 const float* routing_weights, const float* shared_expert,
                                 float shared_weight, const float* norm_weight, int dim,
                                 int num_active, float eps, hipStream_t stream);

/* ======================================================================== */
/* NVFP4 MoE grouped-expert forward (moe.cpp:874-1005 expert loop, with the */
/* fp4.cu:187-252 dequant, activation.cu:17-32 SwiGLU and                   */
/* activation.cu:111-139 combine), all tokens in four launches.             */
/* ======================================================================== */
/* One expert: three NVFP4 matrices in TITAN_LAYOUT_TILED (titan_repack_host
 * of the reference's U8 codes + E4M3 block-16 scales), gate/up [inter][hidden],
 * down [hidden][inter], each with its fp32 global scale. */
typedef struct titan_nvfp4_expert {
    const void* gate;
    const void* up;
    const void* down;
    float gate_scale;
    float up_scale;
    float down_scale;
} titan_nvfp4_expert;

/* Device workspace for titan_moe_nvfp4_forward (bytes, 256-aligned base). */
size_t titan_moe_nvfp4_workspace_bytes(int tokens, int k, int num_experts, int hidden,
                                       int inter);

/* out[t] = residual[t] + sum_j weights[t][j] * E_{indices[t][j]}(x[t])
 *          (+ shared_weight * shared[t]),
 * E(x) = Wd (silu(Wg x) * (Wu x)).  `experts` is a DEVICE array of
 * num_experts descriptors; x [tokens][hidden] fp32/fp16/bf16; indices /
 * weights [tokens][k] (e.g. from titan_moe_topk_batched); residual and shared
 * [tokens][hidden] fp32 or NULL; out [tokens][hidden] in out_dtype.  The
 * activations enter the matrix cores as fp16; the SwiGLU output is kept as
 * fp16; accumulation and the combine are fp32.  hidden and inter must be
 * multiples of 512. */
int titan_moe_nvfp4_forward(const titan_nvfp4_expert* experts, int num_experts, int hidden,
                            int inter, const void* x, int x_dtype, int tokens,
                            const int* indices, const float* weights, int k,
                            const float* residual, const float* shared, float shared_weight,
                            void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

/* ---- library info -------------------------------------------------------- */
/* Dense GEMV, fp32 activations and output (gemv.cu:33-159):
 * BF16 A [rows][cols] (gemv_bf16_to_fp32, gemv.cu:103-159), fp32 A (gemv_fp32,
 * gemv.cu:33-52), and gemv_fp32_batched (gemv.cu:54-72: rows * batch rows of A
 * against one x, as the reference's single sgemv call computes). */
int titan_gemv_bf16_to_fp32(const void* A, const float* x, float* y, int rows, int cols,
                            hipStream_t stream);
int titan_gemv_fp32(const float* A, const float* x, float* y, int rows, int cols, hipStream_t stream);
int titan_gemv_fp32_batched(const float* A, const float* x, float* y, int rows, int cols, int batch,
                            hipStream_t stream);
/* matvec_dispatch (dense.cpp:13-32), format-exact: W->format selects the
 * decoder (INT4, INT2, FP4, NVFP4, Q4_K, Q3_K, FP8_E4M3; TITAN_FP32 / TITAN_BF16
 * for dense row-major weights in W->codes).  fp32 input[cols] -> output[rows]. */
int titan_matvec_dispatch(const titan_qweight* W, const float* input, float* output, hipStream_t stream);

const char* titan_version(void);
const char* titan_status_string(int status);

#ifdef __cplusplus
}
#endif
#endif /* TITAN_QMM_H */
