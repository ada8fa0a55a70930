/*
 * qmm_oracle.h -- CPU oracle for the quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * kernels are compared against.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it; the product library
 * (libtitan_qmm.so) never links, loads or calls it.
 *
 * Every decoder restates the reference's algorithm in plain C and cites the
 * reference file:line it follows (paths relative to the titan-engine tree).
 * Formats the reference has no decoder for (Q4_K, Q3_K) restate the public
 * ggml block format (llama.cpp ggml-quants.c, MIT; not vendored in the
 * reference) and are pinned by known-answer blocks and invariants in tests/.
 *
 * Pinning status per function is listed in the header comment of
 * qmm_oracle.c.
 */
#ifndef TITAN_QMM_ORACLE_H
#define TITAN_QMM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions ------------------------------------------------ */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);              /* round-to-nearest-even */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);             /* round-to-nearest-even */
float    or_e4m3_ref_to_f32(uint8_t v);       /* fp4.cu:173-185, 0x7F/0xFF -> 0 */
float    or_e4m3_ocp_to_f32(uint8_t v);       /* OCP E4M3FN, 0x7F/0xFF -> NaN */
uint8_t  or_f32_to_e4m3(float f);             /* RNE, saturating to +-448 */
float    or_fp4_e2m1_to_f32(uint8_t nib);     /* fp4.cu:23-26 LUT */

/* ---- dequantizers: packed -> fp32 [rows][cols] ------------------------- */
void or_dequant_int4(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     int rows, int cols, int gs, float* out);
void or_dequant_int2(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     int rows, int cols, int gs, float* out);
void or_dequant_fp4(const uint32_t* w, const uint16_t* s,
                    int rows, int cols, int gs, float* out);
void or_dequant_nvfp4(const uint8_t* w, const uint8_t* s, float global_scale,
                      int rows, int cols, float* out);
void or_dequant_q4k(const uint8_t* blocks, int rows, int cols, float* out);
void or_dequant_q3k(const uint8_t* blocks, int rows, int cols, float* out);
void or_dequant_fp8(const uint8_t* w, const float* ch_scale,
                    int rows, int cols, float* out);

/* ---- dense references --------------------------------------------------- */
/* Y[m][n] = sum_k W[n][k] * X[m][k], fp32 accumulation in ascending k. */
void or_gemm_f32(const float* W, const float* X, int M, int N, int K, float* Y);
/* Same in fp64 (brute-force second oracle). */
void or_gemm_f64(const float* W, const float* X, int M, int N, int K, double* Y);

/* ---- reference-loop GEMVs ----------------------------------------------- */
/* matmul_avx.cpp:54-100 / :119-158: row-serial, column-ascending,
 * acc += ((float)q*s + b) * x, single fp32 accumulator. */
void or_matvec_int4_cpu(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                        const float* x, float* y, int rows, int cols, int gs);
/* Same loop, rows partitioned over nthreads pthreads. */
void or_matvec_int4_cpu_mt(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                           const float* x, float* y, int rows, int cols, int gs,
                           int nthreads);
/* fp4.cu:187-238 restated serially (acc += lut*s0*x in column order). */
void or_matvec_nvfp4(const uint8_t* w, const uint8_t* s, float g,
                     const float* x, float* y, int rows, int cols);
/* Row-serial GEMV over a dequantized-on-the-fly format, same loop shape as
 * matmul_avx.cpp (fmt: 0 int4, 1 int2, 2 nvfp4, 3 q4k, 4 q3k, 5 fp8). Used
 * as the CPU baseline for formats the reference has no CPU routine for. */
void or_matvec_fmt_mt(int fmt, const void* codes, const void* s, const void* b,
                      float g, int gs, const float* x, float* y, int rows,
                      int cols, int nthreads);

/* ---- quantizers (fixture generators only) ------------------------------ */
void or_quantize_int4(const float* W, int rows, int cols, int gs,
                      uint32_t* w, uint16_t* s, uint16_t* b);  /* convert_titan.py:43-77 */
void or_quantize_int2(const float* W, int rows, int cols, int gs,
                      uint32_t* w, uint16_t* s, uint16_t* b);
void or_quantize_fp4(const float* W, int numel, int gs,
                     uint32_t* w, uint16_t* s);                /* fp4.cu:90-141 */
void or_quantize_nvfp4(const float* W, int rows, int cols, float global_scale,
                       uint8_t* w, uint8_t* s);
void or_quantize_q4k(const float* W, int rows, int cols, uint8_t* blocks);
void or_quantize_q3k(const float* W, int rows, int cols, uint8_t* blocks);
void or_quantize_fp8_rows(const float* W, int rows, int cols,
                          uint8_t* w, float* ch_scale);
/* bf16 activations -> e4m3 with per-token scale amax/448 */
void or_quantize_act_fp8(const uint16_t* x_bf16, int M, int K,
                         uint8_t* xq, float* x_scale);
/* FP8 GEMM reference: out[m][n] = (sum_k e4m3(a)*e4m3(w)) * sa[m] * sw[n] */
void or_gemm_fp8(const uint8_t* A, const float* sa, const uint8_t* W,
                 const float* sw, int M, int N, int K, float* out);

/* ---- MoE pieces ----------------------------------------------------------- */
/* moe.cu:58-115: softmax over all E (max-subtracted, 1/(sum+1e-8)), top-k by
 * repeated strict-> argmax, renormalise w/(sum+1e-8). */
void or_moe_topk(const float* logits, int E, int k, float* w, int* idx);
/* activation.cu:17-32 */
void or_swiglu(float* out, const float* gate, const float* up, int n);
/* activation.cu:111-139: res += sum_e w_e*y_e + w_s*shared; out = res */
void or_moe_combine(float* out, float* residual, const float* expert_out,
                    const float* w, const float* shared, float shared_w,
                    int dim, int num_active);

#ifdef __cplusplus
}
#endif
#endif
