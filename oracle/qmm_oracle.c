/*
 * qmm_oracle.c -- CPU oracle for the quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY (see qmm_oracle.h).  Built with -ffp-contract=off
 * so that every expression rounds exactly as written.
 *
 * Pinning status (what checks each function in tests/):
 *   or_f16_to_f32 / or_f32_to_f16 / bf16   numpy float16 / exhaustive 65536 sweep
 *   or_e4m3_ref_to_f32                     closed form over all 256 codes; 0x7F/0xFF
 *   or_f32_to_e4m3                         exhaustive round trip + brute-force nearest
 *   or_dequant_int4 / int2                 known-answer words; oracle/_ref (reference
 *                                          matmul_avx.cpp GEMV, bit-exact); brute force
 *   or_dequant_fp4                         hand-built words (nibble order, group
 *                                          of each word, per-row scale stride,
 *                                          group sizes 8/12/16/24); exact round
 *                                          trip of on-grid values through
 *                                          or_quantize_fp4; error bound
 *   or_dequant_nvfp4                       hand-built bytes (nibble order, NaN
 *                                          scale -> 0); fp64 GEMV
 *   or_dequant_q4k / q3k                   known-answer blocks packed by an
 *                                          independent packer in tests/; every
 *                                          sub-scale position; quantize error bound
 *   or_dequant_fp8                         all 256 codes against the OCP table
 *   or_gemm_f32                            fp64 brute force
 *   or_matvec_fmt_mt                       per format: fp64 product of the exact
 *                                          dequantized matrix within the fp32
 *                                          accumulation bound; one-hot columns
 *                                          bit-exact; thread split bit-exact
 *   or_matvec_int4_cpu                     oracle/_ref (bit-exact)
 *   or_moe_topk                            hand-computed softmax / tie cases
 * No function is "parity unpinned".
 */
#include "qmm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* scalar conversions                                                       */
/* ======================================================================== */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {                      /* inf / nan */
        return sign | 0x7C00 | (a > 0x7F800000u ? 0x200 : 0);
    }
    if (a >= 0x477FF000u) return sign | 0x7C00;  /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {                       /* below 2^-14: subnormal */
        /* value / 2^-24, rounded to nearest even; scaling by 2^24 is exact */
        float v = u2f(a) * 16777216.0f;
        float r = rintf(v);
        return sign | (uint16_t)r;
    }
    uint32_t e = (a >> 23) - 112;
    uint32_t m = a & 0x7FFFFF;
    uint32_t rest = m & 0x1FFF;
    uint32_t hm = m >> 13;
    uint32_t out = (e << 10) | hm;
    if (rest > 0x1000 || (rest == 0x1000 && (hm & 1))) out += 1;
    return sign | (uint16_t)out;
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7FFF + ((u >> 16) & 1);
    return (uint16_t)(u >> 16);
}

/* fp4.cu:173-185.  Bias 7; (v & 0x7F) == 0x7F (the NaN codes) decode to 0. */
float or_e4m3_ref_to_f32(uint8_t v) {
    if ((v & 0x7F) == 0x7F) return 0.0f;
    int sign = (v >> 7) & 1;
    int exp = (v >> 3) & 0xF;
    int man = v & 7;
    float mag = exp == 0 ? ldexpf((float)man * 0.125f, -6)
                         : ldexpf(1.0f + (float)man * 0.125f, exp - 7);
    return sign ? -mag : mag;
}

/* OCP FP8 E4M3FN (the encoding gfx950's fp8 MFMA consumes). */
float or_e4m3_ocp_to_f32(uint8_t v) {
    if ((v & 0x7F) == 0x7F) return NAN;
    return or_e4m3_ref_to_f32(v);
}

uint8_t or_f32_to_e4m3(float f) {
    uint8_t sign = (f2u(f) >> 31) ? 0x80 : 0;
    float a = fabsf(f);
    if (a != a) return 0x7F;
    if (a >= 448.0f) return sign | 0x7E;
    if (a < 0.015625f) {                         /* below 2^-6: subnormal */
        float m = rintf(a * 512.0f);             /* units of 2^-9, exact scaling */
        return sign | (uint8_t)m;                /* m == 8 encodes 2^-6 (0x08) */
    }
    int ex;
    frexpf(a, &ex);                              /* a = fr * 2^ex, fr in [0.5,1) */
    int E = ex - 1;                              /* a in [2^E, 2^(E+1)) */
    float t = (ldexpf(a, -E) - 1.0f) * 8.0f;     /* exact */
    float m = rintf(t);
    int mi = (int)m;
    if (mi == 8) { mi = 0; E += 1; }
    if (E > 8 || (E == 8 && mi > 6)) return sign | 0x7E;
    return sign | (uint8_t)(((E + 7) << 3) | mi);
}

/* fp4.cu:23-26 */
static const float kFp4Lut[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float or_fp4_e2m1_to_f32(uint8_t nib) { return kFp4Lut[nib & 0xF]; }

/* ======================================================================== */
/* dequantizers                                                             */
/* ======================================================================== */

/* dequant.cu:23-104 and matmul_avx.cpp:54-100: nibble n of word p is column
 * 8p+n; group = base_col / group_size; value = (float)q * scale + bias. */
void or_dequant_int4(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     int rows, int cols, int gs, float* out) {
    int ppr = cols / 8, gpr = cols / gs;
    for (int r = 0; r < rows; r++) {
        for (int p = 0; p < ppr; p++) {
            uint32_t word = w[(size_t)r * ppr + p];
            int g = (p * 8) / gs;
            float sc = or_f16_to_f32(s[(size_t)r * gpr + g]);
            float bi = or_f16_to_f32(b[(size_t)r * gpr + g]);
            for (int n = 0; n < 8; n++) {
                float q = (float)((word >> (4 * n)) & 0xF);
                out[(size_t)r * cols + p * 8 + n] = q * sc + bi;
            }
        }
    }
}

/* dequant.cu:110-172: 16 two-bit codes per word, code n = (p >> 2n) & 3. */
void or_dequant_int2(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                     int rows, int cols, int gs, float* out) {
    int ppr = cols / 16, gpr = cols / gs;
    for (int r = 0; r < rows; r++) {
        for (int p = 0; p < ppr; p++) {
            uint32_t word = w[(size_t)r * ppr + p];
            int g = (p * 16) / gs;
            float sc = or_f16_to_f32(s[(size_t)r * gpr + g]);
            float bi = or_f16_to_f32(b[(size_t)r * gpr + g]);
            for (int n = 0; n < 16; n++) {
                float q = (float)((word >> (2 * n)) & 0x3);
                out[(size_t)r * cols + p * 16 + n] = q * sc + bi;
            }
        }
    }
}

/* fp4.cu:28-84: value = lut[q] * scale (fp16 group scale). */
void or_dequant_fp4(const uint32_t* w, const uint16_t* s,
                    int rows, int cols, int gs, float* out) {
    int ppr = cols / 8, gpr = cols / gs;
    for (int r = 0; r < rows; r++) {
        for (int p = 0; p < ppr; p++) {
            uint32_t word = w[(size_t)r * ppr + p];
            float sc = or_f16_to_f32(s[(size_t)r * gpr + (p * 8) / gs]);
            for (int n = 0; n < 8; n++)
                out[(size_t)r * cols + p * 8 + n] = kFp4Lut[(word >> (4 * n)) & 0xF] * sc;
        }
    }
}

/* fp4.cu:187-238: s0 = e4m3(S[r][c/16]) * g; value = lut[q] * s0; the low
 * nibble of byte c/2 is the even column. */
void or_dequant_nvfp4(const uint8_t* w, const uint8_t* s, float g,
                      int rows, int cols, float* out) {
    int bpr = cols / 2, spr = cols / 16;
    for (int r = 0; r < rows; r++) {
        for (int c = 0; c < cols; c++) {
            uint8_t byte = w[(size_t)r * bpr + c / 2];
            uint8_t q = (c & 1) ? (byte >> 4) : (byte & 0xF);
            float s0 = or_e4m3_ref_to_f32(s[(size_t)r * spr + c / 16]) * g;
            out[(size_t)r * cols + c] = kFp4Lut[q] * s0;
        }
    }
}

/* ggml Q4_K, 144-byte block {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}
 * (block geometry: gguf_loader.h:62-100).  Sub-block j's 6-bit (sc, m). */
static void q4k_scale_min(const uint8_t* q, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

void or_dequant_q4k(const uint8_t* blocks, int rows, int cols, float* out) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        for (int ib = 0; ib < nb; ib++) {
            const uint8_t* blk = blocks + ((size_t)r * nb + ib) * 144;
            uint16_t dh, mh;
            memcpy(&dh, blk, 2);
            memcpy(&mh, blk + 2, 2);
            float d = or_f16_to_f32(dh), dmin = or_f16_to_f32(mh);
            const uint8_t* sc12 = blk + 4;
            const uint8_t* qs = blk + 16;
            float* y = out + (size_t)r * cols + ib * 256;
            for (int c = 0; c < 4; c++) {
                int sc0, m0, sc1, m1;
                q4k_scale_min(sc12, 2 * c, &sc0, &m0);
                q4k_scale_min(sc12, 2 * c + 1, &sc1, &m1);
                float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                for (int l = 0; l < 32; l++) {
                    y[64 * c + l] = d1 * (float)(qs[32 * c + l] & 0xF) - mm1;
                    y[64 * c + 32 + l] = d2 * (float)(qs[32 * c + l] >> 4) - mm2;
                }
            }
        }
    }
}

/* ggml Q3_K, 110-byte block {u8 hmask[32]; u8 qs[64]; u8 scales[12]; f16 d}.
 * Element 128h + 32j + l (l < 32): 2-bit code (qs[32h+l] >> 2j) & 3, minus 4
 * unless bit (4h+j) of hmask[l] is set; scale index 8h + 2j + (l >= 16). */
static int q3k_scale(const uint8_t* s, int k) {
    int lo = k < 8 ? (s[k] & 0xF) : (s[k - 8] >> 4);
    int hi = (s[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

void or_dequant_q3k(const uint8_t* blocks, int rows, int cols, float* out) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        for (int ib = 0; ib < nb; ib++) {
            const uint8_t* blk = blocks + ((size_t)r * nb + ib) * 110;
            const uint8_t* hm = blk;
            const uint8_t* qs = blk + 32;
            const uint8_t* sc = blk + 96;
            uint16_t dh;
            memcpy(&dh, blk + 108, 2);
            float d = or_f16_to_f32(dh);
            float* y = out + (size_t)r * cols + ib * 256;
            for (int h = 0; h < 2; h++) {
                for (int j = 0; j < 4; j++) {
                    for (int l = 0; l < 32; l++) {
                        int k = 8 * h + 2 * j + (l >= 16);
                        float dl = d * (float)q3k_scale(sc, k);
                        int q = (qs[32 * h + l] >> (2 * j)) & 3;
                        int m = (hm[l] >> (4 * h + j)) & 1;
                        y[128 * h + 32 * j + l] = dl * (float)(q - (m ? 0 : 4));
                    }
                }
            }
        }
    }
}

void or_dequant_fp8(const uint8_t* w, const float* cs, int rows, int cols, float* out) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++)
            out[(size_t)r * cols + c] = or_e4m3_ocp_to_f32(w[(size_t)r * cols + c]) * cs[r];
}

/* ======================================================================== */
/* dense references                                                         */
/* ======================================================================== */

void or_gemm_f32(const float* W, const float* X, int M, int N, int K, float* Y) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            const float* w = W + (size_t)n * K;
            const float* x = X + (size_t)m * K;
            for (int k = 0; k < K; k++) acc += w[k] * x[k];
            Y[(size_t)m * N + n] = acc;
        }
}

void or_gemm_f64(const float* W, const float* X, int M, int N, int K, double* Y) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            const float* w = W + (size_t)n * K;
            const float* x = X + (size_t)m * K;
            for (int k = 0; k < K; k++) acc += (double)w[k] * (double)x[k];
            Y[(size_t)m * N + n] = acc;
        }
}

/* ======================================================================== */
/* reference-loop GEMVs and the CPU baseline                                */
/* ======================================================================== */

static void int4_rows(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                      const float* x, float* y, int r0, int r1, int cols, int gs) {
    int ppr = cols / 8, gpr = cols / gs;
    for (int r = r0; r < r1; r++) {
        float acc = 0.0f;
        const uint32_t* rw = w + (size_t)r * ppr;
        for (int p = 0; p < ppr; p++) {
            uint32_t packed = rw[p];
            int base = p * 8;
            int g = base / gs;
            float sc = or_f16_to_f32(s[(size_t)r * gpr + g]);
            float bi = or_f16_to_f32(b[(size_t)r * gpr + g]);
            for (int n = 0; n < 8 && base + n < cols; n++) {
                float q = (float)((packed >> (n * 4)) & 0xF);
                /* the reference's -O3 -march=native build contracts
                 * acc += t * x into one FMA (checked against oracle/_ref) */
                acc = fmaf(q * sc + bi, x[base + n], acc);
            }
        }
        y[r] = acc;
    }
}

void or_matvec_int4_cpu(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                        const float* x, float* y, int rows, int cols, int gs) {
    int4_rows(w, s, b, x, y, 0, rows, cols, gs);
}

typedef struct {
    int fmt;
    const void *codes, *s, *b;
    float g;
    int gs;
    const float* x;
    float* y;
    int r0, r1, cols;
} RowJob;

static void fmt_rows(const RowJob* j) {
    int cols = j->cols;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)cols);
    for (int r = j->r0; r < j->r1; r++) {
        switch (j->fmt) {
            case 0:
                int4_rows((const uint32_t*)j->codes, (const uint16_t*)j->s,
                          (const uint16_t*)j->b, j->x, j->y, r, r + 1, cols, j->gs);
                continue;
            case 1:
                or_dequant_int2((const uint32_t*)j->codes + (size_t)r * (cols / 16),
                                (const uint16_t*)j->s + (size_t)r * (cols / j->gs),
                                (const uint16_t*)j->b + (size_t)r * (cols / j->gs),
                                1, cols, j->gs, wrow);
                break;
            case 2:
                or_dequant_nvfp4((const uint8_t*)j->codes + (size_t)r * (cols / 2),
                                 (const uint8_t*)j->s + (size_t)r * (cols / 16), j->g,
                                 1, cols, wrow);
                break;
            case 3:
                or_dequant_q4k((const uint8_t*)j->codes + (size_t)r * (cols / 256) * 144,
                               1, cols, wrow);
                break;
            case 4:
                or_dequant_q3k((const uint8_t*)j->codes + (size_t)r * (cols / 256) * 110,
                               1, cols, wrow);
                break;
            default:
                or_dequant_fp8((const uint8_t*)j->codes + (size_t)r * cols,
                               (const float*)j->s + r, 1, cols, wrow);
                break;
        }
        float acc = 0.0f;
        for (int c = 0; c < cols; c++) acc = fmaf(wrow[c], j->x[c], acc);
        j->y[r] = acc;
    }
    free(wrow);
}

static void* fmt_rows_thread(void* arg) {
    fmt_rows((const RowJob*)arg);
    return NULL;
}

void or_matvec_fmt_mt(int fmt, const void* codes, const void* s, const void* b,
                      float g, int gs, const float* x, float* y, int rows,
                      int cols, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > rows) nthreads = rows;
    RowJob* jobs = (RowJob*)calloc((size_t)nthreads, sizeof(RowJob));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; t++) {
        RowJob j = {fmt, codes, s, b, g, gs, x, y,
                    (int)((long long)rows * t / nthreads),
                    (int)((long long)rows * (t + 1) / nthreads), cols};
        jobs[t] = j;
    }
    for (int t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, fmt_rows_thread, &jobs[t]);
    fmt_rows(&jobs[0]);
    for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
    free(jobs);
    free(th);
}

void or_matvec_int4_cpu_mt(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                           const float* x, float* y, int rows, int cols, int gs,
                           int nthreads) {
    or_matvec_fmt_mt(0, w, s, b, 1.0f, gs, x, y, rows, cols, nthreads);
}

void or_matvec_nvfp4(const uint8_t* w, const uint8_t* s, float g,
                     const float* x, float* y, int rows, int cols) {
    int bpr = cols / 2, spr = cols / 16;
    for (int r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (int bc = 0; bc < bpr; bc++) {
            uint8_t packed = w[(size_t)r * bpr + bc];
            int c0 = 2 * bc, c1 = c0 + 1;
            float s0 = or_e4m3_ref_to_f32(s[(size_t)r * spr + c0 / 16]) * g;
            float s1 = or_e4m3_ref_to_f32(s[(size_t)r * spr + c1 / 16]) * g;
            acc += kFp4Lut[packed & 0xF] * s0 * x[c0];
            acc += kFp4Lut[packed >> 4] * s1 * x[c1];
        }
        y[r] = acc;
    }
}

/* ======================================================================== */
/* quantizers (fixture generators)                                          */
/* ======================================================================== */

/* convert_titan.py:43-77: per group gmin/gmax in fp32; scale =
 * max((gmax-gmin)/15, 1e-10); bias = gmin; q = clamp(rne((w-bias)/scale), 0,
 * 15); scale and bias stored as fp16 (RNE); word j of the row holds columns
 * 8j..8j+7 with column 8j+n in bits 4n..4n+3. */
static void quantize_affine(const float* W, int rows, int cols, int gs, int bits,
                            uint32_t* w, uint16_t* s, uint16_t* b) {
    int per = 32 / bits, levels = (1 << bits) - 1;
    int gpr = cols / gs, ppr = cols / per;
    memset(w, 0, sizeof(uint32_t) * (size_t)rows * ppr);
    for (int r = 0; r < rows; r++) {
        for (int g = 0; g < gpr; g++) {
            const float* v = W + (size_t)r * cols + (size_t)g * gs;
            float mn = v[0], mx = v[0];
            for (int i = 1; i < gs; i++) {
                if (v[i] < mn) mn = v[i];
                if (v[i] > mx) mx = v[i];
            }
            float sc = (mx - mn) / (float)levels;
            if (sc < 1e-10f) sc = 1e-10f;
            s[(size_t)r * gpr + g] = or_f32_to_f16(sc);
            b[(size_t)r * gpr + g] = or_f32_to_f16(mn);
            for (int i = 0; i < gs; i++) {
                float q = rintf((v[i] - mn) / sc);
                if (q < 0.0f) q = 0.0f;
                if (q > (float)levels) q = (float)levels;
                int col = g * gs + i;
                w[(size_t)r * ppr + col / per] |= (uint32_t)q << (bits * (col % per));
            }
        }
    }
}

void or_quantize_int4(const float* W, int rows, int cols, int gs,
                      uint32_t* w, uint16_t* s, uint16_t* b) {
    quantize_affine(W, rows, cols, gs, 4, w, s, b);
}

void or_quantize_int2(const float* W, int rows, int cols, int gs,
                      uint32_t* w, uint16_t* s, uint16_t* b) {
    quantize_affine(W, rows, cols, gs, 2, w, s, b);
}

/* fp4.cu:126-133 magnitude thresholds; sign bit 8 for negative values. */
static uint8_t fp4_nearest(float v) {
    float a = fabsf(v);
    uint8_t n;
    if (a < 0.25f) n = 0;
    else if (a < 0.75f) n = 1;
    else if (a < 1.25f) n = 2;
    else if (a < 1.75f) n = 3;
    else if (a < 2.5f) n = 4;
    else if (a < 3.5f) n = 5;
    else if (a < 5.0f) n = 6;
    else n = 7;
    if (v < 0) n |= 8;
    return n;
}

/* fp4.cu:90-141 */
void or_quantize_fp4(const float* W, int numel, int gs, uint32_t* w, uint16_t* s) {
    int ng = numel / gs;
    memset(w, 0, sizeof(uint32_t) * (size_t)(numel / 8));
    for (int g = 0; g < ng; g++) {
        const float* v = W + (size_t)g * gs;
        float amax = 0.0f;
        for (int i = 0; i < gs; i++) if (fabsf(v[i]) > amax) amax = fabsf(v[i]);
        float sc = amax / 6.0f;
        if (sc < 1e-10f) sc = 1e-10f;
        float inv = 1.0f / sc;
        s[g] = or_f32_to_f16(sc);
        for (int i = 0; i < gs; i++) {
            int col = g * gs + i;
            w[col / 8] |= (uint32_t)fp4_nearest(v[i] * inv) << (4 * (col % 8));
        }
    }
}

/* NVFP4 producer (format of fp4.cu:162-170 / moe.cpp:609-611): per 16
 * columns, e4m3 scale = RNE(amax / 6 / g); codes by the fp4.cu thresholds on
 * v / (e4m3(scale) * g). */
void or_quantize_nvfp4(const float* W, int rows, int cols, float g,
                       uint8_t* w, uint8_t* s) {
    int bpr = cols / 2, spr = cols / 16;
    memset(w, 0, (size_t)rows * bpr);
    for (int r = 0; r < rows; r++) {
        for (int q = 0; q < spr; q++) {
            const float* v = W + (size_t)r * cols + q * 16;
            float amax = 0.0f;
            for (int i = 0; i < 16; i++) if (fabsf(v[i]) > amax) amax = fabsf(v[i]);
            uint8_t sc = or_f32_to_e4m3(amax / 6.0f / g);
            s[(size_t)r * spr + q] = sc;
            float s0 = or_e4m3_ref_to_f32(sc) * g;
            for (int i = 0; i < 16; i++) {
                uint8_t n = s0 > 0.0f ? fp4_nearest(v[i] / s0) : 0;
                int c = q * 16 + i;
                w[(size_t)r * bpr + c / 2] |= (uint8_t)(n << (4 * (c & 1)));
            }
        }
    }
}

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Simple Q4_K producer (not ggml's iterative search; any valid block is a
 * valid test input): per sub-block of 32, scale = (max - min')/15 with
 * min' = min(0, min); d, dmin = max over sub-blocks / 63 (fp16). */
void or_quantize_q4k(const float* W, int rows, int cols, uint8_t* blocks) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        for (int ib = 0; ib < nb; ib++) {
            const float* v = W + (size_t)r * cols + ib * 256;
            uint8_t* blk = blocks + ((size_t)r * nb + ib) * 144;
            float scl[8], mins[8], maxs = 0.0f, maxm = 0.0f;
            for (int j = 0; j < 8; j++) {
                float mn = 0.0f, mx = v[32 * j];
                for (int l = 0; l < 32; l++) {
                    if (v[32 * j + l] < mn) mn = v[32 * j + l];
                    if (v[32 * j + l] > mx) mx = v[32 * j + l];
                }
                if (mx < mn) mx = mn;
                scl[j] = (mx - mn) / 15.0f;
                mins[j] = -mn;
                if (scl[j] > maxs) maxs = scl[j];
                if (mins[j] > maxm) maxm = mins[j];
            }
            uint16_t dh = or_f32_to_f16(maxs / 63.0f), mh = or_f32_to_f16(maxm / 63.0f);
            float d = or_f16_to_f32(dh), dmin = or_f16_to_f32(mh);
            int sc[8], mq[8];
            for (int j = 0; j < 8; j++) {
                sc[j] = d > 0 ? clampi((int)rintf(scl[j] / d), 0, 63) : 0;
                mq[j] = dmin > 0 ? clampi((int)rintf(mins[j] / dmin), 0, 63) : 0;
            }
            memcpy(blk, &dh, 2);
            memcpy(blk + 2, &mh, 2);
            uint8_t* s12 = blk + 4;
            memset(s12, 0, 12);
            for (int j = 0; j < 4; j++) {
                s12[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
                s12[j + 4] = (uint8_t)(mq[j] | ((mq[j + 4] >> 4) << 6));
                s12[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mq[j + 4] & 0xF) << 4));
            }
            uint8_t q[256];
            for (int j = 0; j < 8; j++) {
                float ds = d * (float)sc[j], dm = dmin * (float)mq[j];
                for (int l = 0; l < 32; l++) {
                    int qq = ds > 0 ? (int)rintf((v[32 * j + l] + dm) / ds) : 0;
                    q[32 * j + l] = (uint8_t)clampi(qq, 0, 15);
                }
            }
            uint8_t* qs = blk + 16;
            for (int c = 0; c < 4; c++)
                for (int l = 0; l < 32; l++)
                    qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
        }
    }
}

/* Simple Q3_K producer: per 16-element sub-block, signed 6-bit scale of
 * amax/4 relative to d = max|scale|/31; codes in [-4, 3]. */
void or_quantize_q3k(const float* W, int rows, int cols, uint8_t* blocks) {
    int nb = cols / 256;
    for (int r = 0; r < rows; r++) {
        for (int ib = 0; ib < nb; ib++) {
            const float* v = W + (size_t)r * cols + ib * 256;
            uint8_t* blk = blocks + ((size_t)r * nb + ib) * 110;
            memset(blk, 0, 110);
            /* sub-block k covers elements 128h + 32j + 16t + (0..15) where
             * k = 8h + 2j + t */
            float sub[16], dmax = 0.0f;
            for (int k = 0; k < 16; k++) {
                int base = 128 * (k >> 3) + 32 * ((k >> 1) & 3) + 16 * (k & 1);
                float amax = 0.0f, sv = 0.0f;
                for (int l = 0; l < 16; l++)
                    if (fabsf(v[base + l]) > amax) { amax = fabsf(v[base + l]); sv = v[base + l]; }
                /* a negative scale lets the -4 end cover the largest value */
                sub[k] = sv < 0 ? amax / 4.0f : -amax / 4.0f;
                if (fabsf(sub[k]) > dmax) dmax = fabsf(sub[k]);
            }
            uint16_t dh = or_f32_to_f16(dmax / 31.0f);
            float d = or_f16_to_f32(dh);
            memcpy(blk + 108, &dh, 2);
            uint8_t* sc = blk + 96;
            uint8_t* hm = blk;
            uint8_t* qs = blk + 32;
            for (int k = 0; k < 16; k++) {
                int s6 = d > 0 ? clampi((int)rintf(sub[k] / d), -32, 31) : 0;
                int u = s6 + 32;
                if (k < 8) sc[k] |= (uint8_t)(u & 0xF);
                else sc[k - 8] |= (uint8_t)((u & 0xF) << 4);
                sc[8 + (k & 3)] |= (uint8_t)(((u >> 4) & 3) << (2 * (k >> 2)));
                float dl = d * (float)s6;
                int h = k >> 3, j = (k >> 1) & 3, t = k & 1;
                for (int l = 0; l < 16; l++) {
                    int e = 128 * h + 32 * j + 16 * t + l;
                    int q = dl != 0.0f ? clampi((int)rintf(v[e] / dl), -4, 3) : 0;
                    int u3 = q + 4;
                    int ll = 16 * t + l;
                    qs[32 * h + ll] |= (uint8_t)((u3 & 3) << (2 * j));
                    if (u3 & 4) hm[ll] |= (uint8_t)(1 << (4 * h + j));
                }
            }
        }
    }
}

void or_quantize_fp8_rows(const float* W, int rows, int cols, uint8_t* w, float* cs) {
    for (int r = 0; r < rows; r++) {
        const float* v = W + (size_t)r * cols;
        float amax = 0.0f;
        for (int c = 0; c < cols; c++) if (fabsf(v[c]) > amax) amax = fabsf(v[c]);
        float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
        cs[r] = sc;
        for (int c = 0; c < cols; c++) w[(size_t)r * cols + c] = or_f32_to_e4m3(v[c] / sc);
    }
}

/* Per-token activation quantizer; the HIP kernel computes the same
 * expressions (amax over |x|, scale = amax/448 or 1 for an all-zero row,
 * code = RNE-saturating e4m3 of x / scale), so codes match bit for bit. */
void or_quantize_act_fp8(const uint16_t* x, int M, int K, uint8_t* xq, float* xs) {
    for (int m = 0; m < M; m++) {
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = fabsf(or_bf16_to_f32(x[(size_t)m * K + k]));
            if (a > amax) amax = a;
        }
        float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
        xs[m] = sc;
        for (int k = 0; k < K; k++)
            xq[(size_t)m * K + k] = or_f32_to_e4m3(or_bf16_to_f32(x[(size_t)m * K + k]) / sc);
    }
}

void or_gemm_fp8(const uint8_t* A, const float* sa, const uint8_t* W,
                 const float* sw, int M, int N, int K, float* out) {
    float lut[256];
    for (int i = 0; i < 256; i++) lut[i] = or_e4m3_ref_to_f32((uint8_t)i);
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            const uint8_t* a = A + (size_t)m * K;
            const uint8_t* w = W + (size_t)n * K;
            for (int k = 0; k < K; k++) acc += lut[a[k]] * lut[w[k]];
            out[(size_t)m * N + n] = acc * sa[m] * sw[n];
        }
}

/* ======================================================================== */
/* MoE pieces                                                               */
/* ======================================================================== */

void or_moe_topk(const float* logits, int E, int k, float* w, int* idx) {
    float* p = (float*)malloc(sizeof(float) * (size_t)E);
    float mx = -3.402823466e+38f;
    for (int i = 0; i < E; i++) mx = fmaxf(mx, logits[i]);
    float sum = 0.0f;
    for (int i = 0; i < E; i++) { p[i] = expf(logits[i] - mx); sum += p[i]; }
    float inv = 1.0f / (sum + 1e-8f);
    for (int i = 0; i < E; i++) p[i] *= inv;
    for (int j = 0; j < k; j++) {
        float best = -1.0f;
        int bi = -1;
        for (int i = 0; i < E; i++)
            if (p[i] > best) { best = p[i]; bi = i; }
        w[j] = best;
        idx[j] = bi;
        p[bi] = -2.0f;
    }
    float ss = 0.0f;
    for (int j = 0; j < k; j++) ss += w[j];
    float invs = 1.0f / (ss + 1e-8f);
    for (int j = 0; j < k; j++) w[j] *= invs;
    free(p);
}

void or_swiglu(float* out, const float* gate, const float* up, int n) {
    for (int i = 0; i < n; i++) {
        float g = gate[i];
        float sg = 1.0f / (1.0f + expf(-g));
        out[i] = (g * sg) * up[i];
    }
}

void or_moe_combine(float* out, float* residual, const float* eo, const float* w,
                    const float* shared, float shared_w, int dim, int na) {
    for (int i = 0; i < dim; i++) {
        float c = 0.0f;
        /* nvcc contracts `combined += a * b` (default --fmad=true) */
        for (int e = 0; e < na; e++) c = fmaf(eo[(size_t)e * dim + i], w[e], c);
        if (shared) c = fmaf(shared[i], shared_w, c);
        float v = residual[i] + c;
        residual[i] = v;
        out[i] = v;
    }
}
