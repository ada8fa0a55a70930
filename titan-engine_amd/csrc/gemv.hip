// gemv.hip -- host side of the dequant-GEMV path (validation, batching,
// C ABI).  Kernels live in gemv_impl.h, instantiated by gemv_fmt_*.hip.
#include "gemv_impl.h"
#include "qgemm_tok.h"

// ============================================================================
// Host side
// ============================================================================
namespace {

// token count from which INT4 tiled weights go to the token-tiled kernel
// (8B layer: 5-8 tokens 32 us there against 33-34 us in the GEMV; 4 tokens
// 26.6 us in the GEMV)
constexpr int kTokMinTokens = 5;

using namespace tq;

bool fmt_ok(int f) {
    return f == TITAN_INT4 || f == TITAN_INT2 || f == TITAN_FP4 || f == TITAN_NVFP4 ||
           f == TITAN_Q4_K || f == TITAN_Q3_K || f == TITAN_FP8_E4M3;
}

// Validates a weight descriptor against the reference preconditions
// (dequant.cu / fp4.cu wrappers: cols % 8 (int4, fp4) or % 16 (int2, nvfp4),
// cols % group_size; K-quants cols % 256).
int check_weight(const titan_qweight* W) {
    if (!W || !W->codes || W->rows <= 0 || W->cols <= 0) return TITAN_ERR_INVALID_ARG;
    if (!fmt_ok(W->format)) return TITAN_ERR_INVALID_ARG;
    if (W->layout != TITAN_LAYOUT_REF && W->layout != TITAN_LAYOUT_TILED) return TITAN_ERR_INVALID_ARG;
    const int f = W->format, cols = W->cols, gs = W->group_size;
    switch (f) {
        case TITAN_INT4:
        case TITAN_FP4:
        case TITAN_INT2:
            if (gs <= 0 || cols % gs || gs % (f == TITAN_INT2 ? 16 : 8)) return TITAN_ERR_UNSUPPORTED;
            if (cols % (f == TITAN_INT2 ? 16 : 8)) return TITAN_ERR_UNSUPPORTED;
            if (W->layout == TITAN_LAYOUT_REF && (!W->scales || (f != TITAN_FP4 && !W->biases)))
                return TITAN_ERR_INVALID_ARG;
            break;
        case TITAN_NVFP4:
            if (cols % 16) return TITAN_ERR_UNSUPPORTED;
            if (W->layout == TITAN_LAYOUT_REF && !W->scales) return TITAN_ERR_INVALID_ARG;
            break;
        case TITAN_Q4_K:
        case TITAN_Q3_K:
            if (cols % 256) return TITAN_ERR_UNSUPPORTED;
            break;
        case TITAN_FP8_E4M3:
            if (!W->scales) return TITAN_ERR_INVALID_ARG;
            break;
    }
    if (W->layout == TITAN_LAYOUT_TILED &&
        tq::tiled_total_bytes(f, W->rows, cols, gs) == 0)
        return TITAN_ERR_UNSUPPORTED;
    return TITAN_OK;
}

// Can the fast kernel serve this weight?  (Tiled always can.)
bool fast_ok(const titan_qweight* W) {
    if (W->layout == TITAN_LAYOUT_TILED)  // tiled_total_bytes admits only fast shapes
        return ((uintptr_t)W->codes & 15) == 0;
    const int f = W->format, cols = W->cols, gs = W->group_size;
    auto al4 = [](const void* p) { return ((uintptr_t)p & 3) == 0; };
    if (!al4(W->codes)) return false;
    // 32-bit per-lane offsets
    if ((uint64_t)W->rows * (uint64_t)W->cols >= (1ull << 32)) return false;
    const bool pow2 = gs > 0 && (gs & (gs - 1)) == 0;
    switch (f) {  // whole 64-byte chunks per row; groups cover whole word steps
        case TITAN_INT4: case TITAN_FP4:
            return cols % 128 == 0 && gs % 32 == 0 && pow2 && ((uintptr_t)W->scales & 1) == 0;
        case TITAN_INT2: return cols % 256 == 0 && gs % 64 == 0 && pow2;
        case TITAN_NVFP4: return cols % 128 == 0 && al4(W->scales);
        case TITAN_Q4_K: return true;
        case TITAN_Q3_K: return false;  // 110-byte blocks: generic path
        case TITAN_FP8_E4M3: return cols % 64 == 0;
    }
    return false;
}

WDesc make_wdesc(const titan_qweight* W) {
    WDesc d;
    d.codes = (const uint8_t*)W->codes;
    d.scales = (const uint8_t*)W->scales;
    d.biases = (const uint8_t*)W->biases;
    d.g = make_geo(W->format, W->rows, W->cols, W->group_size);
    d.gscale = W->global_scale;
    d.gshift = 0;  // fast-path groups are powers of two
    for (int sh = 0; sh < 31; sh++)
        if (W->group_size == (1 << sh)) d.gshift = sh;
    return d;
}

int chunk_cols_of(int fmt) { return 512 / code_bits(fmt); }

// Runs problems [0, n) of one format/layout for tokens [0, M) in launches of
// at most 8 tokens.
int run_gemv(const titan_qweight* Ws, const void* const* Xs, const int64_t* ldx,
             void* const* Ys, const int64_t* ldy, int n, int xdt, int ydt, int M,
             hipStream_t st, void* ws = nullptr, size_t ws_bytes = 0) {
    if (n <= 0 || n > TITAN_MAX_BATCH || M <= 0) return TITAN_ERR_INVALID_ARG;
    if (!tqh::act_dtype_ok(xdt) || !tqh::act_dtype_ok(ydt)) return TITAN_ERR_INVALID_ARG;
    bool fast = true;
    for (int i = 0; i < n; i++) {
        if (int s = check_weight(&Ws[i])) return s;
        if (!Xs[i] || !Ys[i]) return TITAN_ERR_INVALID_ARG;
        if (Ws[i].format != Ws[0].format || Ws[i].layout != Ws[0].layout) return TITAN_ERR_INVALID_ARG;
        if (ldx[i] < Ws[i].cols || ldy[i] < Ws[i].rows) return TITAN_ERR_INVALID_ARG;
        fast = fast && fast_ok(&Ws[i]);
    }
    const int fmt = Ws[0].format, layout = Ws[0].layout;
    GemvArgs a{};
    a.n = n;
    a.xdt = xdt;
    a.ydt = ydt;
    a.ws = ws;
    a.ws_bytes = ws_bytes;
    int total_tiles = 0;
    bool f16 = xdt == TITAN_FP16;
    for (int i = 0; i < n; i++) {
        GemvProb& p = a.p[i];
        p.w = make_wdesc(&Ws[i]);
        p.x = Xs[i];
        p.y = Ys[i];
        p.ldx = ldx[i];
        p.ldy = ldy[i];
        p.nchunks = Ws[i].cols / chunk_cols_of(fmt);
        p.ntiles = (Ws[i].rows + 15) / 16;
        // MFMA word steps per scale group (INT4: 32 columns a step, INT2: 64)
        const int spc = fmt == TITAN_INT2 ? 64 : 32;
        const int gs = Ws[i].group_size;
        p.gsteps = gs >= 4 * spc ? 4 : (gs >= spc ? gs / spc : 1);
        total_tiles += p.ntiles;
        f16 = f16 && ((uintptr_t)Xs[i] & 15) == 0 && (ldx[i] & 7) == 0;
    }
    if (!fast) {
        // the generic kernel serves one problem per launch
        for (int i = 0; i < n; i++) {
            GemvArgs one = a;
            one.p[0] = a.p[i];
            one.n = 1;
            for (int m0 = 0; m0 < M; m0 += 8) {
                one.m0 = m0;
                int mc = M - m0 < 8 ? M - m0 : 8;
                switch (fmt) {
                    case TITAN_INT4: dispatch_gemv_generic_int4(one, mc, Ws[i].rows, st); break;
                    case TITAN_INT2: dispatch_gemv_generic_int2(one, mc, Ws[i].rows, st); break;
                    case TITAN_FP4: dispatch_gemv_generic_fp4(one, mc, Ws[i].rows, st); break;
                    case TITAN_NVFP4: dispatch_gemv_generic_nvfp4(one, mc, Ws[i].rows, st); break;
                    case TITAN_Q4_K: dispatch_gemv_generic_q4k(one, mc, Ws[i].rows, st); break;
                    case TITAN_Q3_K: dispatch_gemv_generic_q3k(one, mc, Ws[i].rows, st); break;
                    default: dispatch_gemv_generic_fp8(one, mc, Ws[i].rows, st); break;
                }
            }
        }
        return tqh::launch_status();
    }
    // several tokens of INT4 tiled weights: the token-tiled dequant-GEMM
    if (M >= kTokMinTokens && tqh::tok_int4_ok(Ws, Xs, ldx, n, xdt))
        return tqh::run_tok_int4(Ws, Xs, ldx, Ys, ldy, n, xdt, ydt, M, st);
    bool has_mfma = false;
    switch (fmt) {
        case TITAN_INT4: has_mfma = gemv_has_mfma_int4(); break;
        case TITAN_INT2: has_mfma = gemv_has_mfma_int2(); break;
        case TITAN_Q4_K: has_mfma = gemv_has_mfma_q4k(); break;
        case TITAN_Q3_K: has_mfma = gemv_has_mfma_q3k(); break;
        default: break;
    }
    // one group size per launch (the kernels take the word steps per group
    // as a template parameter); mixed group sizes go one problem at a time
    for (int i = 1; i < n; i++)
        if (a.p[i].gsteps != a.p[0].gsteps) {
            for (int q = 0; q < n; q++) {
                int s = run_gemv(&Ws[q], &Xs[q], &ldx[q], &Ys[q], &ldy[q], 1, xdt, ydt, M, st, ws, ws_bytes);
                if (s) return s;
            }
            return TITAN_OK;
        }
    const int mode = !f16 ? kModeF32 : (has_mfma ? kModeMfma : kModeDot2);
    // MFMA: up to 32 tokens a launch; 256-column chunks (INT2, Q3_K) stage
    // twice the columns per round, so 16 (32 would need 256 KiB of LDS)
    const int per_launch = mode != kModeMfma ? 8 : chunk_cols_of(fmt) > 128 ? 16 : 32;
    for (int m0 = 0; m0 < M; m0 += per_launch) {
        a.m0 = m0;
        int mc = M - m0 < per_launch ? M - m0 : per_launch;
        switch (fmt) {
            case TITAN_INT4: dispatch_gemv_int4(a, layout, mc, mode, total_tiles, st); break;
            case TITAN_INT2: dispatch_gemv_int2(a, layout, mc, mode, total_tiles, st); break;
            case TITAN_FP4: dispatch_gemv_fp4(a, layout, mc, mode, total_tiles, st); break;
            case TITAN_NVFP4: dispatch_gemv_nvfp4(a, layout, mc, mode, total_tiles, st); break;
            case TITAN_Q4_K: dispatch_gemv_q4k(a, layout, mc, mode, total_tiles, st); break;
            case TITAN_Q3_K: dispatch_gemv_q3k(a, layout, mc, mode, total_tiles, st); break;
            default: dispatch_gemv_fp8(a, layout, mc, mode, total_tiles, st); break;
        }
    }
    return tqh::launch_status();
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================
extern "C" int titan_qgemm(const titan_qweight* W, const void* X, int x_dtype, int64_t ldx,
                           void* Y, int y_dtype, int64_t ldy, int M, hipStream_t stream) {
    if (!W) return TITAN_ERR_INVALID_ARG;
    const void* xs[1] = {X};
    void* ys[1] = {Y};
    return run_gemv(W, xs, &ldx, ys, &ldy, 1, x_dtype, y_dtype, M, stream);
}

extern "C" int titan_qgemm_batched(const titan_qweight* Ws, const void* const* Xs,
                                   void* const* Ys, int n, int x_dtype, int y_dtype, int M,
                                   hipStream_t stream) {
    if (!Ws || !Xs || !Ys || n <= 0 || n > TITAN_MAX_BATCH) return TITAN_ERR_INVALID_ARG;
    int64_t ldx[TITAN_MAX_BATCH], ldy[TITAN_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        ldx[i] = Ws[i].cols;
        ldy[i] = Ws[i].rows;
    }
    return run_gemv(Ws, Xs, ldx, Ys, ldy, n, x_dtype, y_dtype, M, stream);
}

// ---- K split across workgroups (caller workspace) ---------------------------
extern "C" size_t titan_qgemm_workspace_bytes(const int* rows, int n, int M) {
    if (!rows || n <= 0 || n > TITAN_MAX_BATCH || M <= 0) return 0;
    const int m = M < 32 ? M : 32;  // tokens per launch at most
    size_t b = kGemvXsCntBytes;
    for (int i = 0; i < n; i++) {
        if (rows[i] <= 0) return 0;
        b += gemv_xs_part_bytes(rows[i], m);
    }
    return b;
}

static int ws_check(const titan_qweight* Ws, int n, int M, const void* ws, size_t ws_bytes) {
    if (!ws || ((uintptr_t)ws & 255)) return TITAN_ERR_INVALID_ARG;
    int rows[TITAN_MAX_BATCH];
    for (int i = 0; i < n; i++) rows[i] = Ws[i].rows;
    const size_t need = titan_qgemm_workspace_bytes(rows, n, M);
    return need == 0 ? TITAN_ERR_INVALID_ARG : (ws_bytes < need ? TITAN_ERR_WORKSPACE : TITAN_OK);
}

extern "C" int titan_qgemm_ws(const titan_qweight* W, const void* X, int x_dtype, int64_t ldx,
                              void* Y, int y_dtype, int64_t ldy, int M, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
    if (!W || M <= 0 || W->rows <= 0) return TITAN_ERR_INVALID_ARG;
    if (int s = ws_check(W, 1, M, workspace, workspace_bytes)) return s;
    const void* xs[1] = {X};
    void* ys[1] = {Y};
    return run_gemv(W, xs, &ldx, ys, &ldy, 1, x_dtype, y_dtype, M, stream, workspace,
                    workspace_bytes);
}

extern "C" int titan_qgemm_batched_ws(const titan_qweight* Ws, const void* const* Xs,
                                      void* const* Ys, int n, int x_dtype, int y_dtype, int M,
                                      void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
    if (!Ws || !Xs || !Ys || n <= 0 || n > TITAN_MAX_BATCH || M <= 0) return TITAN_ERR_INVALID_ARG;
    for (int i = 0; i < n; i++)
        if (Ws[i].rows <= 0) return TITAN_ERR_INVALID_ARG;
    if (int s = ws_check(Ws, n, M, workspace, workspace_bytes)) return s;
    int64_t ldx[TITAN_MAX_BATCH], ldy[TITAN_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        ldx[i] = Ws[i].cols;
        ldy[i] = Ws[i].rows;
    }
    return run_gemv(Ws, Xs, ldx, Ys, ldy, n, x_dtype, y_dtype, M, stream, workspace,
                    workspace_bytes);
}

extern "C" int titan_qdequant(const titan_qweight* W, void* out, int out_dtype,
                              hipStream_t stream) {
    if (int s = check_weight(W)) return s;
    if (!out || !tqh::act_dtype_ok(out_dtype)) return TITAN_ERR_INVALID_ARG;
    WDesc d = make_wdesc(W);
    int64_t n = (int64_t)W->rows * W->cols;
    int blocks = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    bool tiled = W->layout == TITAN_LAYOUT_TILED;
#define TQ_DQ(FMTV)                                                                               \
    case FMTV:                                                                                    \
        if (tiled)                                                                                \
            hipLaunchKernelGGL((qdequant_kernel<FMTV, TITAN_LAYOUT_TILED>), dim3(blocks), dim3(256), \
                               0, stream, d, out, out_dtype);                                     \
        else                                                                                      \
            hipLaunchKernelGGL((qdequant_kernel<FMTV, TITAN_LAYOUT_REF>), dim3(blocks), dim3(256),   \
                               0, stream, d, out, out_dtype);                                     \
        break;
    switch (W->format) {
        TQ_DQ(TITAN_INT4)
        TQ_DQ(TITAN_INT2)
        TQ_DQ(TITAN_FP4)
        TQ_DQ(TITAN_NVFP4)
        TQ_DQ(TITAN_Q4_K)
        TQ_DQ(TITAN_Q3_K)
        TQ_DQ(TITAN_FP8_E4M3)
    }
#undef TQ_DQ
    return tqh::launch_status();
}

// ---- reference-signature entry points (dispatch.h) ------------------------------
static int ref_matvec(int fmt, const void* w, const void* s, const void* b, float g,
                      const float* x, float* y, int rows, int cols, int gs, hipStream_t st) {
    titan_qweight W{};
    W.format = fmt;
    W.layout = TITAN_LAYOUT_REF;
    W.rows = rows;
    W.cols = cols;
    W.group_size = gs;
    W.global_scale = g;
    W.codes = w;
    W.scales = s;
    W.biases = b;
    return titan_qgemm(&W, x, TITAN_FP32, cols, y, TITAN_FP32, rows, 1, st);
}

extern "C" int titan_dequant_matvec_int4(const void* weights, const void* scales,
                                         const void* biases, const float* input, float* output,
                                         int rows, int cols, int group_size, hipStream_t stream) {
    return ref_matvec(TITAN_INT4, weights, scales, biases, 1.0f, input, output, rows, cols,
                      group_size, stream);
}
extern "C" int titan_dequant_matvec_int2(const void* weights, const void* scales,
                                         const void* biases, const float* input, float* output,
                                         int rows, int cols, int group_size, hipStream_t stream) {
    return ref_matvec(TITAN_INT2, weights, scales, biases, 1.0f, input, output, rows, cols,
                      group_size, stream);
}
extern "C" int titan_dequant_matvec_fp4(const void* weights, const void* scales, const float* input,
                                        float* output, int rows, int cols, int group_size,
                                        hipStream_t stream) {
    return ref_matvec(TITAN_FP4, weights, scales, nullptr, 1.0f, input, output, rows, cols,
                      group_size, stream);
}
extern "C" int titan_dequant_matvec_nvfp4(const void* weights, const void* scales,
                                          float global_scale, const float* input, float* output,
                                          int rows, int cols, hipStream_t stream) {
    return ref_matvec(TITAN_NVFP4, weights, scales, nullptr, global_scale, input, output, rows,
                      cols, 16, stream);
}
