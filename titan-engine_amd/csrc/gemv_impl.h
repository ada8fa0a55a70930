// gemv.hip -- dequant-GEMV / small-M dequant-GEMM for decode (VALU path).
//
// Replaces the reference's one-block-per-row kernels (dequant.cu:23-172,
// fp4.cu:28-84, fp4.cu:187-238).  Design for gfx950:
//  * A workgroup of 4 waves owns RT tiles of 16 rows and the whole K range.
//    The waves split K (wave w takes 64-byte chunks w, w+4, ...), so at any
//    moment the workgroup streams 256 contiguous code bytes per row, and each
//    wave keeps its next chunk's loads in flight while folding the current.
//  * Lane l = 16*j + r loads row r's 16-byte slot j of a chunk with one
//    128-bit load; in the tiled layout a wave's 64 loads are 1 KiB contiguous.
//  * Activations are staged once per workgroup into LDS as fp32 (phases of
//    at most 40 KiB for long K / many tokens) and read back as 128-bit
//    vectors; each activation segment is reused across the RT row tiles.
//  * Dequantization happens in registers: affine formats fold as
//    scale * sum(q*x) + bias * sum(x); lanes of a row are reduced with two
//    cross-lane shuffles, waves through LDS.
#pragma once
#include "formats.h"

namespace tq {

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kGemvLdsBytes = 16 * 1024;  // activation stage per workgroup

struct GemvProb {
    WDesc w;
    const void* x;
    void* y;
    int64_t ldx, ldy;
    int nchunks;   // ceil(cols / CHUNK_COLS)
    int wg_begin;  // first workgroup of this problem
    int ntiles;    // ceil(rows / 16)
};

struct GemvArgs {
    GemvProb p[TITAN_MAX_BATCH];
    int n;
    int xdt, ydt;
    int m0;   // first token of this launch (launches cover <= 8 tokens)
    int mcount;  // tokens in this launch (<= the kernel's template width)
    int pc;   // staged columns per phase (multiple of kGemvWaves * CHUNK_COLS)
};

// Stage x[m0 .. m0+M)[col0 .. col0+ncols) into lds[m][0 .. ncols) as fp32.
template <int M>
TQ_DEV void stage_x(float* lds, int pc, const void* x, int xdt, int64_t ldx, int m0, int mcount,
                    int col0, int ncols, int tid) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int64_t off = (int64_t)(m0 + m) * ldx + col0;
        float* dst = lds + m * pc;
        if (m >= mcount) {  // padding token of a narrower launch
            for (int c = tid; c < ncols; c += kGemvThreads) dst[c] = 0.0f;
        } else if (xdt == TITAN_FP32) {
            const float* src = (const float*)x + off;
            for (int c = tid; c < ncols; c += kGemvThreads) dst[c] = src[c];
        } else if (xdt == TITAN_FP16) {
            const _Float16* src = (const _Float16*)x + off;
            for (int c = tid; c < ncols; c += kGemvThreads) dst[c] = (float)src[c];
        } else {
            const uint16_t* src = (const uint16_t*)x + off;
            for (int c = tid; c < ncols; c += kGemvThreads) dst[c] = bf16_to_f32(src[c]);
        }
    }
}

// fp16 activations: stage x[m0 .. m0+M)[col0 .. col0+ncols) as fp16,
// permuted inside groups of PERM columns so that one 128-bit LDS read gives
// the activation pairs a format's masked code pairs multiply (PERM 8:
// (n, n+4); 16: (n, n+8); 4: (0, 2), (1, 3)), plus the fp32 sum of every 16
// columns.  ncols is a multiple of 16 and rows of x are 16-byte aligned.
template <int M, int PERM>
TQ_DEV void stage_x_h(_Float16* xh, float* xs, int pc, const void* x, int64_t ldx, int m0,
                      int mcount, int col0, int ncols, int tid) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const _Float16* src = (const _Float16*)x + (int64_t)(m0 + m) * ldx + col0;
        for (int c = tid * 16; c < ncols; c += kGemvThreads * 16) {
            _Float16 h[16], o[16];
            if (m < mcount) {
                const uint4 a = *(const uint4*)(src + c), b = *(const uint4*)(src + c + 8);
                const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    h[2 * i] = __builtin_bit_cast(_Float16, (uint16_t)(v[i] & 0xFFFF));
                    h[2 * i + 1] = __builtin_bit_cast(_Float16, (uint16_t)(v[i] >> 16));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) h[i] = (_Float16)0.0f;
            }
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                s0 += (float)h[i];
                s1 += (float)h[i + 1];
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                int g, n, src_i;
                if constexpr (PERM == 8) { g = i & 8; n = (i & 7) >> 1; src_i = g + n + 4 * (i & 1); }
                else if constexpr (PERM == 16) { n = i >> 1; src_i = n + 8 * (i & 1); }
                else { g = i & 12; n = i & 3; src_i = g + (n == 1 ? 2 : n == 2 ? 1 : n); }
                o[i] = h[src_i];
            }
            uint32_t ov[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                ov[i] = (uint32_t)__builtin_bit_cast(uint16_t, o[2 * i]) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, o[2 * i + 1]) << 16);
            *(uint4*)(xh + m * pc + c) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
            *(uint4*)(xh + m * pc + c + 8) = make_uint4(ov[4], ov[5], ov[6], ov[7]);
            xs[m * (pc / 16) + c / 16] = s0 + s1;
        }
    }
}

template <class F, int M, int RT, bool HX>
__global__ __launch_bounds__(kGemvThreads) void qgemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    int bid = blockIdx.x, pi = 0;
    for (int i = 1; i < a.n; i++)
        if (bid >= a.p[i].wg_begin) pi = i;
    const GemvProb& P = a.p[pi];
    const WDesc& W = P.w;
    const int rows = W.g.rows, cols = W.g.cols, nchunks = P.nchunks;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, j = lane >> 4;
    const int tile0 = (bid - P.wg_begin) * RT;
    const int pc = a.pc;

    int rowt[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        int row = (tile0 + t) * 16 + r;
        rowt[t] = row < rows ? row : rows - 1;  // clamp loads; stores are masked
    }

    float acc[RT][M];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[t][m] = 0.0f;

    // Wave w folds chunks w, w + 4, w + 8, ... in groups of U; two groups of
    // codes are held in registers so that the next group's loads (U*RT KiB
    // per wave) are in flight while the current group is folded.  Every wave
    // runs the same number of groups (out-of-range chunks are masked) so the
    // activation-staging barriers line up.
    constexpr int U = 4 / RT;
    constexpr int GCH = kGemvWaves * U;  // chunks consumed per group by the workgroup
    const int ngroups = (nchunks + GCH - 1) / GCH;
    const int pgroups = pc / (F::CHUNK_COLS * GCH);  // groups per staged phase

    auto chunk_of = [&](int g, int u) { return (g * U + u) * kGemvWaves + wave; };
    auto valid = [&](int cc) { return cc < nchunks && cc * F::CHUNK_COLS + j * F::SLOT_COLS < cols; };
    // Loads are unconditional (a masked chunk re-reads chunk 0, slot 0, which
    // always exists), so no branch forces an early wait on loads in flight.
    auto load_group = [&](int g, typename F::Raw (&R)[U][RT]) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int cc = chunk_of(g, u);
            const bool ok = valid(cc);
#pragma unroll
            for (int t = 0; t < RT; t++) F::load(W, rowt[t], ok ? cc : 0, ok ? j : 0, R[u][t]);
        }
    };
    auto fold_group = [&](int g, const typename F::Raw (&R)[U][RT]) {
        if (g % pgroups == 0) {  // first group of a phase: stage its activations
            const int col0 = (g / pgroups) * pc;
            __syncthreads();
            if constexpr (HX)
                stage_x_h<M, F::PERM>((_Float16*)lds, lds + M * pc / 2, pc, P.x, P.ldx, a.m0,
                                      a.mcount, col0, min(pc, cols - col0), tid);
            else
                stage_x<M>(lds, pc, P.x, a.xdt, P.ldx, a.m0, a.mcount, col0,
                           min(pc, cols - col0), tid);
            __syncthreads();
        }
        const int col0 = (g / pgroups) * pc;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int cc = chunk_of(g, u);
            if (!valid(cc)) continue;
            const int lbase = cc * F::CHUNK_COLS - col0;
            typename F::Dec dec[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) dec[t] = F::decode(W, R[u][t], cc, j);
            if constexpr (HX) {
                const _Float16* xh = (const _Float16*)lds;
                const float* xsum = lds + M * pc / 2;
#pragma unroll
                for (int m = 0; m < M; m++) {
#pragma unroll
                    for (int s = 0; s < F::SEGS; s++) {
                        const int lc = lbase + F::seg_col(j, s);
                        const uint4* xp = (const uint4*)(xh + m * pc + lc);
                        float sx = 0.0f;
                        if constexpr (F::NEEDS_SX) {
#pragma unroll
                            for (int q = 0; q < F::SEGW / 16; q++) sx += xsum[m * (pc / 16) + lc / 16 + q];
                        }
#pragma unroll
                        for (int t = 0; t < RT; t++) acc[t][m] += F::seg_dot_h(R[u][t], dec[t], s, xp, sx);
                    }
                }
                continue;
            }
#pragma unroll
            for (int m = 0; m < M; m++) {
#pragma unroll
                for (int s = 0; s < F::SEGS; s++) {
                    float xv[F::SEGW];
                    const float4* xp = (const float4*)&lds[m * pc + lbase + F::seg_col(j, s)];
#pragma unroll
                    for (int v = 0; v < F::SEGW / 4; v++) {
                        float4 q = xp[v];
                        xv[4 * v] = q.x;
                        xv[4 * v + 1] = q.y;
                        xv[4 * v + 2] = q.z;
                        xv[4 * v + 3] = q.w;
                    }
                    float sx = 0.0f;
                    if constexpr (F::NEEDS_SX) {
                        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                        for (int v = 0; v < F::SEGW; v += 2) {
                            s0 += xv[v];
                            s1 += xv[v + 1];
                        }
                        sx = s0 + s1;
                    }
#pragma unroll
                    for (int t = 0; t < RT; t++) acc[t][m] += F::seg_dot(R[u][t], dec[t], s, xv, sx);
                }
            }
        }
    };

    typename F::Raw ra[U][RT], rb[U][RT];
    load_group(0, ra);
    for (int g = 0; g < ngroups; g += 2) {
        if (g + 1 < ngroups) load_group(g + 1, rb);
        fold_group(g, ra);
        if (g + 1 >= ngroups) break;
        if (g + 2 < ngroups) load_group(g + 2, ra);
        fold_group(g + 1, rb);
    }

    // reduce: 4 slots of a row inside the wave, then the waves via LDS
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int m = 0; m < M; m++) acc[t][m] = sum_slots(acc[t][m]);
    __syncthreads();
    if (j == 0) {
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int m = 0; m < M; m++) lds[((wave * RT + t) * M + m) * 16 + r] = acc[t][m];
    }
    __syncthreads();
    for (int o = tid; o < RT * M * 16; o += kGemvThreads) {
        const int rr = o & 15, m = (o >> 4) % M, t = (o >> 4) / M;
        const int row = (tile0 + t) * 16 + rr;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kGemvWaves; w++) v += lds[((w * RT + t) * M + m) * 16 + rr];
        if (row < rows && m < a.mcount) {
            if constexpr (F::FMT == TITAN_NVFP4) v *= W.gscale;
            if constexpr (F::FMT == TITAN_FP8_E4M3) v *= ((const float*)W.scales)[row];
            store_out(P.y, (int64_t)(a.m0 + m) * P.ldy + row, a.ydt, v);
        }
    }
}

// ---- generic fallback for ragged REF shapes: one workgroup per row -------------
template <int FMT, int M>
__global__ __launch_bounds__(256) void qgemv_generic_kernel(GemvArgs a) {
    __shared__ float red[M][4];
    const GemvProb& P = a.p[0];
    const WDesc& W = P.w;
    const int row = blockIdx.x;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;
    for (int c = threadIdx.x; c < W.g.cols; c += 256) {
        float w = elem<FMT, TITAN_LAYOUT_REF>(W, row, c);
#pragma unroll
        for (int m = 0; m < M; m++) acc[m] += w * load_act(P.x, (int64_t)(a.m0 + m) * P.ldx + c, a.xdt);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = wave_sum(acc[m]);
        if (lane == 0) red[m][wave] = v;
    }
    __syncthreads();
    if (threadIdx.x < M) {
        const int m = threadIdx.x;
        float v = red[m][0] + red[m][1] + red[m][2] + red[m][3];
        store_out(P.y, (int64_t)(a.m0 + m) * P.ldy + row, a.ydt, v);
    }
}

// ---- exact dequantization: one thread per element --------------------------------
template <int FMT, int LAYOUT>
__global__ __launch_bounds__(256) void qdequant_kernel(WDesc w, void* out, int odt) {
    const int64_t n = (int64_t)w.g.rows * w.g.cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const int row = (int)(i / w.g.cols), col = (int)(i % w.g.cols);
        store_out(out, i, odt, elem<FMT, LAYOUT>(w, row, col));
    }
}

}  // namespace tq


namespace tq {
template <int FMT, int LAYOUT> struct Pick;
template <int L> struct Pick<TITAN_INT4, L> { using type = FmtInt4<L>; };
template <int L> struct Pick<TITAN_INT2, L> { using type = FmtInt2<L>; };
template <int L> struct Pick<TITAN_FP4, L> { using type = FmtFp4<L>; };
template <int L> struct Pick<TITAN_NVFP4, L> { using type = FmtNvfp4<L>; };
template <int L> struct Pick<TITAN_Q4_K, L> { using type = FmtQ4K<L>; };
template <int L> struct Pick<TITAN_Q3_K, L> { using type = FmtQ3K<L>; };
template <int L> struct Pick<TITAN_FP8_E4M3, L> { using type = FmtFp8<L>; };

template <class F, int M, bool HX>
void launch_fast_m(GemvArgs& a, int total_tiles, hipStream_t st) {
    // Four row tiles per workgroup for large problems (and for many tokens,
    // which keeps the activation stage small); one tile otherwise.
    const int rt = (total_tiles >= 4 * 1024 || M > 4) ? 4 : 1;
    // phase width: whole groups of chunks, at most kGemvLdsBytes of staged
    // activations (fp32, or fp16 + per-16 sums), at least one group, no
    // wider than the longest row
    const int step = kGemvWaves * (4 / rt) * F::CHUNK_COLS;
    int maxcols = 0;
    for (int i = 0; i < a.n; i++) maxcols = maxcols > a.p[i].w.g.cols ? maxcols : a.p[i].w.g.cols;
    const int per_col_x4 = HX ? 9 : 16;  // 4 x bytes per column per token
    int cap = (kGemvLdsBytes * 4 / per_col_x4 / M) / step * step;
    if (cap < step) cap = step;
    int need = (maxcols + step - 1) / step * step;
    a.pc = need < cap ? need : cap;
    const size_t stage = (size_t)M * a.pc * per_col_x4 / 4;
    const size_t red = (size_t)kGemvWaves * rt * M * 16 * 4;
    const size_t lds = stage > red ? stage : red;
    int wg = 0;
    for (int i = 0; i < a.n; i++) {
        a.p[i].wg_begin = wg;
        wg += (a.p[i].ntiles + rt - 1) / rt;
    }
    if (rt == 4)
        hipLaunchKernelGGL((qgemv_kernel<F, M, 4, HX>), dim3(wg), dim3(kGemvThreads), lds, st, a);
    else
        hipLaunchKernelGGL((qgemv_kernel<F, M, 1, HX>), dim3(wg), dim3(kGemvThreads), lds, st, a);
}

template <class F, int M>
void launch_fast_m(GemvArgs& a, int total_tiles, hipStream_t st) {
    // fp16 activations with 16-byte aligned rows take the packed fp16 path
    bool hx = a.xdt == TITAN_FP16;
    for (int i = 0; i < a.n; i++)
        hx = hx && ((uintptr_t)a.p[i].x & 15) == 0 && (a.p[i].ldx & 7) == 0;
    if (hx) launch_fast_m<F, M, true>(a, total_tiles, st);
    else launch_fast_m<F, M, false>(a, total_tiles, st);
}

template <class F>
void launch_fast(GemvArgs& a, int mcount, int total_tiles, hipStream_t st) {
    a.mcount = mcount;
    if (mcount == 1) launch_fast_m<F, 1>(a, total_tiles, st);
    else if (mcount == 2) launch_fast_m<F, 2>(a, total_tiles, st);
    else if (mcount <= 4) launch_fast_m<F, 4>(a, total_tiles, st);
    else launch_fast_m<F, 8>(a, total_tiles, st);
}

template <int FMT>
void launch_generic(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    switch (mcount) {
#define TQ_G(MM) \
    case MM: hipLaunchKernelGGL((qgemv_generic_kernel<FMT, MM>), dim3(rows), dim3(256), 0, st, a); break;
        TQ_G(1) TQ_G(2) TQ_G(3) TQ_G(4) TQ_G(5) TQ_G(6) TQ_G(7)
        default: hipLaunchKernelGGL((qgemv_generic_kernel<FMT, 8>), dim3(rows), dim3(256), 0, st, a); break;
#undef TQ_G
    }
}

template <int FMT>
void dispatch_fmt(GemvArgs& a, int layout, bool fast, int mcount, int total_tiles, hipStream_t st) {
    if (!fast) {
        launch_generic<FMT>(a, mcount, a.p[0].w.g.rows, st);
    } else if (layout == TITAN_LAYOUT_TILED) {
        launch_fast<typename Pick<FMT, TITAN_LAYOUT_TILED>::type>(a, mcount, total_tiles, st);
    } else {
        if constexpr (FMT != TITAN_Q3_K)
            launch_fast<typename Pick<FMT, TITAN_LAYOUT_REF>::type>(a, mcount, total_tiles, st);
    }
}

}  // namespace tq

// One translation unit per format instantiates the launchers (parallel build).
namespace tq {
void dispatch_gemv_int4(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_int4(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_int2(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_int2(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_fp4(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_fp4(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_nvfp4(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_nvfp4(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_q4k(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_q4k(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_q3k(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_q3k(GemvArgs& a, int mcount, int rows, hipStream_t st);
void dispatch_gemv_fp8(GemvArgs& a, int layout, int mcount, int total_tiles, hipStream_t st);
void dispatch_gemv_generic_fp8(GemvArgs& a, int mcount, int rows, hipStream_t st);
}  // namespace tq
