// gemv.hip -- dequant-GEMV / small-M dequant-GEMM for decode (VALU path).
//
// Replaces the reference's one-block-per-row kernels (dequant.cu:23-172,
// fp4.cu:28-84, fp4.cu:187-238).  Design for gfx950:
//  * A workgroup of 8 waves owns RT tiles of 16 rows and the whole K range.
//    The 8 waves split K (wave w takes 64-byte chunks w, w+8, ...), so at any
//    moment the workgroup streams 512 contiguous code bytes per row.
//  * Lane l = 16*j + r loads row r's 16-byte slot j of a chunk with one
//    128-bit load; in the tiled layout a wave's 64 loads are 1 KiB contiguous.
//  * Activations are staged once per workgroup into LDS as fp32 (phases of
//    at most 64 KiB for long K / many tokens) and read back as 128-bit
//    vectors; each activation segment is reused across the RT row tiles.
//  * Dequantization happens in registers: affine formats fold as
//    scale * sum(q*x) + bias * sum(x); lanes of a row are reduced with two
//    cross-lane shuffles, waves through LDS.
#pragma once
#include "formats.h"

namespace tq {

constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kLdsFloats = 16384;  // 64 KiB of staged activations

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
    int m0;  // first token of this launch (launches cover <= 8 tokens)
};

template <class F, int M, int RT>
__global__ __launch_bounds__(kGemvThreads) void qgemv_kernel(GemvArgs a) {
    __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
    int bid = blockIdx.x, pi = 0;
    for (int i = 1; i < a.n; i++)
        if (bid >= a.p[i].wg_begin) pi = i;
    const GemvProb& P = a.p[pi];
    const WDesc& W = P.w;
    const int rows = W.g.rows, cols = W.g.cols;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, j = lane >> 4;
    const int tile0 = (bid - P.wg_begin) * RT;

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

    // phase width: a multiple of 8 chunks so every wave sees whole chunks
    constexpr int kStep = kGemvWaves * F::CHUNK_COLS;
    constexpr int PC = ((kLdsFloats / M) / kStep) * kStep;
    const float* xg = (const float*)P.x;

    for (int ph0 = 0; ph0 < cols; ph0 += PC) {
        const int pcols = min(PC, cols - ph0);
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; m++) {
            const int64_t xoff = (int64_t)(a.m0 + m) * P.ldx + ph0;
            for (int c = tid; c < pcols; c += kGemvThreads)
                lds[m * PC + c] = load_act(xg, xoff + c, a.xdt);
        }
        __syncthreads();

        const int c_begin = ph0 / F::CHUNK_COLS;
        const int c_end = min(P.nchunks, (ph0 + pcols + F::CHUNK_COLS - 1) / F::CHUNK_COLS);
        for (int c = c_begin + wave; c < c_end; c += kGemvWaves) {
            const int slot_col = c * F::CHUNK_COLS + j * F::SLOT_COLS;
            if (slot_col >= cols) continue;  // ragged REF rows: slot past the end
            typename F::Raw raw[RT];
#pragma unroll
            for (int t = 0; t < RT; t++) F::load(W, rowt[t], c, j, raw[t]);
            const int lbase = c * F::CHUNK_COLS - ph0;
#pragma unroll
            for (int m = 0; m < M; m++) {
#pragma unroll
                for (int s = 0; s < F::SEGS; s++) {
                    float xv[F::SEGW];
                    const float4* xp = (const float4*)&lds[m * PC + lbase + F::seg_col(j, s)];
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
                    for (int t = 0; t < RT; t++) acc[t][m] += F::seg_dot(raw[t], s, xv, sx);
                }
            }
        }
    }

    // reduce: 4 slots of a row inside the wave, then the 8 waves via LDS
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
        if (row < rows) {
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

template <class F, int M>
void launch_fast_m(GemvArgs& a, int total_tiles, hipStream_t st) {
    // Four row tiles per workgroup when that still gives >= 2 workgroups per CU.
    if (total_tiles >= 4 * 512) {
        int wg = 0;
        for (int i = 0; i < a.n; i++) {
            a.p[i].wg_begin = wg;
            wg += (a.p[i].ntiles + 3) / 4;
        }
        hipLaunchKernelGGL((qgemv_kernel<F, M, 4>), dim3(wg), dim3(kGemvThreads), 0, st, a);
    } else {
        int wg = 0;
        for (int i = 0; i < a.n; i++) {
            a.p[i].wg_begin = wg;
            wg += a.p[i].ntiles;
        }
        hipLaunchKernelGGL((qgemv_kernel<F, M, 1>), dim3(wg), dim3(kGemvThreads), 0, st, a);
    }
}

template <class F>
void launch_fast(GemvArgs& a, int mcount, int total_tiles, hipStream_t st) {
    switch (mcount) {
        case 1: launch_fast_m<F, 1>(a, total_tiles, st); break;
        case 2: launch_fast_m<F, 2>(a, total_tiles, st); break;
        case 3: launch_fast_m<F, 3>(a, total_tiles, st); break;
        case 4: launch_fast_m<F, 4>(a, total_tiles, st); break;
        case 5: launch_fast_m<F, 5>(a, total_tiles, st); break;
        case 6: launch_fast_m<F, 6>(a, total_tiles, st); break;
        case 7: launch_fast_m<F, 7>(a, total_tiles, st); break;
        default: launch_fast_m<F, 8>(a, total_tiles, st); break;
    }
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
