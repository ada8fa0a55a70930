// dense.hip -- dense GEMV (fp32 activations and output) for the weights the
// executors keep unquantized: gemv_bf16_to_fp32 (gemv.cu:103-159, BF16 lm_head
// / MLA projections), gemv_fp32 and gemv_fp32_batched (gemv.cu:33-88, cuBLAS
// sgemv in the reference), and the format-exact matvec_dispatch that the
// reference's dense.cpp:13-32 approximates (it sends Q4_K to the INT4 kernel).
//
// Kernel: a workgroup of 4 waves owns 16 rows, each wave 4 of them.  The
// activations are staged once per workgroup in LDS as fp32 (phases of at most
// 8192 columns); lanes stream 16-byte words of their rows (8 bf16 or 4 fp32
// weights) with the next step's words in flight while the current step is
// folded, fp32 FMAs, one wave reduction per row.  HBM-bound: 2 (bf16) or 4
// (fp32) bytes per weight.
#include "common.h"

namespace tq {
namespace {

constexpr int kDenseRowsPerWave = 4;
constexpr int kDenseRowsPerWg = 4 * kDenseRowsPerWave;
constexpr int kDensePhase = 8192;  // staged columns per phase (32 KiB of fp32)

template <bool BF16>
struct DenseW {
    static constexpr int PER = BF16 ? 8 : 4;  // weights per 16-byte word
    TQ_DEV static void fold(const uint4& q, const float* xs, float& acc) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        if constexpr (BF16) {
            const float4 a = *(const float4*)xs, b = *(const float4*)(xs + 4);
            const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                acc = __builtin_fmaf(__builtin_bit_cast(float, w[k] << 16), xv[2 * k], acc);
                acc = __builtin_fmaf(__builtin_bit_cast(float, w[k] & 0xFFFF0000u), xv[2 * k + 1], acc);
            }
        } else {
            const float4 a = *(const float4*)xs;
            acc = __builtin_fmaf(__builtin_bit_cast(float, w[0]), a.x, acc);
            acc = __builtin_fmaf(__builtin_bit_cast(float, w[1]), a.y, acc);
            acc = __builtin_fmaf(__builtin_bit_cast(float, w[2]), a.z, acc);
            acc = __builtin_fmaf(__builtin_bit_cast(float, w[3]), a.w, acc);
        }
    }
};

// cols % PER == 0 and 16-byte aligned rows (checked on the host).
template <bool BF16>
__global__ __launch_bounds__(256) void dense_gemv_kernel(const uint8_t* __restrict__ A,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int rows, int cols) {
    using D = DenseW<BF16>;
    constexpr int R = kDenseRowsPerWave;
    __shared__ __attribute__((aligned(16))) float xs[kDensePhase];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = blockIdx.x * kDenseRowsPerWg + wave * R;
    const size_t row_bytes = (size_t)cols * (BF16 ? 2 : 4);
    const uint8_t* rp[R];
#pragma unroll
    for (int q = 0; q < R; q++) rp[q] = A + (size_t)min(row0 + q, rows - 1) * row_bytes;  // clamped: not stored
    float acc[R];
#pragma unroll
    for (int q = 0; q < R; q++) acc[q] = 0.0f;

    for (int c0 = 0; c0 < cols; c0 += kDensePhase) {
        const int n = min(kDensePhase, cols - c0);
        __syncthreads();
        for (int i = threadIdx.x * 4; i < n; i += 256 * 4) {
            if (i + 4 <= n && ((c0 + i) & 3) == 0 && ((uintptr_t)x & 15) == 0) {
                *(float4*)(xs + i) = *(const float4*)(x + c0 + i);
            } else {
                for (int k = 0; k < 4 && i + k < n; k++) xs[i + k] = x[c0 + i + k];
            }
        }
        __syncthreads();
        // lane word e covers columns [c0 + PER e, +PER); two steps of 64 words in flight
        const int words = n / D::PER;
        uint4 va[R], vb[R];
        auto load = [&](int e, uint4* v) {
            const int ee = e < words ? e : 0;  // past the end: a cached word, not folded
#pragma unroll
            for (int q = 0; q < R; q++)
                v[q] = ld_stream_u128(rp[q] + (size_t)(c0 + ee * D::PER) * (BF16 ? 2 : 4));
        };
        auto fold = [&](int e, const uint4* v) {  // branch-free: words past the end count zero
            const bool live = e < words;
            const int ee = live ? e : 0;
#pragma unroll
            for (int q = 0; q < R; q++)
                D::fold(live ? v[q] : make_uint4(0, 0, 0, 0), xs + ee * D::PER, acc[q]);
        };
        load(lane, va);
        for (int base = 0; base < words; base += 128) {
            const int e = base + lane;
            load(e + 64, vb);
            fold(e, va);
            load(e + 128, va);
            fold(e + 64, vb);
        }
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
        const float s = wave_sum(acc[q]);
        if (lane == 0 && row0 + q < rows) y[row0 + q] = s;
    }
}

// Any shape / alignment: one wave per row, scalar loads.
template <bool BF16>
__global__ __launch_bounds__(256) void dense_gemv_scalar_kernel(const uint8_t* __restrict__ A,
                                                                const float* __restrict__ x,
                                                                float* __restrict__ y, int rows,
                                                                int cols) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    float acc = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        float w;
        if constexpr (BF16) w = __builtin_bit_cast(float, (uint32_t)((const uint16_t*)A)[(size_t)row * cols + c] << 16);
        else w = ((const float*)A)[(size_t)row * cols + c];
        acc = __builtin_fmaf(w, x[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

template <bool BF16>
int run_dense(const void* A, const float* x, float* y, int rows, int cols, hipStream_t st) {
    if (!A || !x || !y || rows <= 0 || cols <= 0) return TITAN_ERR_INVALID_ARG;
    constexpr int PER = DenseW<BF16>::PER;
    const size_t row_bytes = (size_t)cols * (BF16 ? 2 : 4);
    if (cols % PER == 0 && (row_bytes & 15) == 0 && ((uintptr_t)A & 15) == 0)
        hipLaunchKernelGGL(dense_gemv_kernel<BF16>, dim3((rows + kDenseRowsPerWg - 1) / kDenseRowsPerWg),
                           dim3(256), 0, st, (const uint8_t*)A, x, y, rows, cols);
    else
        hipLaunchKernelGGL(dense_gemv_scalar_kernel<BF16>, dim3((rows + 3) / 4), dim3(256), 0, st,
                           (const uint8_t*)A, x, y, rows, cols);
    return tqh::launch_status();
}

}  // namespace
}  // namespace tq

// gemv.cu:103-159 -- BF16 A [rows][cols] x fp32 x -> fp32 y.
extern "C" int titan_gemv_bf16_to_fp32(const void* A, const float* x, float* y, int rows, int cols,
                                       hipStream_t stream) {
    return tq::run_dense<true>(A, x, y, rows, cols, stream);
}

// gemv.cu:33-52 -- fp32 A [rows][cols] x fp32 x -> fp32 y (cuBLAS sgemv there).
extern "C" int titan_gemv_fp32(const float* A, const float* x, float* y, int rows, int cols,
                               hipStream_t stream) {
    return tq::run_dense<false>(A, x, y, rows, cols, stream);
}

// gemv.cu:54-72 -- the reference's batched call is one sgemv over rows * batch
// rows of A against the same x; kept as it is.
extern "C" int titan_gemv_fp32_batched(const float* A, const float* x, float* y, int rows, int cols,
                                       int batch, hipStream_t stream) {
    if (batch <= 0 || (long long)rows * batch > INT32_MAX) return TITAN_ERR_INVALID_ARG;
    return tq::run_dense<false>(A, x, y, rows * batch, cols, stream);
}

// dense.cpp:13-32 matvec_dispatch, format-exact: every quantized format goes to
// its own decoder (Q4_K is not INT4), dense fp32 / bf16 weights to the dense
// GEMV.  fp32 input and output, one token.
extern "C" int titan_matvec_dispatch(const titan_qweight* w, const float* input, float* output,
                                     hipStream_t stream) {
    if (!w || !input || !output) return TITAN_ERR_INVALID_ARG;
    if (w->format == TITAN_FP32) return titan_gemv_fp32((const float*)w->codes, input, output, w->rows, w->cols, stream);
    if (w->format == TITAN_BF16) return titan_gemv_bf16_to_fp32(w->codes, input, output, w->rows, w->cols, stream);
    return titan_qgemm(w, input, TITAN_FP32, w->cols, output, TITAN_FP32, w->rows, 1, stream);
}
