// fp8_gemm.hip -- FP8 (OCP E4M3) prefill GEMM on gfx950 MFMA.
//
// out[m][n] = (sum_k A[m][k] * W[n][k]) * sa[m] * sw[n]
//   A  : e4m3 activations [M][K] with fp32 per-token scale sa (from
//        titan_fp8_quantize_rows)
//   W  : e4m3 weights [N][K] with fp32 per-output-channel scale sw
// The reference has only an unscaled, unlaunched FP8 matvec
// (dequant.cu:179-221); this GEMM is the north-star prefill path.
//
// Tiling: 256 threads (4 waves) per 128x128 output tile, K step 128, A and B
// tiles double-buffered in LDS (rows padded to 144 B: conflict-free 128-bit
// fragment reads).  Each wave owns a 64x64 quadrant = 4x4 MFMA tiles of
// v_mfma_scale_f32_16x16x128_f8f6f4 (unit E8M0 scales), fp32 accumulators.
#include "common.h"

namespace tq {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kFBM = 128, kFBN = 128, kFBK = 128;
constexpr int kFRow = 144;  // padded LDS row bytes
constexpr int kFTile = 128 * kFRow;

TQ_DEV v4f mfma_fp8(const v8i& a, const v8i& b, v4f c) {
    // cbsz = blgp = 0: both operands FP8 E4M3; scale 127 = 2^0 (E8M0)
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__global__ __launch_bounds__(256) void fp8_gemm_kernel(const uint8_t* __restrict__ A,
                                                       const float* __restrict__ sa,
                                                       const uint8_t* __restrict__ W,
                                                       const float* __restrict__ sw,
                                                       void* __restrict__ out, int odt, int M,
                                                       int N, int K) {
    __shared__ __attribute__((aligned(16))) uint8_t sm[2][2][kFTile];  // [buf][A/B]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n0 = blockIdx.x * kFBN, m0 = blockIdx.y * kFBM;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // global -> LDS copy assignment: 8 threads per 128-byte row, 32 rows/pass
    const int crow = tid >> 3, ccol = (tid & 7) * 16;
    const uint8_t* ga = A + (size_t)(m0 + crow) * K + ccol;
    const uint8_t* gb = W + (size_t)(n0 + crow) * K + ccol;

    uint4 ra[4], rb[4];
    auto gload = [&](int k0) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            ra[p] = *(const uint4*)(ga + (size_t)(32 * p) * K + k0);
            rb[p] = *(const uint4*)(gb + (size_t)(32 * p) * K + k0);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < 4; p++) {
            *(uint4*)&sm[buf][0][(crow + 32 * p) * kFRow + ccol] = ra[p];
            *(uint4*)&sm[buf][1][(crow + 32 * p) * kFRow + ccol] = rb[p];
        }
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jn = 0; jn < 4; jn++) acc[i][jn] = (v4f){0.f, 0.f, 0.f, 0.f};

    const int fr = lane & 15, fk = (lane >> 4) * 32;  // fragment row / k offset
    const int nk = K / kFBK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kFBK);
        v8i fa[4], fb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint8_t* pa = &sm[buf][0][(wm + 16 * i + fr) * kFRow + fk];
            const uint8_t* pb = &sm[buf][1][(wn + 16 * i + fr) * kFRow + fk];
            uint4 a0 = *(const uint4*)pa, a1 = *(const uint4*)(pa + 16);
            uint4 b0 = *(const uint4*)pb, b1 = *(const uint4*)(pb + 16);
            fa[i] = (v8i){(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w,
                          (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            fb[i] = (v8i){(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                          (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jn = 0; jn < 4; jn++) acc[i][jn] = mfma_fp8(fa[i], fb[jn], acc[i][jn]);
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // C fragment of a 16x16 tile: lane holds column (lane & 15) of rows
    // 4*(lane >> 4) + 0..3.  A fragment rows are M, B fragment rows are N.
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jn = 0; jn < 4; jn++) {
            const int n = n0 + wn + 16 * jn + (lane & 15);
            const float sn = sw[n];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm + 16 * i + 4 * (lane >> 4) + v;
                store_out(out, (int64_t)m * N + n, odt, acc[i][jn][v] * sa[m] * sn);
            }
        }
}

}  // namespace tq

extern "C" int titan_fp8_gemm(const uint8_t* A, const float* sa, const uint8_t* W, const float* sw,
                              void* out, int out_dtype, int M, int N, int K, hipStream_t stream) {
    if (!A || !sa || !W || !sw || !out || M <= 0 || N <= 0 || K <= 0 ||
        !tqh::act_dtype_ok(out_dtype))
        return TITAN_ERR_INVALID_ARG;
    if (M % tq::kFBM || N % tq::kFBN || K % tq::kFBK || ((uintptr_t)A & 15) || ((uintptr_t)W & 15))
        return TITAN_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(tq::fp8_gemm_kernel, dim3(N / tq::kFBN, M / tq::kFBM), dim3(256), 0, stream,
                       A, sa, W, sw, out, out_dtype, M, N, K);
    return tqh::launch_status();
}
