// sparse.hip -- activation-sparse INT4 GEMV: only the rows listed in
// active_indices are computed (sparse.cu:142-205 sparse_dequant_matvec_int4,
// declared in dispatch.h:127-130).  output[active_indices[i]] = dot(W[row], x)
// with W dequantized as q * s + b (fp16 scale / bias per group); every other
// output element is left untouched, as in the reference.
//
// One wave per active row: lanes stream the row's words with 16-byte loads
// (4 words = 32 columns per lane step), fp32 activations from L1/L2, fp32
// accumulation, a wave reduction at the end.
#include "common.h"

namespace tq {

__global__ __launch_bounds__(256) void sparse_int4_kernel(const uint32_t* __restrict__ w,
                                                          const uint16_t* __restrict__ s,
                                                          const uint16_t* __restrict__ b,
                                                          const float* __restrict__ x,
                                                          float* __restrict__ y,
                                                          const int* __restrict__ idx, int nact,
                                                          int cols, int gs) {
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (i >= nact) return;
    const int row = idx[i];
    if (row < 0) return;  // negative indices compute nothing
    const int wpr = cols / 8, gpr = cols / gs;
    const uint32_t* rw = w + (size_t)row * wpr;
    const uint16_t* rs = s + (size_t)row * gpr;
    const uint16_t* rb = b + (size_t)row * gpr;
    float acc = 0.0f;
    if ((wpr & 3) == 0 && ((uintptr_t)rw & 15) == 0 && ((uintptr_t)x & 15) == 0) {
        for (int p = lane * 4; p < wpr; p += 256) {
            const uint4 q = *(const uint4*)(rw + p);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int c0 = (p + k) * 8, g = c0 / gs;
                const float sc = f16_to_f32(rs[g]), bi = f16_to_f32(rb[g]);
                const float4 xa = *(const float4*)(x + c0), xb = *(const float4*)(x + c0 + 4);
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                float t = 0.0f, sx = 0.0f;
#pragma unroll
                for (int n = 0; n < 8; n++) {
                    t = __builtin_fmaf((float)((qw[k] >> (4 * n)) & 0xF), xv[n], t);
                    sx += xv[n];
                }
                acc = __builtin_fmaf(sc, t, __builtin_fmaf(bi, sx, acc));
            }
        }
    } else {
        for (int p = lane; p < wpr; p += 64) {
            const uint32_t q = rw[p];
            const int c0 = p * 8, g = c0 / gs;
            const float sc = f16_to_f32(rs[g]), bi = f16_to_f32(rb[g]);
            float t = 0.0f, sx = 0.0f;
#pragma unroll
            for (int n = 0; n < 8; n++) {
                const float xv = x[c0 + n];
                t = __builtin_fmaf((float)((q >> (4 * n)) & 0xF), xv, t);
                sx += xv;
            }
            acc = __builtin_fmaf(sc, t, __builtin_fmaf(bi, sx, acc));
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

}  // namespace tq

// dispatch.h:127-130 (titan::cuda::sparse_dequant_matvec_int4).  As in the
// reference call there is no row count: indices must be valid rows of the
// weight buffer (negative ones are skipped).
extern "C" int titan_sparse_dequant_matvec_int4(const void* weights, const void* scales,
                                                const void* biases, const float* input,
                                                float* output, const int* active_indices,
                                                int num_active, int cols, int group_size,
                                                hipStream_t stream) {
    if (!weights || !scales || !biases || !input || !output || (!active_indices && num_active))
        return TITAN_ERR_INVALID_ARG;
    if (num_active < 0 || cols <= 0 || group_size <= 0 || cols % 8) return TITAN_ERR_INVALID_ARG;
    if (num_active == 0) return TITAN_OK;
    hipLaunchKernelGGL(tq::sparse_int4_kernel, dim3((num_active + 3) / 4), dim3(256), 0, stream,
                       (const uint32_t*)weights, (const uint16_t*)scales, (const uint16_t*)biases,
                       input, output, active_indices, num_active, cols, group_size);
    return tqh::launch_status();
}
