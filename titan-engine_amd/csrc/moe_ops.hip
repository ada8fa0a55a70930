// moe_ops.hip -- routing, activation, combine and producer kernels with the
// reference's fp32 semantics (moe.cu:16-115, activation.cu:17-32 / 111-139,
// fp4.cu:90-141), plus the per-token FP8 activation quantizer.
#include "common.h"

namespace tq {

// moe.cu:16-54: logits[e] = dot(G[e], h).  One wave per expert, 128-bit loads.
__global__ __launch_bounds__(256) void moe_gate_kernel(const float* __restrict__ h,
                                                       const float* __restrict__ G,
                                                       float* __restrict__ logits, int hd, int E) {
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (e >= E) return;
    const float* g = G + (size_t)e * hd;
    float acc = 0.0f;
    if ((hd & 3) == 0 && ((uintptr_t)g & 15) == 0 && ((uintptr_t)h & 15) == 0) {
        for (int i = lane * 4; i < hd; i += 256) {
            float4 a = *(const float4*)(g + i), b = *(const float4*)(h + i);
            acc += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
        }
    } else {
        for (int i = lane; i < hd; i += 64) acc += g[i] * h[i];
    }
    acc = wave_sum(acc);
    if (lane == 0) logits[e] = acc;
}

// moe.cu:58-115: softmax over all E (max-subtracted, 1/(sum + 1e-8)), top-k
// by repeated argmax where the lowest index wins ties, then w/(sum w + 1e-8).
// One workgroup of 256 threads; E up to 4096.
__global__ __launch_bounds__(256) void moe_topk_kernel(const float* __restrict__ logits,
                                                       float* __restrict__ weights,
                                                       int* __restrict__ indices, int E, int k,
                                                       int64_t ld_logits, int ld_out) {
    __shared__ float p[4096];
    __shared__ float rv[4];
    __shared__ int ri[4];
    const int tok = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float* lg = logits + (int64_t)tok * ld_logits;
    float mx = -3.402823466e+38f;
    for (int i = tid; i < E; i += 256) {
        p[i] = lg[i];
        mx = fmaxf(mx, p[i]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) rv[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(rv[0], rv[1]), fmaxf(rv[2], rv[3]));
    float s = 0.0f;
    for (int i = tid; i < E; i += 256) {
        p[i] = expf(p[i] - mx);
        s += p[i];
    }
    s = wave_sum(s);
    __syncthreads();
    if (lane == 0) rv[wave] = s;
    __syncthreads();
    const float inv = 1.0f / ((rv[0] + rv[1] + rv[2] + rv[3]) + 1e-8f);
    for (int i = tid; i < E; i += 256) p[i] *= inv;
    __syncthreads();
    float wsum = 0.0f, wsel = 0.0f;
    for (int j = 0; j < k; j++) {
        float bv = -1.0f;
        int bi = 0x7FFFFFFF;
        for (int i = tid; i < E; i += 256)
            if (p[i] > bv) { bv = p[i]; bi = i; }  // ascending i: first max kept
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            float ov = __shfl_xor(bv, o, 64);
            int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { rv[wave] = bv; ri[wave] = bi; }
        __syncthreads();
        bv = rv[0];
        bi = ri[0];
        for (int w = 1; w < 4; w++)
            if (rv[w] > bv || (rv[w] == bv && ri[w] < bi)) { bv = rv[w]; bi = ri[w]; }
        __syncthreads();
        if (tid == 0) {
            p[bi] = -2.0f;
            indices[(int64_t)tok * ld_out + j] = bi;
        }
        if (j == 0) wsum = 0.0f;
        wsum += bv;  // sequential order j = 0..k-1, as the reference
        if (tid == j) wsel = bv;
        __syncthreads();
    }
    const float invs = 1.0f / (wsum + 1e-8f);
    if (tid < k) weights[(int64_t)tok * ld_out + tid] = wsel * invs;
}

// activation.cu:17-32
__global__ void swiglu_kernel(float* __restrict__ out, const float* __restrict__ g,
                              const float* __restrict__ u, int n) {
    int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float gv = g[i];
    float sg = 1.0f / (1.0f + expf(-gv));
    out[i] = (gv * sg) * u[i];
}

// activation.cu:111-139: res += sum_e w_e*y_e + w_s*shared; out = res.  The
// products accumulate with fused multiply-adds, as nvcc compiles the
// reference's `combined += a * b` (default --fmad=true).
__global__ void combine_kernel(float* __restrict__ out, float* __restrict__ res,
                               const float* __restrict__ eo, const float* __restrict__ w,
                               const float* __restrict__ shared, float sw, int dim, int na) {
    int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    float c = 0.0f;
    for (int e = 0; e < na; e++) c = __builtin_fmaf(eo[(size_t)e * dim + i], w[e], c);
    if (shared) c = __builtin_fmaf(shared[i], sw, c);
    float v = res[i] + c;
    res[i] = v;
    out[i] = v;
}

// fp4.cu:90-141 (one thread per group).
__global__ void quantize_fp4_kernel(const float* __restrict__ in, uint32_t* __restrict__ out,
                                    uint16_t* __restrict__ scales, int numel, int gs) {
    int g = blockIdx.x * 256 + threadIdx.x;
    int ng = numel / gs;
    if (g >= ng) return;
    const float* v = in + (size_t)g * gs;
    float amax = 0.0f;
    for (int i = 0; i < gs; i++) amax = fmaxf(amax, fabsf(v[i]));
    float sc = amax / 6.0f;
    if (sc < 1e-10f) sc = 1e-10f;
    float inv = 1.0f / sc;
    scales[g] = f32_to_f16_rne(sc);
    for (int i = 0; i < gs; i += 8) {
        uint32_t packed = 0;
        for (int n = 0; n < 8 && i + n < gs; n++) {
            float val = __fmul_rn(v[i + n], inv);
            float a = fabsf(val);
            uint32_t nib = a < 0.25f ? 0 : a < 0.75f ? 1 : a < 1.25f ? 2 : a < 1.75f ? 3
                         : a < 2.5f ? 4 : a < 3.5f ? 5 : a < 5.0f ? 6 : 7;
            if (val < 0) nib |= 8;
            packed |= nib << (4 * n);
        }
        out[((size_t)g * gs + i) / 8] = packed;
    }
}

// Per-token e4m3 quantization: scale = amax/448 (1 if amax == 0).
__global__ __launch_bounds__(256) void fp8_quant_rows_kernel(const void* __restrict__ x, int xdt,
                                                             int K, uint8_t* __restrict__ xq,
                                                             float* __restrict__ xs) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int64_t base = (int64_t)m * K;
    float amax = 0.0f;
    for (int k = tid; k < K; k += 256) amax = fmaxf(amax, fabsf(load_act(x, base + k, xdt)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (tid == 0) xs[m] = sc;
    for (int k = tid; k < K; k += 256)
        xq[base + k] = (uint8_t)f32_to_e4m3_rne_sat(load_act(x, base + k, xdt) / sc);
}

// Same result, 8 elements per thread step with 16-byte loads (rows of K % 8 ==
// 0 elements, 16-byte aligned); the second pass re-reads the row from cache.
template <int XDT>
__global__ __launch_bounds__(256) void fp8_quant_rows_vec_kernel(const void* __restrict__ x, int K,
                                                                 uint8_t* __restrict__ xq,
                                                                 float* __restrict__ xs) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const int64_t base = (int64_t)m * K;
    auto load8 = [&](int k, float* v) {
        if constexpr (XDT == TITAN_FP32) {
            const float4 a = *(const float4*)((const float*)x + base + k);
            const float4 b = *(const float4*)((const float*)x + base + k + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 a = *(const uint4*)((const uint16_t*)x + base + k);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[2 * i] = XDT == TITAN_FP16 ? f16_to_f32(w[i] & 0xFFFFu) : bf16_to_f32(w[i] & 0xFFFFu);
                v[2 * i + 1] = XDT == TITAN_FP16 ? f16_to_f32(w[i] >> 16) : bf16_to_f32(w[i] >> 16);
            }
        }
    };
    // rows of up to 16384 elements stay in registers: every load of the row
    // is in flight at once and the row is read from memory once
    constexpr int NR = 8;
    float keep[NR][8];
    const bool held = K <= NR * 256 * 8;
    float amax = 0.0f;
    if (held) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int k = (r * 256 + tid) * 8;
            if (k < K) load8(k, keep[r]);
            else {
#pragma unroll
                for (int i = 0; i < 8; i++) keep[r][i] = 0.0f;
            }
        }
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(keep[r][i]));
    } else {
        for (int k = tid * 8; k < K; k += 256 * 8) {
            float v[8];
            load8(k, v);
#pragma unroll
            for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (tid == 0) xs[m] = sc;
    auto put8 = [&](int k, const float* v) {
#ifndef TQ_FP8_SOFT_CVT
        // hardware RNE conversion (v_cvt_pk_fp8_f32, OCP e4m3): |v / sc| <=
        // 448 (1 + 2^-23) here, which rounds to at most 448, so no input
        // reaches the saturating range.  The hardware writes NaN as 0xFF (no
        // finite code); those bytes become 0x7F, the software conversion's NaN.
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = v[i] / sc;
        uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
        lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], (int)lo, true);
        uint32_t hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], 0, false);
        hi = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], (int)hi, true);
        auto nan_fix = [](uint32_t w) {  // bit 7 of every 0xFF byte cleared (no carries: bytes <= 0x80)
            return w ^ (((w & 0x7F7F7F7Fu) + 0x01010101u) & w & 0x80808080u);
        };
        *(uint2*)(xq + base + k) = make_uint2(nan_fix(lo), nan_fix(hi));
#else
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = f32_to_e4m3_rne_sat(v[i] / sc);
        *(uint2*)(xq + base + k) = make_uint2(q[0] | q[1] << 8 | q[2] << 16 | q[3] << 24,
                                              q[4] | q[5] << 8 | q[6] << 16 | q[7] << 24);
#endif
    };
    if (held) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int k = (r * 256 + tid) * 8;
            if (k < K) put8(k, keep[r]);
        }
    } else {
        for (int k = tid * 8; k < K; k += 256 * 8) {
            float v[8];
            load8(k, v);
            put8(k, v);
        }
    }
}

}  // namespace tq

using namespace tq;

extern "C" int titan_moe_gate(const float* hidden, const float* gate_weight, float* logits,
                              int hidden_dim, int num_experts, hipStream_t stream) {
    if (!hidden || !gate_weight || !logits || hidden_dim <= 0 || num_experts <= 0)
        return TITAN_ERR_INVALID_ARG;
    hipLaunchKernelGGL(moe_gate_kernel, dim3((num_experts + 3) / 4), dim3(256), 0, stream,
                       hidden, gate_weight, logits, hidden_dim, num_experts);
    return tqh::launch_status();
}

extern "C" int titan_moe_topk(const float* logits, float* weights, int* indices,
                              int num_experts, int k, hipStream_t stream) {
    if (!logits || !weights || !indices || num_experts <= 0 || k <= 0 || k > num_experts ||
        num_experts > 4096 || k > 256)
        return TITAN_ERR_INVALID_ARG;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(256), 0, stream, logits, weights, indices,
                       num_experts, k, (int64_t)num_experts, k);
    return tqh::launch_status();
}

// Batched routing: one top-k per token row of logits [T][E].
extern "C" int titan_moe_topk_batched(const float* logits, float* weights, int* indices,
                                      int tokens, int num_experts, int k, hipStream_t stream) {
    if (!logits || !weights || !indices || tokens <= 0 || num_experts <= 0 || k <= 0 ||
        k > num_experts || num_experts > 4096 || k > 256)
        return TITAN_ERR_INVALID_ARG;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(tokens), dim3(256), 0, stream, logits, weights,
                       indices, num_experts, k, (int64_t)num_experts, k);
    return tqh::launch_status();
}

extern "C" int titan_swiglu(float* output, const float* gate, const float* up, int dim,
                            hipStream_t stream) {
    if (!output || !gate || !up || dim <= 0) return TITAN_ERR_INVALID_ARG;
    hipLaunchKernelGGL(swiglu_kernel, dim3((dim + 255) / 256), dim3(256), 0, stream, output, gate,
                       up, dim);
    return tqh::launch_status();
}

extern "C" int titan_fused_moe_combine_norm(float* output, float* residual,
                                            const float* expert_outputs,
                                            const float* routing_weights,
                                            const float* shared_expert, float shared_weight,
                                            const float* norm_weight, int dim, int num_active,
                                            float eps, hipStream_t stream) {
    (void)norm_weight;  // unused by the reference too (activation.cu:118-123)
    (void)eps;
    if (!output || !residual || dim <= 0 || num_active < 0 ||
        (num_active > 0 && (!expert_outputs || !routing_weights)))
        return TITAN_ERR_INVALID_ARG;
    hipLaunchKernelGGL(combine_kernel, dim3((dim + 255) / 256), dim3(256), 0, stream, output,
                       residual, expert_outputs, routing_weights, shared_expert, shared_weight,
                       dim, num_active);
    return tqh::launch_status();
}

extern "C" int titan_quantize_fp4(const float* input, void* output, void* scales, int numel,
                                  int group_size, hipStream_t stream) {
    if (!input || !output || !scales || numel <= 0 || group_size <= 0 || group_size % 8 ||
        numel % group_size)
        return TITAN_ERR_INVALID_ARG;
    int ng = numel / group_size;
    hipLaunchKernelGGL(quantize_fp4_kernel, dim3((ng + 255) / 256), dim3(256), 0, stream, input,
                       (uint32_t*)output, (uint16_t*)scales, numel, group_size);
    return tqh::launch_status();
}

extern "C" int titan_fp8_quantize_rows(const void* x, int x_dtype, int M, int K, uint8_t* xq,
                                       float* x_scale, hipStream_t stream) {
    if (!x || !xq || !x_scale || M <= 0 || K <= 0 || !tqh::act_dtype_ok(x_dtype))
        return TITAN_ERR_INVALID_ARG;
    const int esz = x_dtype == TITAN_FP32 ? 4 : 2;
    if (K % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)xq & 7) == 0 && (K * esz) % 16 == 0) {
        switch (x_dtype) {
            case TITAN_FP32:
                hipLaunchKernelGGL(fp8_quant_rows_vec_kernel<TITAN_FP32>, dim3(M), dim3(256), 0, stream, x, K, xq, x_scale);
                break;
            case TITAN_FP16:
                hipLaunchKernelGGL(fp8_quant_rows_vec_kernel<TITAN_FP16>, dim3(M), dim3(256), 0, stream, x, K, xq, x_scale);
                break;
            default:
                hipLaunchKernelGGL(fp8_quant_rows_vec_kernel<TITAN_BF16>, dim3(M), dim3(256), 0, stream, x, K, xq, x_scale);
                break;
        }
    } else {
        hipLaunchKernelGGL(fp8_quant_rows_kernel, dim3(M), dim3(256), 0, stream, x, x_dtype, K, xq,
                           x_scale);
    }
    return tqh::launch_status();
}

extern "C" const char* titan_version(void) { return "titan-qmm-gfx950 0.1"; }

extern "C" const char* titan_status_string(int s) {
    switch (s) {
        case TITAN_OK: return "ok";
        case TITAN_ERR_INVALID_ARG: return "invalid argument";
        case TITAN_ERR_UNSUPPORTED: return "unsupported shape/format/layout";
        case TITAN_ERR_LAUNCH: return "kernel launch failed";
        case TITAN_ERR_WORKSPACE: return "workspace missing or too small";
        case TITAN_ERR_IO: return "checkpoint file missing, unreadable or malformed";
        case TITAN_ERR_NOT_FOUND: return "tensor not found";
        case TITAN_ERR_SCRATCH_LIMIT: return "problem needs more than the static scratch (TITAN_NOALLOC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}
