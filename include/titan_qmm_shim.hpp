// titan_qmm_shim.hpp -- header-only C++ names for drop-in callers.
//
// Restores the free functions of the reference's `namespace titan::cuda`
// (src/compute/dispatch.h:30-130) on top of the C ABI in titan_qmm.h, with
// the reference's argument order and meaning; the stream type is
// hipStream_t.  Like the reference they return void; the status of the
// underlying call is available from titan::cuda::last_status() (thread
// local), and titan::cuda::set_status_handler installs a callback that sees
// every non-zero status (the reference prints launch errors in debug builds
// only, src/compute/cuda/cuda_check.h:6-18).
#ifndef TITAN_QMM_SHIM_HPP
#define TITAN_QMM_SHIM_HPP

#include "titan_qmm.h"

namespace titan {
namespace cuda {

using status_handler = void (*)(int status, const char* what);

namespace detail {
inline int& last() {
    static thread_local int s = TITAN_OK;
    return s;
}
inline status_handler& handler() {
    static status_handler h = nullptr;
    return h;
}
inline void note(int st, const char* what) {
    last() = st;
    if (st != TITAN_OK && handler()) handler()(st, what);
}
}  // namespace detail

inline int last_status() { return detail::last(); }
inline void set_status_handler(status_handler h) { detail::handler() = h; }

// dispatch.h:32-37 (dequant.cu)
inline void dequant_matvec_int4(const void* weights, const void* scales, const void* biases,
                                const float* input, float* output, int rows, int cols,
                                int group_size, hipStream_t stream) {
    detail::note(titan_dequant_matvec_int4(weights, scales, biases, input, output, rows, cols,
                                           group_size, stream),
                 "dequant_matvec_int4");
}
inline void dequant_matvec_int2(const void* weights, const void* scales, const void* biases,
                                const float* input, float* output, int rows, int cols,
                                int group_size, hipStream_t stream) {
    detail::note(titan_dequant_matvec_int2(weights, scales, biases, input, output, rows, cols,
                                           group_size, stream),
                 "dequant_matvec_int2");
}

// dispatch.h:47-48, 61-65 (activation.cu)
inline void swiglu(float* output, const float* gate, const float* up, int dim, hipStream_t stream) {
    detail::note(titan_swiglu(output, gate, up, dim, stream), "swiglu");
}
inline void fused_moe_combine_norm(float* output, float* residual, const float* expert_outputs,
                                   const float* routing_weights, const float* shared_expert,
                                   float shared_weight, const float* norm_weight, int dim,
                                   int num_active, float eps, hipStream_t stream) {
    detail::note(titan_fused_moe_combine_norm(output, residual, expert_outputs, routing_weights,
                                              shared_expert, shared_weight, norm_weight, dim,
                                              num_active, eps, stream),
                 "fused_moe_combine_norm");
}

// dispatch.h:82-86 (moe.cu)
inline void moe_gate(const float* hidden, const float* gate_weight, float* logits, int hidden_dim,
                     int num_experts, hipStream_t stream) {
    detail::note(titan_moe_gate(hidden, gate_weight, logits, hidden_dim, num_experts, stream), "moe_gate");
}
inline void moe_topk(const float* logits, float* weights, int* indices, int num_experts, int k,
                     hipStream_t stream) {
    detail::note(titan_moe_topk(logits, weights, indices, num_experts, k, stream), "moe_topk");
}

// dispatch.h:93-100 (gemv.cu): the dense GEMV keeps no library handle
inline void init_cublas() {}
inline void destroy_cublas() {}
inline void gemv_fp32(const float* A, const float* x, float* y, int rows, int cols, hipStream_t stream) {
    detail::note(titan_gemv_fp32(A, x, y, rows, cols, stream), "gemv_fp32");
}
inline void gemv_fp32_batched(const float* A, const float* x, float* y, int rows, int cols, int batch,
                              hipStream_t stream) {
    detail::note(titan_gemv_fp32_batched(A, x, y, rows, cols, batch, stream), "gemv_fp32_batched");
}
inline void gemv_bf16_to_fp32(const void* A, const float* x, float* y, int rows, int cols,
                              hipStream_t stream) {
    detail::note(titan_gemv_bf16_to_fp32(A, x, y, rows, cols, stream), "gemv_bf16_to_fp32");
}

// dispatch.h:107-115 (fp4.cu)
inline void dequant_matvec_fp4(const void* weights, const void* scales, const float* input,
                               float* output, int rows, int cols, int group_size, hipStream_t stream) {
    detail::note(titan_dequant_matvec_fp4(weights, scales, input, output, rows, cols, group_size, stream),
                 "dequant_matvec_fp4");
}
inline void dequant_matvec_nvfp4(const void* weights, const void* scales, float global_scale,
                                 const float* input, float* output, int rows, int cols,
                                 hipStream_t stream) {
    detail::note(titan_dequant_matvec_nvfp4(weights, scales, global_scale, input, output, rows, cols, stream),
                 "dequant_matvec_nvfp4");
}
inline void quantize_fp4(const float* input, void* output, void* scales, int numel, int group_size,
                         hipStream_t stream) {
    detail::note(titan_quantize_fp4(input, output, scales, numel, group_size, stream), "quantize_fp4");
}

// dispatch.h:127-130 (sparse.cu)
inline void sparse_dequant_matvec_int4(const void* weights, const void* scales, const void* biases,
                                       const float* input, float* output, const int* active_indices,
                                       int num_active, int cols, int group_size, hipStream_t stream) {
    detail::note(titan_sparse_dequant_matvec_int4(weights, scales, biases, input, output, active_indices,
                                                  num_active, cols, group_size, stream),
                 "sparse_dequant_matvec_int4");
}

}  // namespace cuda
}  // namespace titan

#endif  // TITAN_QMM_SHIM_HPP
