// ref_shim.cpp -- C entry points over the reference's own CPU expert path.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's
// src/compute/cpu/matmul_avx.cpp and src/compute/cpu/expert_cpu.cpp (read in
// place from the reference tree, never copied) into oracle/_ref/.  The
// reference exports C++-linkage functions in namespace titan::cpu
// (dispatch.h:139-152); these wrappers give ctypes plain C names.
#include <cstdint>
#include <vector>

namespace titan {
namespace cpu {
void dequant_matvec_int4_avx512(const uint32_t* weights, const uint16_t* scales,
                                const uint16_t* biases, const float* input,
                                float* output, int rows, int cols, int group_size);
void expert_forward_int4_cpu(const float* input, const uint32_t* gate_w,
                             const uint16_t* gate_s, const uint16_t* gate_b,
                             const uint32_t* up_w, const uint16_t* up_s,
                             const uint16_t* up_b, const uint32_t* down_w,
                             const uint16_t* down_s, const uint16_t* down_b,
                             float* output, float* scratch, int hidden_dim,
                             int inter_dim, int group_size);
// Field order of the task record consumed by execute_experts_parallel
// (expert_cpu.cpp:29-37); the binding needs the identical layout.
struct ExpertTask {
    const float* input;
    const void* expert_data;
    float* output;
    float* scratch;
    int hidden_dim;
    int inter_dim;
    int group_size;
};
void execute_experts_parallel(const std::vector<ExpertTask>& tasks,
                              int num_threads_per_expert);
}  // namespace cpu
}  // namespace titan

extern "C" {

void ref_dequant_matvec_int4(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                             const float* x, float* y, int rows, int cols, int gs) {
    titan::cpu::dequant_matvec_int4_avx512(w, s, b, x, y, rows, cols, gs);
}

// One task per expert, each over a blob laid out as in expert_cpu.cpp:50-86.
void ref_execute_experts_parallel(const float* const* inputs, const void* const* blobs,
                                  float* const* outputs, float* const* scratch,
                                  int n, int hidden_dim, int inter_dim, int gs) {
    std::vector<titan::cpu::ExpertTask> tasks;
    for (int i = 0; i < n; i++)
        tasks.push_back({inputs[i], blobs[i], outputs[i], scratch[i],
                         hidden_dim, inter_dim, gs});
    titan::cpu::execute_experts_parallel(tasks, 1);
}

}  // extern "C"
