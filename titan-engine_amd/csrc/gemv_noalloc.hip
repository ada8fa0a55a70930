// gemv_noalloc.hip -- the batched dequant-GEMV with its K-split workspace in
// a static device array, for callers that cannot allocate device memory.
//
// The array `scratch` is a file-scope device variable: in host code its name
// stands for a host-side handle, not a device address.  The device address is
// looked up once per device with hipGetSymbolAddress and kept in
// g_scratch[device]; only that pointer is handed to kernels.
#include <mutex>

#include "gemv_impl.h"

static __device__ __align__(256) unsigned char scratch[TITAN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];

// the split's counters: the fixed region at the start of the workspace
constexpr int kCounterWords = (int)(tq::kGemvXsCntBytes / 4);
static_assert(tq::kGemvXsCntBytes < TITAN_NOALLOC_SCRATCH_BYTES, "scratch holds the counters");

__global__ void scratch_clear_kernel(unsigned* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The device address of this device's scratch; on the first call on a device
// its counter region is cleared by a kernel on `st` (a kernel, not a memset,
// so that a first call under stream capture records no memset node).
int scratch_for_current_device(hipStream_t st, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TITAN_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TITAN_ERR_LAUNCH;
        hipLaunchKernelGGL(scratch_clear_kernel, dim3(8), dim3(256), 0, st, (unsigned*)p, kCounterWords);
        if (hipGetLastError() != hipSuccess) return TITAN_ERR_LAUNCH;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return TITAN_OK;
}

}  // namespace

extern "C" int titan_qgemm_batched_noalloc(const titan_qweight* Ws, const void* const* Xs,
                                           void* const* Ys, int n, int x_dtype, int y_dtype,
                                           int M, hipStream_t stream) {
    if (!Ws || !Xs || !Ys || n <= 0 || n > TITAN_MAX_BATCH || M <= 0) return TITAN_ERR_INVALID_ARG;
    int rows[TITAN_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        if (Ws[i].rows <= 0) return TITAN_ERR_INVALID_ARG;
        rows[i] = Ws[i].rows;
    }
    const size_t need = titan_qgemm_workspace_bytes(rows, n, M);
    if (need == 0) return TITAN_ERR_INVALID_ARG;
    if (need > TITAN_NOALLOC_SCRATCH_BYTES) return TITAN_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (int s = scratch_for_current_device(stream, &ws)) return s;
    // the same launches as titan_qgemm_batched_ws with this workspace; its
    // checks and kernels are shared, and it allocates nothing either
    return titan_qgemm_batched_ws(Ws, Xs, Ys, n, x_dtype, y_dtype, M, ws,
                                  (size_t)TITAN_NOALLOC_SCRATCH_BYTES, stream);
}
