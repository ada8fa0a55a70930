// gemv_fmt_nvfp4.hip -- instantiates the GEMV kernels for TITAN_NVFP4.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_nvfp4(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_NVFP4>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_nvfp4(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_NVFP4>(a, mcount, rows, st);
}
bool gemv_has_mfma_nvfp4() { return fmt_has_mfma<TITAN_NVFP4>(); }
}  // namespace tq
