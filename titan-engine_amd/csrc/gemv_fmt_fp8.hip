// gemv_fmt_fp8.hip -- instantiates the GEMV kernels for TITAN_FP8_E4M3.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_fp8(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_FP8_E4M3>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_fp8(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_FP8_E4M3>(a, mcount, rows, st);
}
bool gemv_has_mfma_fp8() { return fmt_has_mfma<TITAN_FP8_E4M3>(); }
}  // namespace tq
