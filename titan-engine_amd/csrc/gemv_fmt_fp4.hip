// gemv_fmt_fp4.hip -- instantiates the GEMV kernels for TITAN_FP4.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_fp4(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_FP4>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_fp4(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_FP4>(a, mcount, rows, st);
}
bool gemv_has_mfma_fp4() { return fmt_has_mfma<TITAN_FP4>(); }
}  // namespace tq
