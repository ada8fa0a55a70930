// gemv_fmt_int2.hip -- instantiates the GEMV kernels for TITAN_INT2.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_int2(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_INT2>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_int2(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_INT2>(a, mcount, rows, st);
}
bool gemv_has_mfma_int2() { return fmt_has_mfma<TITAN_INT2>(); }
}  // namespace tq
