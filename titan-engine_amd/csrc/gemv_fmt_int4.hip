// gemv_fmt_int4.hip -- instantiates the GEMV kernels for TITAN_INT4.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_int4(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_INT4>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_int4(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_INT4>(a, mcount, rows, st);
}
bool gemv_has_mfma_int4() { return fmt_has_mfma<TITAN_INT4>(); }
}  // namespace tq
