// gemv_fmt_q3k.hip -- instantiates the GEMV kernels for TITAN_Q3_K.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_q3k(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_Q3_K>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_q3k(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_Q3_K>(a, mcount, rows, st);
}
bool gemv_has_mfma_q3k() { return fmt_has_mfma<TITAN_Q3_K>(); }
}  // namespace tq
