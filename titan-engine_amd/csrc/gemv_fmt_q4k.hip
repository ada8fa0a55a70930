// gemv_fmt_q4k.hip -- instantiates the GEMV kernels for TITAN_Q4_K.
#include "gemv_impl.h"

namespace tq {
void dispatch_gemv_q4k(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    dispatch_fmt<TITAN_Q4_K>(a, layout, mcount, mode, total_tiles, st);
}
void dispatch_gemv_generic_q4k(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    launch_generic<TITAN_Q4_K>(a, mcount, rows, st);
}
bool gemv_has_mfma_q4k() { return fmt_has_mfma<TITAN_Q4_K>(); }
}  // namespace tq
