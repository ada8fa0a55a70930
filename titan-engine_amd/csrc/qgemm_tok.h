// qgemm_tok.h -- host entry of the token-tiled INT4 dequant-GEMM (qgemm_tok.hip).
#pragma once

#include "titan_qmm.h"

namespace tqh {

// Whether the token-tiled kernel serves these problems (INT4, TILED, one
// group size, 16-byte aligned codes and activation rows).
bool tok_int4_ok(const titan_qweight* Ws, const void* const* Xs, const int64_t* ldx, int n,
                 int xdt);
// Y_i = W_i X_i for M tokens; problems of one launch share M.
int run_tok_int4(const titan_qweight* Ws, const void* const* Xs, const int64_t* ldx,
                 void* const* Ys, const int64_t* ldy, int n, int xdt, int ydt, int M,
                 hipStream_t st);

}  // namespace tqh
