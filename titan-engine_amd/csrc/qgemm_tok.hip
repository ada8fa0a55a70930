// qgemm_tok.hip -- INT4 dequant-GEMM for several tokens (M >= 5), TILED layout.
//
// Y[m][r] = sum_c x[m][c] * (q[r][c] * s[r][g] + b[r][g]),  g = c / group_size
// (dequant.cu:23-104 semantics, fp32 accumulation) for up to TITAN_MAX_BATCH
// problems that share the token count.
//
// The GEMV kernel stages every token's whole activation row per workgroup,
// which stops scaling past a few tokens.  Here a workgroup owns 16 * RT
// weight rows of one problem and a tile of TM tokens; its 4 waves split K.
// Each wave stages its tokens' activations in 128-column K slabs (one 64-byte
// weight chunk per row) in LDS as fp16 and streams the packed codes of the RT
// tiles two slabs ahead in three rotating register sets.
//
// Matrix cores: v_mfma_f32_16x16x32_f16 with tokens as A and codes as B.  A
// lane's code word holds 8 consecutive columns; masking nibble fields into
// fp16 mantissas gives the exact subnormals q * 2^-24:
//   {w, w >> 4, w >> 8, w >> 12} & 0x000F000F = columns (0,4) (1,5) (2,6) (3,7)
// and the staged activations use the same column order.  Each scale group
// (32..128 columns, a power of two) accumulates into its own fp32 tile,
// folded exactly as acc += (s * 2^24) * C + b * sum(x) -- the activation
// sums come from one more MFMA against ones, shared by the RT tiles.
#include "common.h"
#include "layout.h"
#include "fast.h"
#include "qgemm_tok.h"
#include "xitem.h"

namespace tq {

typedef _Float16 th8 __attribute__((ext_vector_type(8)));
typedef float tf4 __attribute__((ext_vector_type(4)));

constexpr int kTokThreads = 256;
constexpr int kTokSlab = 128;            // K columns per slab = one chunk
constexpr int kTokLdr = kTokSlab + 8;    // halves per LDS row (16 B pad)

struct TokProb {
    const uint8_t* w;    // TILED INT4 buffer
    const void* x;
    void* y;
    int64_t ldx, ldy;
    int rows, cols, gs;
};
struct TokArgs {
    TokProb p[TITAN_MAX_BATCH];
    int M;
};

// columns (0,4,1,5,2,6,3,7) of 8 staged fp16 activations
TQ_DEV uint4 tok_perm8(uint4 h) {
    return make_uint4(__builtin_amdgcn_perm(h.z, h.x, 0x05040100u),
                      __builtin_amdgcn_perm(h.z, h.x, 0x07060302u),
                      __builtin_amdgcn_perm(h.w, h.y, 0x05040100u),
                      __builtin_amdgcn_perm(h.w, h.y, 0x07060302u));
}

TQ_DEV th8 tok_b8(uint32_t w) {
    const uint4 v = make_uint4(w & 0x000F000Fu, (w >> 4) & 0x000F000Fu, (w >> 8) & 0x000F000Fu,
                               (w >> 12) & 0x000F000Fu);
    return __builtin_bit_cast(th8, v);
}

// TM tokens per workgroup (blockIdx.x walks row blocks and token tiles,
// blockIdx.y the problems); the workgroup owns
// RT 16-row tiles and its 4 waves split K in quarters, each wave staging its
// own activation slabs (no barrier in the main loop), with a deterministic
// reduction of the 4 partial sums through LDS at the end.  FW code words (32
// columns each) per scale fold.
// STREAM: one token tile reads each weight once (nontemporal loads); with
// more tiles the later tiles re-read the codes from the caches.
// BF (launches of up to 8 tokens): every load issued without a branch and the
// activations two slabs ahead (three register sets, like the weights); the
// slab count is rounded up to whole triples, the extra slabs reading zero
// codes and their folds discarded.  8B layer: 5 tokens 31.8 -> 28.2 us,
// 8 tokens 32.4 -> 30.4 us; from 12 tokens on it measured 2-6% slower.
template <int TM, int RT, int FW, int XDT, int ODT, bool STREAM, bool BF>
__global__ __launch_bounds__(kTokThreads) void qgemm_tok_int4_kernel(TokArgs a) {
    constexpr int NB = TM / 16;
    constexpr int NI = TM * kTokSlab / 8 / 64;  // staging items per lane
    constexpr int NF = 4 / FW;                  // folds per chunk
    constexpr int XS = TM * kTokLdr;            // halves of one wave's stage
    constexpr int RED = 4 * RT * NB * 64 * 16 / 2;  // halves of the K-quarter reduction
    __shared__ __attribute__((aligned(16))) _Float16 xs_all[4 * XS > RED ? 4 * XS : RED];

    // blockIdx.x = (row block, token tile) with the token tiles of a row block
    // 8 workgroups apart: on the same XCD, so the second reads of a row
    // block's weights come from its L2
    const TokProb P = a.p[blockIdx.y];
    const int ntt = (a.M + TM - 1) / TM;
    const int grp = blockIdx.x / (8 * ntt), rem = blockIdx.x - grp * 8 * ntt;
    const int rb0 = (grp * 8 + (rem & 7)) * (16 * RT);
    if (rb0 >= P.rows) return;  // uniform per workgroup
    const int t0 = (rem >> 3) * TM;
    const int nt = min(TM, a.M - t0), nb = (nt + 15) >> 4;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane >> 4, r = lane & 15;
    const Geo geo = make_geo(TITAN_INT4, P.rows, P.cols, P.gs);
    const int ntile = P.rows >> 4;
    const int nslab = P.cols / kTokSlab;
    const int s_beg = (wave * nslab) >> 2, s_end = ((wave + 1) * nslab) >> 2;  // this wave's K
    const int gshift = 31 - __builtin_clz(P.gs);  // group = column >> gshift
    _Float16* xs = xs_all + wave * XS;

    // tile q (clamped past the last row: loaded, never stored).  BF: its
    // codes through a buffer resource over this wave's slabs (a slab past
    // the wave's last one reads zeros and fetches nothing), the activation
    // and scale slabs clamped into [0, s_end).
    uint32_t code_off[RT], sb_base[RT];
    CodeSrc csrc[RT];
    const uint32_t lane16 = (uint32_t)(j * 16 + r) * 16u;
#pragma unroll
    for (int q = 0; q < RT; q++) {
        const int t = min((rb0 >> 4) + q, ntile - 1);
        code_off[q] = (uint32_t)tiled_code_off(geo, t * 16 + r, 0, j);
        sb_base[q] = (uint32_t)tiled_sb_off(geo, t * 16 + r, 0);
        csrc[q] = CodeSrc{P.w + ((size_t)t * geo.nchunks + s_beg) * 1024u,
                          (uint32_t)(s_end > s_beg ? s_end - s_beg : 0) * 1024u, lane16};
    }
    auto in_k = [&](int s) { return BF ? max(min(s, s_end - 1), 0) : s; };

    // staging: item it covers token row rr, columns [8 cg, 8 cg + 8) of a slab
    int64_t src[NI];
    int ldsi[NI];
#pragma unroll
    for (int it = 0; it < NI; it++) {
        const int idx = it * 64 + lane, rr = idx / (kTokSlab / 8), cg = idx % (kTokSlab / 8);
        ldsi[it] = rr * kTokLdr + cg * 8;
        src[it] = rr < nt ? (int64_t)(t0 + rr) * P.ldx + cg * 8 : -1;
    }
    auto load_x = [&](int s, XItem<XDT>* xr) {
        const int sk = in_k(s);
#pragma unroll
        for (int it = 0; it < NI; it++) {
            if (src[it] >= 0) xr[it].load(P.x, src[it] + (int64_t)sk * kTokSlab);
            else xr[it].zero();
        }
    };
    struct WSet { uint4 c[RT]; uint32_t sb[RT][NF]; };
    auto load_w = [&](int s, WSet& w) {
        const int sk = in_k(s);
#pragma unroll
        for (int q = 0; q < RT; q++) {
            if constexpr (BF) {
                w.c[q] = ld_code_chunk<STREAM>(csrc[q].at(s - s_beg), lane16, 0);
            } else {
                const uint8_t* cp = P.w + code_off[q] + (uint32_t)s * 1024u;
                w.c[q] = STREAM ? ld_stream_u128(cp) : *(const uint4*)cp;
            }
#pragma unroll
            for (int f = 0; f < NF; f++) {
                // scale slot: one per chunk for groups of a chunk or more, else one per group
                const uint32_t g = (uint32_t)((sk * kTokSlab + f * FW * 32) >> gshift);
                const uint32_t sl = P.gs >= kTokSlab ? (uint32_t)sk : g;
                w.sb[q][f] = *(const uint32_t*)(P.w + sb_base[q] + (sl >> 2) * 256u + (sl & 3u) * 4u);
            }
        }
    };

    tf4 acc[RT][NB];
#pragma unroll
    for (int q = 0; q < RT; q++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[q][b] = tf4{0, 0, 0, 0};
    const th8 ones = __builtin_bit_cast(th8, make_uint4(0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u));

    // Per wave: activations one slab ahead, weights two slabs ahead in three
    // rotating register sets.  The stage is the wave's own, and LDS
    // operations of one wave complete in order, so a slab's reads finish
    // before the next slab overwrites it.
    XItem<XDT> x0[NI], x1[NI], x2[NI];  // x1, x2: BF only
    // weights WD slabs ahead (WD + 1 register sets); four row tiles a wave
    // keep one slab ahead in two sets, for fewer registers
    constexpr int WD = (!BF && RT >= 4) ? 1 : 2;
    WSet w0, w1, w2;
    if constexpr (BF) {
        load_x(s_beg, x0);
        load_w(s_beg, w0);
        load_x(s_beg + 1, x1);
        load_w(s_beg + 1, w1);
    } else if (s_beg < s_end) {
        load_x(s_beg, x0);
        load_w(s_beg, w0);
        if (WD == 2 && s_beg + 1 < s_end) load_w(s_beg + 1, w1);
    }
    auto step = [&](int s, const WSet& wc, WSet& wnext2, XItem<XDT>* xc, XItem<XDT>* xnext2) {
        const bool live = !BF || s < s_end;
#pragma unroll
        for (int it = 0; it < NI; it++) *(uint4*)(xs + ldsi[it]) = tok_perm8(xc[it].h());
        if constexpr (BF) {
            load_x(s + 2, xnext2);
            load_w(s + 2, wnext2);
        } else {
            if (s + 1 < s_end) load_x(s + 1, xc);
            if (s + WD < s_end) load_w(s + WD, wnext2);
        }
#pragma unroll
        for (int f = 0; f < NF; f++) {
            tf4 C[RT][NB], O[NB];
#pragma unroll
            for (int ii = 0; ii < FW; ii++) {
                const int i = f * FW + ii;
                th8 B[RT];
#pragma unroll
                for (int q = 0; q < RT; q++) {
                    const uint4 cw = wc.c[q];
                    B[q] = tok_b8(i == 0 ? cw.x : i == 1 ? cw.y : i == 2 ? cw.z : cw.w);
                }
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    if (b < nb) {
                        const th8 A = *(const th8*)(xs + (b * 16 + r) * kTokLdr + 32 * i + 8 * j);
                        const tf4 z = tf4{0, 0, 0, 0};
                        O[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, ones, ii == 0 ? z : O[b], 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < RT; q++)
                            C[q][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[q], ii == 0 ? z : C[q][b], 0, 0, 0);
                    }
                }
            }
            // fold the scale group: acc += s 2^24 C + b sum(x)
#pragma unroll
            for (int q = 0; q < RT; q++) {
                const uint32_t sbv = wc.sb[q][f];
                const float sc = f16_to_f32(sbv & 0xFFFFu) * 16777216.0f, bi = f16_to_f32(sbv >> 16);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    if (b < nb) {
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const float nv = __builtin_fmaf(bi, O[b][v], __builtin_fmaf(sc, C[q][b][v], acc[q][b][v]));
                            acc[q][b][v] = live ? nv : acc[q][b][v];
                        }
                    }
                }
            }
        }
    };
    if constexpr (!BF && WD == 1) {  // two sets: pairs of slabs
        for (int s = s_beg; s < s_end; s += 2) {
            step(s, w0, w1, x0, x0);
            if (s + 1 < s_end) step(s + 1, w1, w0, x0, x0);
        }
    } else
    for (int s = s_beg; s < s_end; s += 3) {
        if constexpr (BF) {
            step(s, w0, w2, x0, x2);
            step(s + 1, w1, w0, x1, x0);
            step(s + 2, w2, w1, x2, x1);
        } else {
            step(s, w0, w2, x0, x0);
            if (s + 1 < s_end) step(s + 1, w1, w0, x0, x0);
            if (s + 2 < s_end) step(s + 2, w2, w1, x0, x0);
        }
    }

    // reduce the 4 K quarters: wave w sums tiles q = w, w + 4, ... in wave order
    __syncthreads();
    tf4* red = (tf4*)xs_all;  // [wave][q][b][lane]
#pragma unroll
    for (int q = 0; q < RT; q++)
#pragma unroll
        for (int b = 0; b < NB; b++) red[((wave * RT + q) * NB + b) * 64 + lane] = acc[q][b];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RT; q++) {
        if ((q & 3) != wave) continue;
        const int t = (rb0 >> 4) + q;
        if (t >= ntile) continue;
        const int row = t * 16 + r;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            if (b >= nb) break;
            tf4 sum = red[((0 * RT + q) * NB + b) * 64 + lane];
#pragma unroll
            for (int w2 = 1; w2 < 4; w2++) {
                const tf4 o = red[((w2 * RT + q) * NB + b) * 64 + lane];
                sum[0] += o[0]; sum[1] += o[1]; sum[2] += o[2]; sum[3] += o[3];
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int tok = b * 16 + 4 * j + v;
                if (tok < nt) store_out(P.y, (int64_t)(t0 + tok) * P.ldy + row, ODT, sum[v]);
            }
        }
    }
}

template <int TM, int RT, int FW, int XDT, int ODT>
void launch_tok(const TokArgs& a, int maxrows, hipStream_t st) {
    const int nrb = ((maxrows + 16 * RT - 1) / (16 * RT) + 7) / 8 * 8;
    dim3 grid(nrb * ((a.M + TM - 1) / TM), TITAN_MAX_BATCH, 1);
    if (TM == 16 && a.M <= 8)
        hipLaunchKernelGGL((qgemm_tok_int4_kernel<TM, RT, FW, XDT, ODT, true, true>), grid, dim3(kTokThreads), 0, st, a);
    else if (a.M <= TM)
        hipLaunchKernelGGL((qgemm_tok_int4_kernel<TM, RT, FW, XDT, ODT, true, false>), grid, dim3(kTokThreads), 0, st, a);
    else
        hipLaunchKernelGGL((qgemm_tok_int4_kernel<TM, RT, FW, XDT, ODT, false, false>), grid, dim3(kTokThreads), 0, st, a);
}

template <int TM, int RT, int FW, int XDT>
void launch_tok_o(const TokArgs& a, int maxrows, int ydt, hipStream_t st) {
    switch (ydt) {
        case TITAN_FP32: launch_tok<TM, RT, FW, XDT, TITAN_FP32>(a, maxrows, st); break;
        case TITAN_FP16: launch_tok<TM, RT, FW, XDT, TITAN_FP16>(a, maxrows, st); break;
        default: launch_tok<TM, RT, FW, XDT, TITAN_BF16>(a, maxrows, st); break;
    }
}

template <int TM, int RT, int FW>
void launch_tok_x(const TokArgs& a, int maxrows, int xdt, int ydt, hipStream_t st) {
    switch (xdt) {
        case TITAN_FP32: launch_tok_o<TM, RT, FW, TITAN_FP32>(a, maxrows, ydt, st); break;
        case TITAN_FP16: launch_tok_o<TM, RT, FW, TITAN_FP16>(a, maxrows, ydt, st); break;
        default: launch_tok_o<TM, RT, FW, TITAN_BF16>(a, maxrows, ydt, st); break;
    }
}

template <int TM, int RT>
void launch_tok_f(const TokArgs& a, int maxrows, int fw, int xdt, int ydt, hipStream_t st) {
    if (fw == 4) launch_tok_x<TM, RT, 4>(a, maxrows, xdt, ydt, st);
    else if (fw == 2) launch_tok_x<TM, RT, 2>(a, maxrows, xdt, ydt, st);
    else launch_tok_x<TM, RT, 1>(a, maxrows, xdt, ydt, st);
}

}  // namespace tq

namespace tqh {

bool tok_int4_ok(const titan_qweight* Ws, const void* const* Xs, const int64_t* ldx, int n,
                 int xdt) {
    const int esz = xdt == TITAN_FP32 ? 4 : 2;
    for (int i = 0; i < n; i++) {
        const titan_qweight& W = Ws[i];
        if (W.format != TITAN_INT4 || W.layout != TITAN_LAYOUT_TILED) return false;
        if (!tq::tiled_total_bytes(TITAN_INT4, W.rows, W.cols, W.group_size)) return false;
        if (((uintptr_t)W.codes & 15) || ((uintptr_t)Xs[i] & 15) || (ldx[i] * esz) % 16) return false;
        if (W.group_size != Ws[0].group_size) return false;
    }
    return true;
}

int run_tok_int4(const titan_qweight* Ws, const void* const* Xs, const int64_t* ldx,
                 void* const* Ys, const int64_t* ldy, int n, int xdt, int ydt, int M,
                 hipStream_t st) {
    tq::TokArgs a{};
    a.M = M;
    // problems in launch order long rows first: grid.y walks the problems, so
    // the workgroups of the longest rows (which take longest) start first
    // instead of forming the launch's tail (8B layer, 16 tokens: the
    // down projection started at 15 us and ended at 43 us)
    int order[TITAN_MAX_BATCH];
    for (int i = 0; i < n; i++) order[i] = i;
    for (int i = 1; i < n; i++)
        for (int k = i; k > 0 && Ws[order[k]].cols > Ws[order[k - 1]].cols; k--) {
            const int t = order[k]; order[k] = order[k - 1]; order[k - 1] = t;
        }
    int maxrows = 0;
    for (int i = 0; i < TITAN_MAX_BATCH; i++) {
        tq::TokProb& p = a.p[i];
        if (i < n) {
            const int q = order[i];
            p.w = (const uint8_t*)Ws[q].codes;
            p.x = Xs[q];
            p.y = Ys[q];
            p.ldx = ldx[q];
            p.ldy = ldy[q];
            p.rows = Ws[q].rows;
            p.cols = Ws[q].cols;
            p.gs = Ws[q].group_size;
            maxrows = maxrows > p.rows ? maxrows : p.rows;
        } else {
            p.rows = 0;  // idle grid.y slots exit at once
        }
    }
    const int gs = Ws[0].group_size;
    const int fw = gs >= 128 ? 4 : gs / 32;
    // 16-token tiles (measured on the 8B layer): two row tiles a wave up to 16
    // tokens, four beyond (32-token tiles, or two row tiles, measured 1-8%
    // slower at 24 and 32 tokens; 64-token tiles 10-36% slower from 80 to
    // 512 tokens)
    if (M <= 16) tq::launch_tok_f<16, 2>(a, maxrows, fw, xdt, ydt, st);
    else tq::launch_tok_f<16, 4>(a, maxrows, fw, xdt, ydt, st);
    return launch_status();
}

}  // namespace tqh
