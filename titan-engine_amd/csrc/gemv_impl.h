// gemv_impl.h -- dequant-GEMV / small-M dequant-GEMM kernels for decode.
//
// Replaces the reference's one-block-per-row kernels (dequant.cu:23-172,
// fp4.cu:28-84, fp4.cu:187-238).  Design for gfx950:
//  * A workgroup of 4 waves owns up to 4 row tiles of 16 rows; waves that
//    share a tile (K split) take contiguous spans of its 1 KiB chunks, and
//    long rows may also be split across workgroups (caller workspace).
//  * Each wave holds two groups of U chunks of codes in registers, so the
//    next group's loads (4 KiB per wave) are in flight while the current one
//    is folded; loads never depend on a branch, and the code plane is read
//    through a buffer resource whose range check turns the loads past a
//    wave's last group into zero-traffic reads.
//  * Activations are staged per workgroup into LDS (phases of at most
//    kGemvLdsBytes for long K / many tokens): fp32 in column order for fp32 /
//    bf16 inputs, fp16 in each format's pairing order for fp16 inputs.
//  * Folding (fast.h): fp32 FMA, packed fp16 dot products, or MFMA with the
//    activations as the A operand and the codes as exact fp16 subnormals.
//  * Lanes of a row (VALU modes) are reduced with two cross-lane shuffles,
//    waves through LDS; MFMA accumulators already hold whole-row sums.
#pragma once
#include "fast.h"
#include <type_traits>

namespace tq {

// the kernels' helper lambdas carry register arrays by reference: they must
// be inlined, or the arrays go to scratch memory
#ifndef TQ_AI
#define TQ_AI __attribute__((always_inline))
#endif

template <class F, class = void>
struct has_stage_local : std::false_type {};
template <class F>
struct has_stage_local<F, std::void_t<decltype(F::STAGE_LOCAL)>> : std::true_type {};
template <class F, class = void>
struct requires_sb_cell : std::false_type {};
template <class F>
struct requires_sb_cell<F, std::void_t<decltype(F::SB_CELL)>> : std::true_type {};

template <class F, class = void>
struct has_no_exact : std::false_type {};
template <class F>
struct has_no_exact<F, std::void_t<decltype(F::NO_EXACT)>> : std::true_type {};
// Whether one-phase launches take the EXACT kernel (a format may opt out when
// that kernel's register allocation costs more than its simpler loop saves)
template <class F>
constexpr bool allow_exact() {
    if constexpr (has_no_exact<F>::value) return !F::NO_EXACT;
    else return true;
}

#ifndef TQ_GEMV_WAVES_TARGET
#define TQ_GEMV_WAVES_TARGET 2048
#endif
template <class F, class = void>
struct has_xs_min_m : std::false_type {};
template <class F>
struct has_xs_min_m<F, std::void_t<decltype(F::XS_MIN_M)>> : std::true_type {};
// fewest tokens for which a caller workspace splits K across workgroups
template <class F>
constexpr int xs_min_m() {
    if constexpr (has_xs_min_m<F>::value) return F::XS_MIN_M;
    else return 1;
}
template <class F, class = void>
struct has_waves_target_m1 : std::false_type {};
template <class F>
struct has_waves_target_m1<F, std::void_t<decltype(F::WAVES_TARGET_M1)>> : std::true_type {};
template <class F, class = void>
struct has_waves_target : std::false_type {};
template <class F>
struct has_waves_target<F, std::void_t<decltype(F::WAVES_TARGET)>> : std::true_type {};
// Waves a launch aims for (the K split per row tile follows from it); a
// format may set its own figure for every token count (WAVES_TARGET) or for
// one token (WAVES_TARGET_M1)
template <class F, int M>
constexpr long long waves_target() {
    if constexpr (M == 1 && has_waves_target_m1<F>::value) return F::WAVES_TARGET_M1;
    else if constexpr (has_waves_target<F>::value) return F::WAVES_TARGET;
    else return TQ_GEMV_WAVES_TARGET;
}

template <class F, class = void>
struct has_ks1_mp : std::false_type {};
template <class F>
struct has_ks1_mp<F, std::void_t<decltype(F::KS1_MULTI_PHASE)>> : std::true_type {};
template <class F>
constexpr bool has_ks1_multi_phase() {
    if constexpr (has_ks1_mp<F>::value) return F::KS1_MULTI_PHASE;
    else return false;
}

template <class F, class = void>
struct has_sx_max_m : std::false_type {};
template <class F>
struct has_sx_max_m<F, std::void_t<decltype(F::SX_MAX_M)>> : std::true_type {};

// Most tokens for which the MFMA fold takes activation sums from LDS (SX)
// instead of an extra MFMA against ones.  Sums over 32 or more columns keep
// four tokens per 32 columns; 16-column sums (SX_MAX_M = 2) keep two tokens
// per 16 columns, in the same space.
template <class F>
constexpr int sx_max_m() {
    if constexpr (has_sx_max_m<F>::value) return F::SX_MAX_M;
    else return 4;
}
// LDS index of the sum of window `b` (SW columns each) for token m
template <int SW>
TQ_DEV int sx_index(int b, int m) {
    static_assert(SW == 16 || SW % 32 == 0, "sum window");
    if constexpr (SW == 16) return 2 * b + m;
    else return 4 * (b * (SW / 32)) + m;
}

#ifndef TQ_GEMV_U
#define TQ_GEMV_U 4
#endif
constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
#ifndef TQ_GEMV_LDS_KB
#define TQ_GEMV_LDS_KB 32
#endif
#ifndef TQ_GEMV_KS_MAX
#define TQ_GEMV_KS_MAX 2
#endif
constexpr int kGemvLdsBytes = TQ_GEMV_LDS_KB * 1024;  // activation stage per workgroup
constexpr int kGemvMaxLdsBytes = 96 * 1024;  // larger stage of small launches (dynamic LDS limit set)

enum { kModeF32 = 0, kModeDot2 = 1, kModeMfma = 2 };

struct GemvProb {
    WDesc w;
    const void* x;
    void* y;
    int64_t ldx, ldy;
    int nchunks;   // cols / CHUNK_COLS
    int wg_begin;  // first workgroup of this problem
    int ntiles;    // row tiles of this problem: [tile0, tile0 + ntiles)
    int tile0;     // first row tile (0 unless the launch split the matrix's rows)
    int gsteps;    // MFMA word steps per scale group (power of two <= 4)
    int ks_log;    // log2 of the waves sharing one row tile (K split)
    // K split across workgroups (xs_log > 0 only with a caller workspace):
    // 2^xs_log consecutive workgroups take equal contiguous chunk ranges of
    // the same row tiles, write fp32 partials to wsp[part][token][row]
    // (row stride rpad) and the last to arrive (counter wsc[tile group])
    // adds them in part order and stores the outputs.
    int xs_log;
    int rpad;
    float* wsp;
    int* wsc;
};

// a launch holds the caller's problems plus at most one row split of one of them
constexpr int kGemvMaxProbs = TITAN_MAX_BATCH + 1;

struct GemvArgs {
    // first workgroup of each problem (ascending), INT_MAX past the last one:
    // the kernel finds its problem from this one block of scalar loads
    int wgb[kGemvMaxProbs];
    GemvProb p[kGemvMaxProbs];
    int n;
    int xdt, ydt;
    int m0;      // first token of this launch
    int mcount;  // tokens in this launch (<= the kernel's template width)
    int pc;      // staged columns per phase (whole groups of chunks)
    // host only: caller workspace for the cross-workgroup K split (null: none)
    void* ws;
    size_t ws_bytes;
};

#ifndef TQ_GEMV_XS_WAVES
#define TQ_GEMV_XS_WAVES 2048  // waves the cross-workgroup split aims for
#endif
#ifndef TQ_GEMV_XS_MAX_LOG
#define TQ_GEMV_XS_MAX_LOG 4   // at most 16 workgroups share a row tile
#endif

// Workspace of the cross-workgroup K split.  The counters (one int per tile
// group) of every problem of a call live in one fixed region at the start of
// the workspace, indexed by the call's running tile count: the split engages
// only below TQ_GEMV_XS_WAVES row tiles in total, so every counter of every
// call falls in that region, which nothing else writes.  Calls with other
// problem sets and token counts can therefore share one workspace: the
// counters a call finds are the zeros the previous call left.  The partials
// [16][m][rpad] fp32 of each problem follow the counter region.
constexpr size_t kGemvXsCntBytes = (size_t)TQ_GEMV_XS_WAVES * 4;
inline size_t gemv_xs_part_bytes(int rows, int m) {
    return (size_t)m * ((size_t)(rows + 15) / 16 * 16) * 4 << TQ_GEMV_XS_MAX_LOG;
}

// fp32 activations in column order plus fp32 sums of every 16 columns.
template <int M>
TQ_DEV void stage_f32(float* xf, float* s16, int pc, const void* x, int xdt, int64_t ldx,
                      int m0, int mcount, int col0, int ncols, int tid) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const int64_t off = (int64_t)(m0 + m) * ldx + col0;
        float* dst = xf + m * pc;
        for (int c = tid; c < ncols; c += kGemvThreads)
            dst[c] = m < mcount ? load_act(x, off + c, xdt) : 0.0f;
    }
    __syncthreads();
    for (int e = tid; e < M * (ncols >> 4); e += kGemvThreads) {
        const int m = e / (ncols >> 4), g = e % (ncols >> 4);
        const float* p = xf + m * pc + 16 * g;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            a += p[i];
            b += p[i + 1];
        }
        s16[m * (pc >> 4) + g] = a + b;
    }
}

// fp16 activations in the format's pairing order (F::stage8) and, for the
// VALU fold, fp32 sums of every 16 columns.  Rows of x are 16-byte aligned.
// SX (MFMA with at most 4 tokens): fp32 sums of the activations over every
// SW columns (one scale group, or one 32-column sub-block), token slots 0..3,
// at s16[4 * (col / 32) + token] for the first column of each span.
template <int M, int SW>
TQ_DEV void stage_sums(float* sx, const void* x, int64_t ldx, int m0, int mcount, int col0,
                       int ncols, int tid) {
    constexpr int TPW = SW == 16 ? 2 : 4;  // token slots per window
    for (int e = tid; e < TPW * (ncols / SW); e += kGemvThreads) {
        const int b = e / TPW, m = e % TPW;
        float s = 0.0f;
        if (m < mcount && m < M) {
            const _Float16* src = (const _Float16*)x + (int64_t)(m0 + m) * ldx + col0 + SW * b;
            float a0 = 0.0f, a1 = 0.0f;
            for (int q = 0; q < SW; q += 8) {
                _Float16 h[8];
                ldh8(src + q, h);
#pragma unroll
                for (int i = 0; i < 8; i += 2) {
                    a0 += (float)h[i];
                    a1 += (float)h[i + 1];
                }
            }
            s = a0 + a1;
        }
        sx[sx_index<SW>(b, m)] = s;
    }
}

template <class F, int M, bool SUMS>
TQ_DEV void stage_f16(_Float16* xh, float* s16, int pc, const void* x, int64_t ldx, int m0,
                      int mcount, int col0, int ncols, int tid) {
#pragma unroll
    for (int m = 0; m < M; m++) {
        const _Float16* src = (const _Float16*)x + (int64_t)(m0 + m) * ldx + col0;
        for (int d0 = tid * 8; d0 < ncols; d0 += kGemvThreads * 8)
            *(uint4*)(xh + m * pc + d0) = m < mcount ? F::stage8(src, d0) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (SUMS) {
        for (int e = tid; e < M * (ncols >> 4); e += kGemvThreads) {
            const int m = e / (ncols >> 4), g = e % (ncols >> 4);
            float s = 0.0f;
            if (m < mcount) {
                const _Float16* src = (const _Float16*)x + (int64_t)(m0 + m) * ldx + col0 + 16 * g;
                _Float16 h[8], k[8];
                ldh8(src, h);
                ldh8(src + 8, k);
                float a = 0.0f, b = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    a += (float)h[i];
                    b += (float)k[i];
                }
                s = a + b;
            }
            s16[m * (pc >> 4) + g] = s;
        }
    }
}

// chunks per load group (a larger group needs a proportionally larger
// activation stage, which costs more in occupancy than it gains); a format
// that sets U2_MIN_M / U2_MAX_M folds U2_MIN_M..U2_MAX_M tokens of fp16
// activations (its matrix-core or dot2 fold) in groups of two chunks (half
// the registers in flight a wave, so more waves a SIMD)
template <class F, class = void>
struct has_u2 : std::false_type {};
template <class F>
struct has_u2<F, std::void_t<decltype(F::U2_MIN_M), decltype(F::U2_MAX_M)>> : std::true_type {};
template <class F, int M, int MODE>
constexpr int gemv_u() {
    if constexpr (MODE == (F::HAS_MFMA ? kModeMfma : kModeDot2) && has_u2<F>::value)
        return M >= F::U2_MIN_M && M <= F::U2_MAX_M ? 2 : TQ_GEMV_U;
    else
        return TQ_GEMV_U;
}

template <class F, class = void>
struct has_half_from_u : std::false_type {};
template <class F>
struct has_half_from_u<F, std::void_t<decltype(F::HALF_FROM_U)>> : std::true_type {};
template <class F>
constexpr bool half_from_u() {
    if constexpr (has_half_from_u<F>::value) return F::HALF_FROM_U;
    else return false;
}
static_assert(TQ_GEMV_U % 2 == 0, "chunk groups start at even chunks");

// Formats whose tiled scales come in 16-byte cells (SB_CELL) decode chunk u
// of a group from the cell loaded with chunk u - u % GS.
template <class F>
constexpr bool has_sb_cell() {
    if constexpr (requires_sb_cell<F>::value) return F::SB_CELL;
    else return false;
}
template <class F, int GS, class RawArr>
TQ_DEV typename F::Dec decode_u(const WDesc& W, const RawArr& R, int u, int cc, int j) {
    if constexpr (has_sb_cell<F>()) return F::template decode_cell<GS>(R[u - u % GS].q, u);
    // HALF_FROM_U: the decoder needs only the chunk's parity, and chunk
    // groups start at a multiple of U (even), so u's parity is the chunk's:
    // known at compile time
    else if constexpr (half_from_u<F>()) return F::template decode<GS>(W, R[u], u, j);
    else return F::template decode<GS>(W, R[u], cc, j);
}

// Formats whose stage8 permutes only its own 8 columns (STAGE_LOCAL) turn a
// loaded item into its staged form in registers (stage8_raw).
template <class F>
constexpr bool stage_local() {
    if constexpr (has_stage_local<F>::value) return F::STAGE_LOCAL;
    else return false;
}
// Item e of a staging round: token m, 8-column group d of a row of nb8 groups
// (one token: no division)
template <int M>
TQ_DEV void item_of_m(int e, int nb8, int& m, int& d) {
    if constexpr (M == 1) {
        m = e < nb8 ? 0 : 1;
        d = e;
    } else {
        m = e / nb8;
        d = e - m * nb8;
    }
}
// Sum over the WL lanes ending at this lane within its DPP row of 16 (lanes
// before the row's start count 0): Hillis-Steele steps of row shifts.
template <int N>
TQ_DEV float row_shr_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + N, 0xF, 0xF, true));
}
template <int WL>
TQ_DEV float row_window_sum(float v) {
    if constexpr (WL >= 2) v += row_shr_f<1>(v);
    if constexpr (WL >= 4) v += row_shr_f<2>(v);
    if constexpr (WL >= 8) v += row_shr_f<4>(v);
    if constexpr (WL >= 16) v += row_shr_f<8>(v);
    if constexpr (WL >= 32) {
        // row_bcast:15 with rows 1 and 3 written: the last lane of each odd
        // row adds the even row's sum (rows 0 and 2 add 0)
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    }
    static_assert(WL <= 32, "a sum window spans at most two DPP rows");
    return v;
}
constexpr int kStageItems = 8;  // 16-byte activation loads per thread and round
template <int NI>
struct XStage { uint4 v[NI]; unsigned live; };
template <class F>
TQ_DEV uint4 stage8_raw_of(uint4 v) {
    if constexpr (stage_local<F>()) return F::stage8_raw(v);
    else return v;
}


// EXACT: every problem of the launch has one phase whose groups cover its
// chunks exactly (no chunk past the end of a row inside a group); the host
// picks the kernel, so each kernel holds a single copy of the main loop (a
// second copy in one kernel raised its register allocation by up to 2.5x)
template <class F, int M, int MODE, int GS = 4, bool EXACT = false>
__global__ __launch_bounds__(kGemvThreads) void qgemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // this workgroup's problem: a count over the first-workgroup table, with
    // no chain of dependent scalar loads (a scan over the problems one by one
    // took 2 us to issue the first load of a seven-problem launch)
    // One-problem launches come as a (1, workgroups) grid: their workgroups
    // have blockIdx.x == 0 and skip the table, so the problem's own scalar
    // loads are the first ones (one round trip less before the first
    // weight load); other launches are (workgroups, 1).
    const int bid = blockIdx.x + blockIdx.y;
    int pi = 0;
    if (blockIdx.x != 0) {
#pragma unroll
        for (int i = 1; i < kGemvMaxProbs; i++) pi += bid >= a.wgb[i] ? 1 : 0;
    }
    const GemvProb& P = a.p[pi];
    const WDesc& W = P.w;
    const int rows = W.g.rows;

    // the wave index is uniform: keep the chunk bookkeeping in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r = lane & 15, j = lane >> 4;
    // KS waves share one row tile and split its chunks (part, part + KS, ...)
    const int ks_log = P.ks_log, KS = 1 << ks_log;
    const int part = wave & (KS - 1);
    const int xs_log = P.xs_log, XS = 1 << xs_log;
    const int wgl = bid - P.wg_begin, xpart = wgl & (XS - 1), wgt = wgl >> xs_log;
    const int tile = P.tile0 + wgt * (kGemvWaves >> ks_log) + (wave >> ks_log);
    const int pc = a.pc;
    // this workgroup's chunk range [c0, c0 + nchunks); chunk indices below
    // are relative to c0
    const int nchunks = P.nchunks >> xs_log;
    const int c0 = xpart * nchunks;
    const int colend = XS == 1 ? W.g.cols : (c0 + nchunks) * F::CHUNK_COLS;

    float* xf = lds;
    _Float16* xh = (_Float16*)lds;
    float* s16 = MODE == kModeF32 ? lds + M * pc : lds + M * pc / 2;  // MFMA + SX: 32-col sums

    const int row = tile * 16 + r;
    const typename F::Off off = F::base(W, row < rows ? row : rows - 1, j);  // past the end: not stored
    // tiled code plane: this wave's tile, chunks [c0, c0 + nchunks) (a tile's
    // chunk c sits at ((tile * chunks per row + c) * 64 + lane) * 16)
    const CodeSrc csrc{W.codes + ((size_t)tile * (size_t)W.g.nchunks + (size_t)c0) * 1024u,
                       (uint32_t)nchunks * 1024u, (uint32_t)lane * 16u};

    constexpr int NB = (M + 15) / 16;  // MFMA token blocks
    constexpr int NV = M < 4 ? M : 4;  // accumulator entries holding tokens
    constexpr bool SX = MODE == kModeMfma && M <= sx_max_m<F>();  // activation sums from LDS
    f4_t macc[NB];
    float acc[M];
#pragma unroll
    for (int n = 0; n < NB; n++) macc[n] = f4_zero();
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;

    // The wave's chunks come in groups of U; the next group's loads are in
    // flight while the current group is folded.  Every wave runs the same
    // number of groups (chunks past the end are masked) so the staging
    // barriers line up.
    constexpr int U = gemv_u<F, M, MODE>();
    // chunks per phase: the LDS stage (pc columns) or the whole row, in
    // whole rounds of U chunks for each of the KS waves
    const int round = U << ks_log;
    const int pchunks = min(pc / F::CHUNK_COLS, (nchunks + round - 1) / round * round);
    const int gpp = pchunks / round;                // groups per phase per wave
    const int nph = (nchunks + pchunks - 1) / pchunks;

    // group q = ph * gpp + g: chunks ph * pchunks + (g * U + u) * KS + part.
    // Groups are visited in order; the phase of a group is tracked
    // incrementally (no division per chunk).
    // Each of the KS waves takes a contiguous quarter (half) of the phase, so
    // a group is U consecutive chunks starting at a multiple of U.
    const int pspan = pchunks >> ks_log;
    auto chunk_at = [&](int ph, int g, int u) TQ_AI { return ph * pchunks + part * pspan + g * U + u; };
    // Loop variants, as a compile-time tag: bit 0 = more than one phase,
    // bit 1 = every chunk of every group lies inside the row (EXACT kernels),
    // so no result needs a select.  The code plane is read through the
    // wave's buffer resource with the chunk index unclamped (chunks past the
    // row read zeros, without a memory access); the small scale / header
    // planes are read with ordinary loads at a chunk clamped into the row.
    auto in_row = [&](int cc) TQ_AI { return cc < nchunks ? cc : 0; };
    // stream: nontemporal code loads (each byte is read once)
    auto load_group = [&](int ph, int g, typename F::Raw (&R)[U]) TQ_AI {
        // scale cells first: their decode is the first use of the group, and
        // waiting for a load waits for every load issued before it
        if constexpr (has_sb_cell<F>()) {
            static_assert(U % GS == 0, "a chunk group holds whole scale cells");
#pragma unroll
            for (int u = 0; u < U; u += GS)
                F::template load_cell<GS>(W, off, c0 + in_row(chunk_at(ph, g, u)), R[u]);
        }
        // a group is U consecutive chunks: one resource, immediate offsets
        const int cb = chunk_at(ph, g, 0);
        const __amdgpu_buffer_rsrc_t rs = csrc.at(cb);
#pragma unroll
        for (int u = 0; u < U; u++)
            F::template load<GS, true>(W, off, c0 + in_row(cb + u), j, R[u], rs, csrc.lane, u);
        // the group's loads go out before the fold of the previous group
        __builtin_amdgcn_sched_barrier(0);
    };
    // One-round staging (fp16 activations): item e of a phase is token
    // e / nb8, columns [8 (e % nb8), +8); every load of a round is issued
    // before any is used (for phase 0 ahead of the first weights), and the
    // column sums come from the same registers (a shuffle over the lanes of
    // one sum window).  STAGE_LOCAL formats permute each item in registers;
    // the others, for one token, store the raw rows and permute them in place
    // in LDS (with more tokens their multi-phase stages measured faster with
    // the per-phase staging below).
    constexpr bool ONE = MODE != kModeF32 && (stage_local<F>() || M == 1);
    constexpr bool PERM = !stage_local<F>();
    auto phase_cols = [&](int ph, int& col0, int& ncols) TQ_AI {
        col0 = (c0 + ph * pchunks) * F::CHUNK_COLS;
        ncols = min(pchunks * F::CHUNK_COLS, colend - col0);
    };
    auto item_of = [&](int e, int nb8, int& m, int& d) TQ_AI { item_of_m<M>(e, nb8, m, d); };
    auto stage_issue = [&](int ph, int round, auto& S) TQ_AI {
        constexpr int NI = sizeof(S.v) / sizeof(uint4);
        int col0, ncols;
        phase_cols(ph, col0, ncols);
        const int nb8 = ncols >> 3;
        const _Float16* xb = (const _Float16*)P.x;
        S.live = 0;
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int e = round + k * kGemvThreads + tid;
            int m, d;
            item_of(e, nb8, m, d);
            const bool live = m < M && m < a.mcount;
            const int64_t src = live ? (int64_t)(a.m0 + m) * P.ldx + col0 + 8 * d : (int64_t)a.m0 * P.ldx + col0;
            S.v[k] = *(const uint4*)(xb + src);
            S.live |= live ? 1u << k : 0u;
        }
    };
    auto stage_commit = [&](int ph, int round, const auto& S) TQ_AI {
        constexpr int NI = sizeof(S.v) / sizeof(uint4);
        int col0, ncols;
        phase_cols(ph, col0, ncols);
        const int nb8 = ncols >> 3;
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int e = round + k * kGemvThreads + tid;
            int m, d;
            item_of(e, nb8, m, d);
            const uint4 v = (S.live >> k) & 1u ? S.v[k] : make_uint4(0, 0, 0, 0);
            if (m < M) *(uint4*)(xh + m * pc + 8 * d) = PERM ? v : stage8_raw_of<F>(v);
            if constexpr (SX || MODE == kModeDot2) {
                // SX: sums over one scale window at s16[sx_index(col / window, token)];
                // VALU fold: sums over 16 columns at s16[token * (pc / 16) + col / 16].
                // The WL items of a window are WL consecutive lanes (one DPP
                // row, or two for 32: nb8 and the rounds are multiples of WL
                // items): the window's last lane holds its sum.
                constexpr int SW = SX ? F::template sx_cols<GS>() : 16, WL = SW / 8;
                float sum = dot2(v.x, kOnes2, dot2(v.y, kOnes2, 0.0f)) + dot2(v.z, kOnes2, dot2(v.w, kOnes2, 0.0f));
                sum = row_window_sum<WL>(sum);
                if (m < M && d % WL == WL - 1) {
                    if constexpr (SX) s16[sx_index<SW>(8 * d / SW, m)] = sum;
                    else s16[m * (pc >> 4) + d / 2] = sum;
                }
            }
        }
    };
    // raw rows -> the format's staged order, in place: every window a stage8
    // reads lies inside one round, so a round's reads precede its writes
    auto stage_permute = [&](int ph) TQ_AI {
        int col0, ncols;
        phase_cols(ph, col0, ncols);
        const int nb8 = ncols >> 3;
        for (int round = 0; round < M * nb8; round += 2 * kGemvThreads) {
            uint4 o[2];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int e = round + k * kGemvThreads + tid;
                int m, d;
                item_of(e, nb8, m, d);
                o[k] = m < M ? F::stage8(xh + m * pc, 8 * d) : make_uint4(0, 0, 0, 0);
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int e = round + k * kGemvThreads + tid;
                int m, d;
                item_of(e, nb8, m, d);
                if (m < M) *(uint4*)(xh + m * pc + 8 * d) = o[k];
            }
            __syncthreads();
        }
    };
    auto stage_all = [&](int ph) TQ_AI {  // later phases: one round after another
        int col0, ncols;
        phase_cols(ph, col0, ncols);
        // (a whole 32 KiB stage is one round: every load of it is in flight
        // before the first is used; two items a round took four round trips
        // per phase, INT4 8B layer at eight tokens 39 -> 35 us)
        for (int round = 0; round < M * (ncols >> 3); round += kStageItems * kGemvThreads) {
            XStage<kStageItems> S;
            stage_issue(ph, round, S);
            stage_commit(ph, round, S);
        }
        if constexpr (PERM) {
            __syncthreads();
            stage_permute(ph);
        }
    };
    // multi_tag: whether the launch has more than one phase (only then can a
    // group of a one-round-staging launch have to stage activations)
    auto fold_group = [&](int ph, int g, const typename F::Raw (&R)[U], auto tag) TQ_AI {
        constexpr bool EX = (decltype(tag)::value & 2) != 0;  // whole groups inside the row
        if constexpr (MODE == kModeMfma) {
            // chunk u's MFMAs are issued before chunk u-1 is scaled
            const _Float16* xt[NB];
#pragma unroll
            for (int n = 0; n < NB; n++) {
                // A-operand rows of padding tokens re-read token 0: they only
                // feed accumulator rows that are never stored
                const int tok = 16 * n + r;
                xt[n] = xh + (tok < M ? tok : 0) * pc;
            }
            // Branch-free over the group (a branch per chunk would leave the
            // compiler unsure which loads have landed, and it would then drain
            // the next group's loads too): chunks past the end of the row fold
            // the staged columns of chunk 0 and are discarded by a select.
            auto lbase_of = [&](int cc) TQ_AI {
                return EX || cc < nchunks ? (cc - ph * pchunks) * F::CHUNK_COLS : 0;
            };
            auto fold_into = [&](const typename F::template Tmp<NB, GS, SX>& T, const typename F::Dec& dec,
                                 int cc, int lbase) TQ_AI {
                f4_t m2[NB];
#pragma unroll
                for (int n = 0; n < NB; n++) m2[n] = macc[n];
                F::template finish<NB, NV, GS, SX>(T, dec, s16 + 4 * (lbase >> 5), m2);
                const bool live = EX || cc < nchunks;
#pragma unroll
                for (int n = 0; n < NB; n++) macc[n] = live ? m2[n] : macc[n];
            };
            if constexpr (!F::PIPE) {
                typename F::template Tmp<NB, GS, SX> T1;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    const int cc = chunk_at(ph, g, u);
                    const int lbase = lbase_of(cc);
                    const _Float16* xu[NB];
#pragma unroll
                    for (int n = 0; n < NB; n++) xu[n] = xt[n] + lbase;
                    F::template issue<NB, GS, SX>(R[u], j, xu, T1);
                    const typename F::Dec dec = decode_u<F, GS>(W, R, u, c0 + cc, j);
                    fold_into(T1, dec, cc, lbase);
                }
            } else {
            typename F::template Tmp<NB, GS, SX> T[2];
#pragma unroll
            for (int u = 0; u <= U; u++) {
                if (u < U) {
                    const int cc = chunk_at(ph, g, u);
                    const int lbase = lbase_of(cc);
                    const _Float16* xu[NB];
#pragma unroll
                    for (int n = 0; n < NB; n++) xu[n] = xt[n] + lbase;
                    F::template issue<NB, GS, SX>(R[u], j, xu, T[u & 1]);
                }
                if (u > 0) {
                    const int cp = chunk_at(ph, g, u - 1);
                    const typename F::Dec dec = decode_u<F, GS>(W, R, u - 1, c0 + cp, j);
                    fold_into(T[(u - 1) & 1], dec, cp, lbase_of(cp));
                }
            }
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int cc = chunk_at(ph, g, u);
                if (cc >= nchunks) continue;  // uniform per wave
                const int lbase = (cc - ph * pchunks) * F::CHUNK_COLS;
                const typename F::Dec dec = decode_u<F, GS>(W, R, u, c0 + cc, j);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    if constexpr (MODE == kModeF32)
                        acc[m] += F::fold_f32(R[u], dec, j, xf + m * pc + lbase,
                                              s16 + m * (pc >> 4) + (lbase >> 4));
                    else
                        acc[m] += F::fold_h(R[u], dec, j, xh + m * pc + lbase,
                                            s16 + m * (pc >> 4) + (lbase >> 4));
                }
            }
        }
    };

    // Two register sets of weights: the next group's loads are in flight
    // while a group is folded.
    typename F::Raw rbuf[2][U];
    using kMulti = std::integral_constant<int, 1>;
    using kExact = std::integral_constant<int, 2>;
    // Group (ph, g) with g possibly one past the phase's last group: the next
    // phase's first group, or past the last phase chunks beyond the row,
    // which read zeros and fetch nothing.
    auto load_next = [&](int ph, int g, typename F::Raw (&R)[U]) TQ_AI {
        if (g >= gpp) {
            ph++;
            g -= gpp;
        }
        load_group(ph, g, R);
    };
    if constexpr (ONE) {
        // the activations' loads go out ahead of the first weights
        XStage<kStageItems> S;
        stage_issue(0, 0, S);
        load_group(0, 0, rbuf[0]);
        stage_commit(0, 0, S);
        int col0, ncols;
        phase_cols(0, col0, ncols);
        for (int round = kStageItems * kGemvThreads; round < M * (ncols >> 3);
             round += kStageItems * kGemvThreads) {
            stage_issue(0, round, S);
            stage_commit(0, round, S);
        }
        if constexpr (PERM) {
            __syncthreads();
            stage_permute(0);
        }
        __syncthreads();
    } else {
        load_group(0, 0, rbuf[0]);
    }
    // Activations of phase ph (the one-round staging has phase 0 staged
    // above); between two phases, so no fold waits on its loads or barriers.
    auto stage_phase = [&](int ph) TQ_AI {
        __syncthreads();  // the previous phase's folds are done with the stage
        if constexpr (ONE) {
            stage_all(ph);
        } else {
            const int col0 = (c0 + ph * pchunks) * F::CHUNK_COLS;
            const int ncols = min(pchunks * F::CHUNK_COLS, colend - col0);
            if constexpr (MODE == kModeF32)
                stage_f32<M>(xf, s16, pc, P.x, a.xdt, P.ldx, a.m0, a.mcount, col0, ncols, tid);
            else
                stage_f16<F, M, MODE == kModeDot2>(xh, s16, pc, P.x, P.ldx, a.m0, a.mcount, col0, ncols, tid);
            if constexpr (SX)
                stage_sums<M, F::template sx_cols<GS>()>(s16, P.x, P.ldx, a.m0, a.mcount, col0, ncols, tid);
        }
        __syncthreads();
    };
    // Main loop: phases outside, groups inside.  The inner loop holds no
    // branch with loads or barriers, so the compiler keeps the next group's
    // loads in flight under each fold (a staging branch inside it made the
    // compiler drain them before every fold).  Register set 0 holds each
    // phase's even groups: with more than one phase the host makes the group
    // count per phase even, so the next phase's first group lands in set 0.
    auto main_loop = [&](auto tag) TQ_AI {
        constexpr bool MULTI = (decltype(tag)::value & 1) != 0;
        const int nphl = MULTI ? nph : 1;
        for (int ph = 0; ph < nphl; ph++) {
            if (!ONE || ph > 0) stage_phase(ph);
            for (int g = 0; g < gpp; g += 2) {
                load_next(ph, g + 1, rbuf[1]);
                fold_group(ph, g, rbuf[0], tag);
                if (g + 1 >= gpp) break;
                load_next(ph, g + 2, rbuf[0]);
                fold_group(ph, g + 1, rbuf[1], tag);
            }
        }
    };
    if constexpr (EXACT) main_loop(kExact{});
    else main_loop(kMulti{});

    // per-lane results: MFMA lane (r, q = j) holds tokens 16n + 4j + v of row
    // r; VALU lanes hold partial sums of row r over their words.
    float res[M];
#pragma unroll
    for (int m = 0; m < M; m++) res[m] = 0.0f;
    if constexpr (MODE == kModeMfma) {
#pragma unroll
        for (int n = 0; n < NB; n++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int tok = 16 * n + 4 * j + v;
#pragma unroll
                for (int m = 0; m < M; m++)
                    if (m == tok) res[m] = macc[n][v];
            }
    } else {
#pragma unroll
        for (int m = 0; m < M; m++) res[m] = sum_slots(acc[m]);
    }
    // waves sharing a tile (KS > 1) add up through LDS: red[wave][token][row]
    if (KS > 1) {
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; m++) {
            const bool mine = MODE == kModeMfma ? (m >> 2) % 4 == j : j == 0;
            if (mine) lds[(wave * M + m) * 16 + r] = res[m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                float v = 0.0f;
                for (int w = 1; w < KS; w++) v += lds[((wave + w) * M + m) * 16 + r];
                res[m] += v;
            }
        }
    }
    if (XS > 1) {
        // K split across workgroups: publish this part's sums; the last of
        // the XS workgroups of the tile group adds the parts in order
        // (deterministic) and stores.  Every workspace access is an
        // agent-scope atomic (exchange, fetch-add, load), coherent across the
        // XCDs without the write-back and invalidation of their whole L2
        // caches that agent-scope fences cost (measured 4x slower); a part's
        // exchanges have returned (their results are consumed) before its
        // counter increment is issued.
        __shared__ unsigned last_wg, sink;
        unsigned got = 0;
        if (part == 0 && row < rows) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                const bool mine = MODE == kModeMfma ? (m >> 2) % 4 == j : j == 0;
                if (mine && m < a.mcount)
                    got ^= __hip_atomic_exchange((unsigned*)P.wsp + ((int64_t)xpart * a.mcount + m) * P.rpad + row,
                                                 __float_as_uint(res[m]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (got == 0x7FC00001u) sink = got;  // keeps the exchanges' results live
        __syncthreads();
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(P.wsc + wgt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_wg = old == XS - 1;
            // the counter goes back to zero for the next call on this workspace
            if (old == XS - 1) __hip_atomic_exchange(P.wsc + wgt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (!last_wg) return;
        if (part == 0 && row < rows) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                const bool mine = MODE == kModeMfma ? (m >> 2) % 4 == j : j == 0;
                if (mine && m < a.mcount) {
                    // every part's load is issued before the first is used
                    constexpr int XMAX = 1 << TQ_GEMV_XS_MAX_LOG;
                    unsigned pv[XMAX];
#pragma unroll
                    for (int x = 0; x < XMAX; x++)
                        pv[x] = x < XS ? __hip_atomic_load((unsigned*)P.wsp + ((int64_t)x * a.mcount + m) * P.rpad + row,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                       : 0u;
                    float v = 0.0f;
#pragma unroll
                    for (int x = 0; x < XMAX; x++) v += __uint_as_float(pv[x]);
                    res[m] = v;
                }
            }
        }
    }
    if (part == 0 && row < rows) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            const bool mine = MODE == kModeMfma ? (m >> 2) % 4 == j : j == 0;
            if (mine && m < a.mcount) {
                float v = res[m];
                if constexpr (F::FMT == TITAN_NVFP4) v *= W.gscale;
                if constexpr (F::FMT == TITAN_FP8_E4M3) v *= ((const float*)W.scales)[row];
                store_out(P.y, (int64_t)(a.m0 + m) * P.ldy + row, a.ydt, v);
            }
        }
    }
}

// ---- generic fallback for shapes the fast kernel does not take ------------------
template <int FMT, int M>
__global__ __launch_bounds__(256) void qgemv_generic_kernel(GemvArgs a) {
    __shared__ float red[M][4];
    const GemvProb& P = a.p[0];
    const WDesc& W = P.w;
    const int row = blockIdx.x;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.0f;
    for (int c = threadIdx.x; c < W.g.cols; c += 256) {
        float w = elem<FMT, TITAN_LAYOUT_REF>(W, row, c);
#pragma unroll
        for (int m = 0; m < M; m++)
            if (m < a.mcount) acc[m] += w * load_act(P.x, (int64_t)(a.m0 + m) * P.ldx + c, a.xdt);
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = wave_sum(acc[m]);
        if (lane == 0) red[m][wave] = v;
    }
    __syncthreads();
    if (threadIdx.x < a.mcount && threadIdx.x < M) {
        const int m = threadIdx.x;
        float v = red[m][0] + red[m][1] + red[m][2] + red[m][3];
        store_out(P.y, (int64_t)(a.m0 + m) * P.ldy + row, a.ydt, v);
    }
}

// ---- exact dequantization: one thread per element --------------------------------
template <int FMT, int LAYOUT>
__global__ __launch_bounds__(256) void qdequant_kernel(WDesc w, void* out, int odt) {
    const int64_t n = (int64_t)w.g.rows * w.g.cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const int row = (int)(i / w.g.cols), col = (int)(i % w.g.cols);
        store_out(out, i, odt, elem<FMT, LAYOUT>(w, row, col));
    }
}

// ============================================================================
// launchers
// ============================================================================
template <int FMT, int LAYOUT> struct Pick;
template <int L> struct Pick<TITAN_INT4, L> { using type = FxInt4<L>; };
template <int L> struct Pick<TITAN_INT2, L> { using type = FxInt2<L>; };
template <int L> struct Pick<TITAN_FP4, L> { using type = FxFp4<L>; };
template <int L> struct Pick<TITAN_NVFP4, L> { using type = FxNvfp4<L>; };
template <int L> struct Pick<TITAN_Q4_K, L> { using type = FxQ4K<L>; };
template <int L> struct Pick<TITAN_Q3_K, L> { using type = FxQ3K<L>; };
template <int L> struct Pick<TITAN_FP8_E4M3, L> { using type = FxFp8<L>; };

// Lets a kernel take up to kGemvMaxLdsBytes of dynamic LDS (above the 64 KiB
// default); setting it again is harmless.
inline void set_max_lds(const void* kern) {
    (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kGemvMaxLdsBytes);
}

template <class F, int M, int MODE>
void launch_mode(const GemvArgs& args, int, hipStream_t st) {
    GemvArgs a = args;  // this launch's split and phase choices stay local
    const int gsteps = a.p[0].gsteps;  // MFMA: word steps per scale group (same for all problems)
    // K split per problem so that every wave folds a similar number of
    // chunks (long rows are shared by 2 or 4 waves); the wave count aimed for
    // is waves_target<F, M>() (TQ_GEMV_WAVES_TARGET unless the format sets
    // its own), with at least 8 chunks per wave
    long long work = 0;
    for (int i = 0; i < a.n; i++) work += (long long)a.p[i].ntiles * a.p[i].nchunks;
    constexpr long long wt = waves_target<F, M>();
    const long long target = work / wt > 8 ? work / wt : 8;
    for (int i = 0; i < a.n; i++) {
        int ks = 0;
        while (ks < TQ_GEMV_KS_MAX && a.p[i].nchunks > target << ks) ks++;
        a.p[i].ks_log = ks;
        a.p[i].xs_log = 0;
    }
    // Few waves (small matrices): with a caller workspace, split K across
    // workgroups too.  Each wave keeps at least one whole group of U chunks;
    // the problems' waves keep one workgroup per row tile group within the K
    // split (ks = 0: four row tiles a workgroup, the smallest activation stage).
    // For the 128-column-chunk formats (INT4, Q4_K 4096^2: 8.2 -> 10.2 us)
    // the partials' round trips cost more than the extra waves gain, so they
    // keep the single-workgroup tiles.
    // The split aims for the same wave count as the in-workgroup split (the
    // smaller of TQ_GEMV_XS_WAVES and the format's target) and engages only
    // for launches of fewer waves than CUs: Q3_K 256 x 28672 one token
    // 24.0 -> 13.2 us, 128 x 8192 8.9 -> 7.2 us, INT2 256 x 8192 four tokens
    // 12.2 -> 11.2 us; at 256 to 768 waves (1024 x 8192, 4096^2) it measured
    // up to 20% slower (Q3_K 4096^2 four tokens 11.6 -> 14.1 us).
    if (a.ws && F::CHUNK_COLS > 128 && M >= xs_min_m<F>()) {
        constexpr int U = gemv_u<F, M, MODE>();
        constexpr long long xs_waves = wt < TQ_GEMV_XS_WAVES ? wt : TQ_GEMV_XS_WAVES;
        long long waves = 0;
        for (int i = 0; i < a.n; i++) waves += (long long)a.p[i].ntiles << a.p[i].ks_log;
        if (waves < 256) {
            int xs = 0;
            long long w0 = 0;
            for (int i = 0; i < a.n; i++) w0 += a.p[i].ntiles;
            auto fits = [&](int x) {
                for (int i = 0; i < a.n; i++)
                    if ((a.p[i].nchunks >> x) < U || (a.p[i].nchunks % (U << x)) != 0) return false;
                return true;
            };
            while (xs < TQ_GEMV_XS_MAX_LOG && (w0 << xs) < xs_waves && fits(xs + 1)) xs++;
            static_assert(xs_waves <= TQ_GEMV_XS_WAVES, "counter region holds TQ_GEMV_XS_WAVES tiles");
            size_t need = kGemvXsCntBytes;
            for (int i = 0; i < a.n; i++) need += gemv_xs_part_bytes(a.p[i].w.g.rows, a.mcount);
            // w0 << xs < xs_waves: fewer tiles than the counter region holds
            if (xs > 0 && (w0 << xs) > waves && need <= a.ws_bytes) {
                int tiles = 0;
                for (int i = 0; i < a.n; i++) {
                    a.p[i].wsc = (int*)a.ws + tiles;
                    tiles += a.p[i].ntiles;
                }
                char* part = (char*)a.ws + kGemvXsCntBytes;
                for (int i = 0; i < a.n; i++) {
                    GemvProb& p = a.p[i];
                    p.ks_log = 0;
                    p.xs_log = xs;
                    p.rpad = p.ntiles * 16;
                    p.wsp = (float*)part;
                    part += gemv_xs_part_bytes(p.w.g.rows, a.mcount);
                }
            }
        }
    }
    // The last round of workgroups.  Workgroup b runs on XCD b % 8 and there
    // on CU slot (b / 8) % 32 (round robin; the workgroups of these launches
    // are resident together), so with a workgroup count that is not a multiple
    // of the CU count, the last (count mod 256) workgroups are one more
    // workgroup on only some of the CUs, and those CUs finish last.  For the
    // 256-column-chunk formats the row tiles of those last workgroups get a
    // K split of four waves instead (a workgroup of one row tile), which
    // spreads them over every CU (INT2 28672 x 8192, one token: 19.7-20.2 ->
    // 18.5 us).  For INT4 / Q4_K the small workgroups' fixed costs outweigh
    // it (INT4 8B layer 22.7 -> 23.8 us).  The problem the tail begins in is
    // split at a workgroup boundary into two problems.
    if constexpr (F::CHUNK_COLS > 128) {
        constexpr int kCUs = 256;
        constexpr int U = gemv_u<F, M, MODE>();
        bool xs = false;
        for (int i = 0; i < a.n; i++) xs = xs || a.p[i].xs_log > 0;
        int ord[kGemvMaxProbs];
        for (int i = 0; i < a.n; i++) ord[i] = i;
        for (int i = 1; i < a.n; i++)  // launch order: long rows first (stable)
            for (int k2 = i; k2 > 0 && a.p[ord[k2]].nchunks > a.p[ord[k2 - 1]].nchunks; k2--) {
                int t2 = ord[k2]; ord[k2] = ord[k2 - 1]; ord[k2 - 1] = t2;
            }
        auto wgs_of = [](const GemvProb& p) {
            return (p.ntiles + (kGemvWaves >> p.ks_log) - 1) / (kGemvWaves >> p.ks_log);
        };
        long long nwg = 0;
        for (int i = 0; i < a.n; i++) nwg += wgs_of(a.p[i]);
        const int tail = (int)(nwg % kCUs);
        if (!xs && a.n < kGemvMaxProbs && nwg > kCUs && tail > 0 && tail <= kCUs / 2) {
            int left = tail;
            for (int q = a.n - 1; q >= 0 && left > 0; q--) {
                GemvProb& p = a.p[ord[q]];
                // each wave keeps at least two groups of U chunks
                const int ks2 = (p.nchunks >> TQ_GEMV_KS_MAX) >= 2 * U ? TQ_GEMV_KS_MAX : p.ks_log;
                if (ks2 <= p.ks_log) break;
                const int w = wgs_of(p);
                if (w <= left) {
                    p.ks_log = ks2;
                    left -= w;
                } else {
                    const int keep = (w - left) * (kGemvWaves >> p.ks_log);  // tiles
                    GemvProb s = p;
                    s.tile0 = p.tile0 + keep;
                    s.ntiles = p.ntiles - keep;
                    s.ks_log = ks2;
                    p.ntiles = keep;
                    a.p[a.n++] = s;
                    left = 0;
                }
            }
        }
    }
    // phase width: whole rounds of 4 waves x U = 4 chunks, at most
    // kGemvLdsBytes of staged activations (at least one round), no wider
    // than the longest row
    const int step = kGemvWaves * gemv_u<F, M, MODE>() * F::CHUNK_COLS;
    int maxcols = 0;
    for (int i = 0; i < a.n; i++) {
        const int c = a.p[i].w.g.cols >> a.p[i].xs_log;
        maxcols = maxcols > c ? maxcols : c;
    }
    // bytes per column per token, x4: fp32 + sums 17, fp16 + sums 9, fp16 8
    const int per4 = MODE == kModeF32 ? 17 : MODE == kModeDot2 ? 9 : 8;
    int cap = (kGemvLdsBytes * 4 / per4 / M) / step * step;
    if (cap < step) cap = step;
    const int need = (maxcols + step - 1) / step * step;
    a.pc = need < cap ? need : cap;
    // A problem folded in several phases needs an even number of groups per
    // phase per wave (the kernel pairs groups in two register sets across
    // phase boundaries).  A phase is a whole number of 4-wave rounds of U
    // chunks, so a K split over at most two waves always gives an even count;
    // a 4-wave split needs phases of an even number of rounds.  When the
    // launch holds few workgroups per CU the stage doubles (the K split, and
    // with it the wave count, stays); otherwise the split drops to two waves.
    auto odd_phases = [&](int pcx) {
        for (int i = 0; i < a.n; i++) {
            const GemvProb& p = a.p[i];
            const int nch = p.nchunks >> p.xs_log;
            const int rnd = gemv_u<F, M, MODE>() << p.ks_log;
            const int full = (nch + rnd - 1) / rnd * rnd;
            const int pch = pcx / F::CHUNK_COLS < full ? pcx / F::CHUNK_COLS : full;
            if ((nch + pch - 1) / pch > 1 && (pch / rnd) % 2 != 0) return true;
        }
        return false;
    };
    // Formats that fold several tokens best with at least two groups per wave
    // and phase (KS1_MULTI_PHASE): rows folded in several phases split over
    // at most two waves, while the launch keeps 1024 waves or more.  Decided
    // before the stage doubling below: two phases at two waves measured
    // faster than one doubled phase at four (INT2 8192 x 8192, four tokens).
    if constexpr (M > 1 && has_ks1_multi_phase<F>()) {
        long long waves = 0, capped = 0;
        for (int i = 0; i < a.n; i++) {
            const GemvProb& p = a.p[i];
            const bool multi = (long long)(p.nchunks >> p.xs_log) * F::CHUNK_COLS > a.pc;
            waves += (long long)p.ntiles << p.ks_log;
            capped += (long long)p.ntiles << (multi && p.ks_log > 1 ? 1 : p.ks_log);
        }
        if (capped < waves && capped >= 1024)
            for (int i = 0; i < a.n; i++) {
                GemvProb& p = a.p[i];
                if ((long long)(p.nchunks >> p.xs_log) * F::CHUNK_COLS > a.pc && p.ks_log > 1) p.ks_log = 1;
            }
    }
    if (odd_phases(a.pc) && 2 * a.pc <= need) {
        long long wgs = 0;
        for (int i = 0; i < a.n; i++)
            wgs += (long long)((a.p[i].ntiles + (kGemvWaves >> a.p[i].ks_log) - 1) /
                               (kGemvWaves >> a.p[i].ks_log)) << a.p[i].xs_log;
        const long long per_cu = (wgs + 255) / 256;
        const size_t stage2 = (size_t)M * 2 * a.pc * per4 / 4 + (MODE == kModeMfma ? a.pc : 0) + 16;
        if (stage2 <= kGemvMaxLdsBytes && (long long)stage2 * per_cu <= 160 * 1024) a.pc *= 2;
    }
    for (int i = 0; i < a.n; i++) {
        GemvProb& p = a.p[i];
        const int nch = p.nchunks >> p.xs_log;
        for (;;) {
            const int rnd = gemv_u<F, M, MODE>() << p.ks_log;
            const int full = (nch + rnd - 1) / rnd * rnd;
            const int pch = a.pc / F::CHUNK_COLS < full ? a.pc / F::CHUNK_COLS : full;
            const int nph = (nch + pch - 1) / pch;
            if (nph == 1 || (pch / rnd) % 2 == 0 || p.ks_log == 0) break;
            p.ks_log--;
        }
    }
    const size_t stage = (size_t)M * a.pc * per4 / 4 + (MODE == kModeMfma ? a.pc / 2 : 0) + 16;
    const size_t red = (size_t)kGemvWaves * M * 16 * 4;
    const size_t lds = stage > red ? stage : red;
    // workgroups: long-K problems first (they take longest)
    int order[kGemvMaxProbs];
    for (int i = 0; i < a.n; i++) order[i] = i;
    for (int i = 1; i < a.n; i++)
        for (int k2 = i; k2 > 0 && a.p[order[k2]].nchunks > a.p[order[k2 - 1]].nchunks; k2--) {
            int t = order[k2]; order[k2] = order[k2 - 1]; order[k2 - 1] = t;
        }
    GemvArgs b = a;
    for (int i = 0; i < kGemvMaxProbs; i++) b.wgb[i] = INT_MAX;
    int wg = 0;
    for (int i = 0; i < a.n; i++) {
        b.p[i] = a.p[order[i]];
        b.p[i].wg_begin = wg;
        b.wgb[i] = wg;
        wg += (b.p[i].ntiles + (kGemvWaves >> b.p[i].ks_log) - 1) / (kGemvWaves >> b.p[i].ks_log)
              << b.p[i].xs_log;
    }
    if constexpr (MODE == kModeMfma) {
        // EXACT kernel: every problem folds its chunks in one phase of whole
        // groups (the kernel's pchunks == its workgroup's chunk count)
        bool exact = allow_exact<F>();
        for (int i = 0; i < a.n; i++) {
            const int nch = a.p[i].nchunks >> a.p[i].xs_log;
            const int rnd = gemv_u<F, M, MODE>() << a.p[i].ks_log;
            const int full = (nch + rnd - 1) / rnd * rnd;
            const int pch = a.pc / F::CHUNK_COLS < full ? a.pc / F::CHUNK_COLS : full;
            exact = exact && pch == nch;
        }
        auto go = [&](auto kern) {
            if (lds > 64 * 1024) set_max_lds((const void*)kern);
            const dim3 grid = b.n == 1 ? dim3(1, wg) : dim3(wg, 1);
            hipLaunchKernelGGL(kern, grid, dim3(kGemvThreads), lds, st, b);
        };
        if constexpr (allow_exact<F>()) {
            if (exact) {
                if (gsteps == 4) go(qgemv_kernel<F, M, MODE, 4, true>);
                else if (gsteps == 2) go(qgemv_kernel<F, M, MODE, 2, true>);
                else go(qgemv_kernel<F, M, MODE, 1, true>);
                return;
            }
        }
        {
            if (gsteps == 4) go(qgemv_kernel<F, M, MODE, 4, false>);
            else if (gsteps == 2) go(qgemv_kernel<F, M, MODE, 2, false>);
            else go(qgemv_kernel<F, M, MODE, 1, false>);
        }
    } else {
        constexpr bool grouped = F::FMT == TITAN_INT4 || F::FMT == TITAN_INT2 || F::FMT == TITAN_FP4;
        auto go = [&](auto kern) {
            if (lds > 64 * 1024) set_max_lds((const void*)kern);
            const dim3 grid = b.n == 1 ? dim3(1, wg) : dim3(wg, 1);
            hipLaunchKernelGGL(kern, grid, dim3(kGemvThreads), lds, st, b);
        };
        if (grouped && gsteps == 1) go(qgemv_kernel<F, M, MODE, 1>);
        else if (grouped && gsteps == 2) go(qgemv_kernel<F, M, MODE, 2>);
        else go(qgemv_kernel<F, M, MODE, 4>);
    }
}

// Launches tokens [a.m0, a.m0 + mcount) (mcount <= 8 for the VALU modes, <= 32
// for MFMA).
template <class F>
void launch_fast(GemvArgs& a, int mcount, int mode, int total_tiles, hipStream_t st) {
    a.mcount = mcount;
    if (mode == kModeMfma) {
        if constexpr (F::HAS_MFMA) {
            if (mcount == 1) launch_mode<F, 1, kModeMfma>(a, total_tiles, st);
            else if (mcount == 2) launch_mode<F, 2, kModeMfma>(a, total_tiles, st);
            else if (mcount <= 4) launch_mode<F, 4, kModeMfma>(a, total_tiles, st);
            else if (mcount <= 8) launch_mode<F, 8, kModeMfma>(a, total_tiles, st);
            else if (mcount <= 16) launch_mode<F, 16, kModeMfma>(a, total_tiles, st);
            // 256-column chunks take at most 16 tokens a launch (run_gemv)
            else if constexpr (F::CHUNK_COLS <= 128) launch_mode<F, 32, kModeMfma>(a, total_tiles, st);
        }
    } else if (mode == kModeDot2) {
        if (mcount == 1) launch_mode<F, 1, kModeDot2>(a, total_tiles, st);
        else if (mcount == 2) launch_mode<F, 2, kModeDot2>(a, total_tiles, st);
        else if (mcount <= 4) launch_mode<F, 4, kModeDot2>(a, total_tiles, st);
        else launch_mode<F, 8, kModeDot2>(a, total_tiles, st);
    } else {
        if (mcount == 1) launch_mode<F, 1, kModeF32>(a, total_tiles, st);
        else if (mcount == 2) launch_mode<F, 2, kModeF32>(a, total_tiles, st);
        else if (mcount <= 4) launch_mode<F, 4, kModeF32>(a, total_tiles, st);
        else launch_mode<F, 8, kModeF32>(a, total_tiles, st);
    }
}

template <int FMT>
void launch_generic(GemvArgs& a, int mcount, int rows, hipStream_t st) {
    a.mcount = mcount;
    if (mcount == 1) hipLaunchKernelGGL((qgemv_generic_kernel<FMT, 1>), dim3(rows), dim3(256), 0, st, a);
    else if (mcount <= 4) hipLaunchKernelGGL((qgemv_generic_kernel<FMT, 4>), dim3(rows), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((qgemv_generic_kernel<FMT, 8>), dim3(rows), dim3(256), 0, st, a);
}

template <int FMT>
void dispatch_fmt(GemvArgs& a, int layout, int mcount, int mode, int total_tiles, hipStream_t st) {
    if (layout == TITAN_LAYOUT_TILED) {
        launch_fast<typename Pick<FMT, TITAN_LAYOUT_TILED>::type>(a, mcount, mode, total_tiles, st);
    } else {
        if constexpr (FMT != TITAN_Q3_K)
            launch_fast<typename Pick<FMT, TITAN_LAYOUT_REF>::type>(a, mcount, mode, total_tiles, st);
    }
}

template <int FMT>
bool fmt_has_mfma() { return Pick<FMT, TITAN_LAYOUT_TILED>::type::HAS_MFMA; }

}  // namespace tq

// One translation unit per format instantiates the launchers (parallel build).
namespace tq {
#define TQ_DECL(name)                                                                              \
    void dispatch_gemv_##name(GemvArgs& a, int layout, int mcount, int mode, int total_tiles,       \
                              hipStream_t st);                                                     \
    void dispatch_gemv_generic_##name(GemvArgs& a, int mcount, int rows, hipStream_t st);          \
    bool gemv_has_mfma_##name();
TQ_DECL(int4)
TQ_DECL(int2)
TQ_DECL(fp4)
TQ_DECL(nvfp4)
TQ_DECL(q4k)
TQ_DECL(q3k)
TQ_DECL(fp8)
#undef TQ_DECL
}  // namespace tq
