// fp8_gemm.hip -- FP8 (OCP E4M3) prefill GEMM on gfx950 MFMA.
//
// out[m][n] = (sum_k A[m][k] * W[n][k]) * sa[m] * sw[n]
//   A  : e4m3 activations [M][K] with fp32 per-token scale sa (from
//        titan_fp8_quantize_rows)
//   W  : e4m3 weights [N][K] with fp32 per-output-channel scale sw
// The reference has only an unscaled, unlaunched FP8 matvec
// (dequant.cu:179-221); this GEMM is the north-star prefill path.
//
// Block tile BM x BN (256 x 256, 256 x 128 or 128 x 128), 4 waves in a 2 x 2
// grid, each wave a (BM/2) x (BN/2) tile of v_mfma_scale_f32_32x32x64_f8f6f4
// (unit E8M0 scales) with its fp32 accumulators in AGPRs.  K advances 64
// bytes per stage; both operand tiles of a stage go global -> LDS by
// direct-to-LDS 16-byte loads (no VGPR staging) into four stage buffers, so
// three stages of loads are in flight under the matrix-core work.
//
// LDS layout of an operand stage: [16-row block][row][4 slots of 16 B], the
// 64 K-bytes of a row in swizzled slot order.  One wave load instruction
// fills one 16-row KiB block (64 contiguous global bytes per row); one
// ds_read_b128 gives every lane half of its MFMA fragment, conflict-free.
// The k order inside a fragment is a permutation of the hardware's, the
// same for both operands, so every product term still meets its partner.
//
// Workgroups are mapped XCD-aware: the hardware sends workgroup i to XCD
// i % 8, so consecutive tiles of the (grouped) tile order are handed to the
// same XCD and share its L2.
#include "common.h"

namespace tq {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

#ifndef TQ_F8_M128
#define TQ_F8_M128 2  // 256x128 tiles: waves along M (8 waves)
#endif
#ifndef TQ_F8_WGN
#define TQ_F8_WGN 4  // waves along N for the 256-row tiles (8 waves per workgroup)
#endif
constexpr int kF8BK = 64;     // K bytes per pipeline stage
constexpr int kF8Stages = 4;  // LDS stage buffers (up to 3 stages of loads in flight)

TQ_DEV v16f mfma_fp8_32(const v8i& a, const v8i& b, v16f c) {
    // cbsz = blgp = 0: both operands FP8 E4M3; scale 127 = 2^0 (E8M0)
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// One 16-byte-per-lane direct-to-LDS load: lane l's 16 bytes from `src` land
// at LDS byte offset (dst + 16 l).  Issued as inline assembly so that the
// compiler's wait-count insertion does not order every later LDS read behind
// it (it cannot tell which stage buffer the load writes); the kernel waits
// for these loads itself with s_waitcnt vmcnt before the barrier that
// publishes a stage.
TQ_DEV void lds_dma16(const uint8_t* src, uint8_t* dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)dst;
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

// Workgroup barrier without the memory fence of __syncthreads (which would
// wait for every outstanding load, including the stages still in flight).
TQ_DEV void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// s_waitcnt immediate waiting for vmcnt <= n only (gfx9 encoding).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Epilogue through LDS: a 32x32 C fragment gives a lane one column
// (lane & 31) of rows 8 (v / 4) + 4 (lane / 32) + v % 4 (A rows are M, B rows
// are N).  Each wave scales and converts 32-row bands of its WM x WN tile
// (rows mw.., columns nw..) into its own LDS region, then writes whole rows
// with 16-byte stores.  The caller has synchronised the workgroup.
template <int WM, int WN, int TI, int TJ, int ODT>
TQ_DEV void fp8_epilogue(uint8_t* sm, const v16f (&acc)[TI][TJ], int mw, int nw, int wave, int lane,
                         const float* __restrict__ sa, const float* __restrict__ sw,
                         void* __restrict__ out, int N) {
    constexpr int OSZ = ODT == TITAN_FP32 ? 4 : 2;
    constexpr int RB = WN * OSZ + 16;      // LDS bytes per band row (padded)
    constexpr int PR = WN * OSZ / 16;      // 16-byte pieces per row
    uint8_t* ep = sm + wave * 32 * RB;
    float sn[TJ];
#pragma unroll
    for (int jn = 0; jn < TJ; jn++) sn[jn] = sw[nw + 32 * jn + (lane & 31)];
#pragma unroll
    for (int i = 0; i < TI; i++) {
        const int mb = mw + 32 * i;  // first row of the band
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int ml = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            const float sm_ = sa[mb + ml];
#pragma unroll
            for (int jn = 0; jn < TJ; jn++) {
                const float val = acc[i][jn][v] * sm_ * sn[jn];
                uint8_t* dst = ep + ml * RB + (32 * jn + (lane & 31)) * OSZ;
                if constexpr (ODT == TITAN_FP32) *(float*)dst = val;
                else if constexpr (ODT == TITAN_FP16) *(uint16_t*)dst = f32_to_f16_rne(val);
                else *(uint16_t*)dst = f32_to_bf16_rne(val);
            }
        }
        // LDS operations of one wave complete in order: the band is readable
        const int row = lane >> 1;
        uint8_t* gout = (uint8_t*)out + ((int64_t)(mb + row) * N + nw) * OSZ;
#pragma unroll
        for (int p = 0; p < PR / 2; p++) {
            const int piece = (lane & 1) * (PR / 2) + p;
            *(uint4*)(gout + piece * 16) = *(const uint4*)(ep + row * RB + piece * 16);
        }
    }
}
template <int WN, int ODT>
constexpr int fp8_epilogue_lds(int nwaves) { return nwaves * 32 * (WN * (ODT == TITAN_FP32 ? 4 : 2) + 16); }

template <int BM, int BN, int WGM, int WGN, int ODT>
__global__ __launch_bounds__(64 * WGM * WGN) void fp8_gemm_kernel(const uint8_t* __restrict__ A,
                                                          const float* __restrict__ sa,
                                                          const uint8_t* __restrict__ W,
                                                          const float* __restrict__ sw,
                                                          void* __restrict__ out, int M, int N,
                                                          int K) {
    constexpr int NW = WGM * WGN;  // waves: WGM along M x WGN along N
    constexpr int WM = BM / WGM, WN = BN / WGN, TI = WM / 32, TJ = WN / 32;
    static_assert(TJ >= 1, "wave tile");
    constexpr int ABYTES = BM * kF8BK, BBYTES = BN * kF8BK, SBYTES = ABYTES + BBYTES;
    constexpr int ABLK = BM / 16, BBLK = BN / 16;  // 16-row KiB blocks per stage
    constexpr int LPW = (ABLK + BBLK) / NW;                // load instructions per wave per stage
    constexpr int S = kF8Stages;
    static_assert((ABLK + BBLK) % NW == 0, "loads split over the waves");
    extern __shared__ __attribute__((aligned(1024))) uint8_t sm[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // ---- tile order: XCD chunks, then groups of 8 tile rows (m fastest)
    const int ntm = M / BM, ntn = N / BN, ntiles = ntm * ntn;
    int t = blockIdx.x;
    if (ntiles % 8 == 0) t = (t % 8) * (ntiles / 8) + t / 8;
    constexpr int GROUP = 8;
    const int per_group = GROUP * ntn, g = t / per_group, first_m = g * GROUP;
    const int gsize = min(ntm - first_m, GROUP);
    const int tm = first_m + (t % per_group) % gsize, tn = (t % per_group) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    // ---- direct-to-LDS loads: uniform (scalar) row-block base + one per-lane
    // 32-bit offset (row lane % 32 of the block, 16 bytes at 16 (lane / 32))
    // DMA lane l fills row l / 4 of a 16-row block, 16-byte slot l % 4, with
    // chunk (l % 4) ^ swz(row) of the row's 64 bytes (a full 64-byte segment
    // per row); swz(row) = (row / 4) % 4 makes the fragment reads below
    // conflict-free.
    const int drow = lane >> 2, dchunk = (lane & 3) ^ ((drow >> 2) & 3);
    const uint32_t loff = (uint32_t)drow * (uint32_t)K + 16u * (uint32_t)dchunk;
    const uint8_t* ta = A + (size_t)m0 * K;
    const uint8_t* tb = W + (size_t)n0 * K;
    auto issue = [&](int kt) {
        uint8_t* st = sm + (kt % S) * SBYTES;
        const int k0 = kt * kF8BK;
#pragma unroll
        for (int q = 0; q < LPW; q++) {
            const int blk = q * NW + wave;  // 16-row KiB block of the stage, A blocks first
            const bool isa = blk < ABLK;
            const int b2 = isa ? blk : blk - ABLK;
            const uint8_t* base = (isa ? ta : tb) + (size_t)(b2 * 16) * K + k0;
            lds_dma16(base + loff, st + (isa ? 0 : ABYTES) + b2 * 1024);
        }
    };
    // fragment of a 32-row block: lane l takes row r = l % 32, chunks
    // 2 p + l / 32 for pieces p = 0, 1 (the same k order for both operands)
    const int fr = lane & 31, frr = fr & 15, fkq = lane >> 5;
    const uint32_t fbase = (uint32_t)((fr >> 4) * 1024 + frr * 64);
    const uint32_t fo0 = fbase + (uint32_t)(((0 + fkq) ^ ((frr >> 2) & 3)) << 4);
    const uint32_t fo1 = fbase + (uint32_t)(((2 + fkq) ^ ((frr >> 2) & 3)) << 4);
    auto frag = [&](const uint8_t* blk2) {
        const uint4 x0 = *(const uint4*)(blk2 + fo0);
        const uint4 x1 = *(const uint4*)(blk2 + fo1);
        return (v8i){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                     (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    };

    v16f acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int jn = 0; jn < TJ; jn++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][jn][v] = 0.0f;

    const int nk = K / kF8BK;
    // Iteration kt: stage kt's fragments are in registers.  It publishes
    // stage kt + 1, refills stage kt's (already read) buffer with stage
    // kt + S, and reads stage kt + 1's fragments while stage kt's
    // matrix-core instructions run -- so after each barrier the matrix cores
    // restart at once, with no LDS latency in front of them.
    if constexpr (TJ <= 2) {
        // two waves per SIMD: every fragment of stage kt + 1 is read while
        // stage kt's matrix-core instructions run; stage kt's buffer is
        // refilled with stage kt + S as soon as the barrier has passed
        v8i fa[2][TI], fb[2][TJ];  // ping-pong fragment sets (indices fold to registers)
        auto read_frags = [&](int kt, v8i* a, v8i* b) {
            const uint8_t* st = sm + (kt % S) * SBYTES;
#pragma unroll
            for (int jn = 0; jn < TJ; jn++) b[jn] = frag(st + ABYTES + (wn * TJ + jn) * 2048);
#pragma unroll
            for (int i = 0; i < TI; i++) a[i] = frag(st + (wm * TI + i) * 2048);
        };
#pragma unroll
        for (int kt = 0; kt < S; kt++)
            if (kt < nk) issue(kt);
        // stage 0 landed: at most stages 1 .. min(S, nk) - 1 outstanding
        if (nk >= S) __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 1) * LPW));
        else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        wg_barrier();
        read_frags(0, fa[0], fb[0]);
        for (int k2 = 0; k2 < nk; k2 += 2) {
#pragma unroll
            for (int ph = 0; ph < 2; ph++) {
                const int kt = k2 + ph;
                if (kt >= nk) break;
                // stages issued after kt + 1: kt + 2 .. min(kt + S - 1, nk - 1)
                if (kt + S - 1 < nk) __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * LPW));
                else if (kt + S - 2 < nk) __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 3) * LPW));
                else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
                wg_barrier();  // stage kt + 1 landed everywhere; stage kt's buffer is free
                if (kt + S < nk) issue(kt + S);
                // past the last stage this reads a stale buffer; the values are unused
                read_frags(kt + 1, fa[ph ^ 1], fb[ph ^ 1]);
#pragma unroll
                for (int jn = 0; jn < TJ; jn++) {
#pragma unroll
                    for (int i = 0; i < TI; i++)
                        acc[i][jn] = mfma_fp8_32(fa[ph][i], fb[ph][jn], acc[i][jn]);
                }
            }
        }
    } else {
        // one wave per SIMD (large wave tile, fewer LDS reads): this stage's
        // B fragments stream one ahead of their matrix-core instructions and
        // the next stage's A fragments and first B fragment are read under
        // the last ones; stage kt - 1's buffer is refilled with stage kt + S - 1
        v8i fa[TI], fan[TI], fb, fbn;
        auto read_a = [&](int kt, v8i* a) {
            const uint8_t* st = sm + (kt % S) * SBYTES;
#pragma unroll
            for (int i = 0; i < TI; i++) a[i] = frag(st + (wm * TI + i) * 2048);
        };
        auto b_at = [&](int kt, int jn) { return sm + (kt % S) * SBYTES + ABYTES + (wn * TJ + jn) * 2048; };
#pragma unroll
        for (int kt = 0; kt < S - 1; kt++)
            if (kt < nk) issue(kt);
        // stage 0 landed: at most stages 1 .. min(S - 1, nk) - 1 outstanding
        if (nk >= S - 1) __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * LPW));
        else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        wg_barrier();
        read_a(0, fa);
        fb = frag(b_at(0, 0));
        for (int kt = 0; kt < nk; kt++) {
            // stages issued after kt + 1: kt + 2 .. min(kt + S - 2, nk - 1)
            if (kt + S - 2 < nk) __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 3) * LPW));
            else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
            wg_barrier();  // stage kt + 1 landed everywhere; stage kt - 1's buffer is free
            if (kt + S - 1 < nk) issue(kt + S - 1);
#pragma unroll
            for (int jn = 0; jn < TJ; jn++) {
                if (jn + 1 < TJ) {
                    fbn = frag(b_at(kt, jn + 1));
                } else {  // past the last stage: a stale buffer, values unused
                    read_a(kt + 1, fan);
                    fbn = frag(b_at(kt + 1, 0));
                }
#pragma unroll
                for (int i = 0; i < TI; i++) acc[i][jn] = mfma_fp8_32(fa[i], fb, acc[i][jn]);
                fb = fbn;
            }
#pragma unroll
            for (int i = 0; i < TI; i++) fa[i] = fan[i];
        }
    }

    static_assert(fp8_epilogue_lds<WN, ODT>(NW) <= kF8Stages * (BM + BN) * kF8BK, "epilogue fits in LDS");
    __syncthreads();  // every wave is done with the stage buffers
    fp8_epilogue<WM, WN, TI, TJ, ODT>(sm, acc, m0 + wm * WM, n0 + wn * WN, wave, lane, sa, sw, out, N);
}

template <int BM, int BN, int WGM, int WGN, int ODT>
int launch_fp8_t(const uint8_t* A, const float* sa, const uint8_t* W, const float* sw, void* out,
                 int M, int N, int K, hipStream_t stream) {
    constexpr int lds = kF8Stages * (BM + BN) * kF8BK;
    static bool attr_set = false;  // per kernel; setting it twice is harmless
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)fp8_gemm_kernel<BM, BN, WGM, WGN, ODT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return TITAN_ERR_LAUNCH;
        attr_set = true;
    }
    const int ntiles = (M / BM) * (N / BN);
    hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, WGM, WGN, ODT>), dim3(ntiles), dim3(64 * WGM * WGN), lds, stream, A, sa,
                       W, sw, out, M, N, K);
    return tqh::launch_status();
}

template <int BM, int BN, int WGM, int WGN>
int launch_fp8(const uint8_t* A, const float* sa, const uint8_t* W, const float* sw, void* out,
               int odt, int M, int N, int K, hipStream_t stream) {
    switch (odt) {
        case TITAN_FP32: return launch_fp8_t<BM, BN, WGM, WGN, TITAN_FP32>(A, sa, W, sw, out, M, N, K, stream);
        case TITAN_FP16: return launch_fp8_t<BM, BN, WGM, WGN, TITAN_FP16>(A, sa, W, sw, out, M, N, K, stream);
        default: return launch_fp8_t<BM, BN, WGM, WGN, TITAN_BF16>(A, sa, W, sw, out, M, N, K, stream);
    }
}

}  // namespace tq

extern "C" int titan_fp8_gemm(const uint8_t* A, const float* sa, const uint8_t* W, const float* sw,
                              void* out, int out_dtype, int M, int N, int K, hipStream_t stream) {
    if (!A || !sa || !W || !sw || !out || M <= 0 || N <= 0 || K <= 0 ||
        !tqh::act_dtype_ok(out_dtype))
        return TITAN_ERR_INVALID_ARG;
    if (M % 128 || N % 128 || K % tq::kF8BK || ((uintptr_t)A & 15) || ((uintptr_t)W & 15))
        return TITAN_ERR_UNSUPPORTED;
    if ((int64_t)M * K >= (1ll << 31) || (int64_t)N * K >= (1ll << 31)) return TITAN_ERR_UNSUPPORTED;
    // the largest tile that still gives every CU a tile
    if (M % 256 == 0 && N % 256 == 0 && (int64_t)(M / 256) * (N / 256) >= 256)
        return tq::launch_fp8<256, 256, 2, TQ_F8_WGN>(A, sa, W, sw, out, out_dtype, M, N, K, stream);
    if (M % 256 == 0 && (int64_t)(M / 256) * (N / 128) >= 256)
        return tq::launch_fp8<256, 128, TQ_F8_M128, 8 / TQ_F8_M128>(A, sa, W, sw, out, out_dtype, M, N, K, stream);
    return tq::launch_fp8<128, 128, 2, 2>(A, sa, W, sw, out, out_dtype, M, N, K, stream);
}
