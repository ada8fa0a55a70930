// moe_gemm.hip -- NVFP4 grouped-expert MoE forward on gfx950.
//
// Restates the reference's expert loop (moe.cpp:874-1005): for every token and
// each of its k selected experts, g = Wg x and u = Wu x with the NVFP4 dequant
// of fp4.cu:187-252, a = silu(g) * u (activation.cu:17-32), y = Wd a, then the
// weighted combine into the residual (activation.cu:111-139).  Instead of
// 3 GEMV launches per (token, expert) it runs four launches for all tokens:
//
//   1. permute   group the (token, slot) pairs by expert (counting sort)
//   2. gate/up   per (expert, 64-row block): both projections of all of the
//                expert's tokens in one pass over the weights, SwiGLU fused,
//                activations written as fp16 rows in expert order
//   3. down      per (expert, 64-row block), fp32 rows in expert order
//   4. combine   per token: residual + sum_j w_j y_j (+ shared), in slot order
//
// GEMM kernel: one wave owns a 16-row tile of the weights (TILED NVFP4 layout)
// and runs v_mfma_f32_16x16x32_f16 with the tokens as A (staged per K-slab in
// LDS as fp16) and the weights as B.  A lane's code word holds 8 consecutive
// columns of one 16-column scale block, so its B operand is
//   cvt_scalef32_pk_f16_fp4(word, 2^8) * (e4m3 scale as fp16 * 2^-8)
// -- four conversions and four packed multiplies per 8 weights, all exact
// (E2M1 x E4M3 products have at most 5 significant bits and stay inside the
// fp16 normal range); the fp32 global scale multiplies the accumulator.
#include "common.h"
#include "layout.h"
#include "xitem.h"


namespace tq {

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
typedef float mf4 __attribute__((ext_vector_type(4)));

constexpr int kMoeThreads = 256;
constexpr int kMoeRowsPerWg = 64;  // 4 waves x 16 rows
constexpr int kMoeMaxExperts = 4096;

struct MoeGemmArgs {
    const titan_nvfp4_expert* experts;  // device array [E]
    const void* x;                      // activation rows
    int64_t ldx;                        // elements between activation rows
    const int* pair_at;                 // gate/up: position -> pair id; down: nullptr
    int k;                              // experts per token (pair id / k = token)
    const int* off;                     // [E + 1] first position of each expert
    int N, K;                           // weight rows / columns
    void* out;                          // gate/up: fp16 [P][N]; down: fp32 [P][N]
    int64_t ldo;
};

// A lane's four E4M3 block scales -- bytes jj and 2 + jj of both 32-bit
// halves of its 8-byte chunk scale word (sel gathers them) -- as fp16 of
// value * 2^-8, two per register: the hardware conversion with a 2^-8 scale
// (exact: E4M3 * 2^-8 is an fp16 normal or subnormal), then the E4M3 NaNs
// 0x7F / 0xFF, which fp4.cu:173-185 reads as 0, cleared: every finite scale
// * 2^-8 is below 2, so only a NaN half has exponent bit 14 set.
TQ_DEV uint32_t clear_nan_halves(uint32_t h) {
    const uint32_t t = (h & 0x40004000u) >> 14;
    return h & ~__umul24(t, 0xFFFFu);
}
TQ_DEV void e4m3x4_scaled(uint2 sv, uint32_t sel, mh2& s01, mh2& s23) {
    const uint32_t g = __builtin_amdgcn_perm(sv.y, sv.x, sel);
    const uint32_t a = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(g, 0.00390625f, false));
    const uint32_t b = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(g, 0.00390625f, true));
    s01 = __builtin_bit_cast(mh2, clear_nan_halves(a));
    s23 = __builtin_bit_cast(mh2, clear_nan_halves(b));
}

// 8 fp4 codes of one word (low nibble first) times one scale -> B operand.
TQ_DEV mh8 nvfp4_b8(uint32_t w, _Float16 sc) {
    const mh2 s = {sc, sc};
    const mh2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 256.0f, 0) * s;
    const mh2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 256.0f, 1) * s;
    const mh2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 256.0f, 2) * s;
    const mh2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 256.0f, 3) * s;
    return mh8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// TM tokens per pass, SL columns per LDS slab, RT 16-row tiles per wave (a
// workgroup covers 64 RT rows and stages the tokens' activations once for
// all of them).  GATED: gate and up together with the SwiGLU epilogue;
// otherwise one matrix, fp32 rows out.
template <int TM, int SL, int RT, bool GATED, int XDT>
__global__ __launch_bounds__(kMoeThreads) __attribute__((amdgpu_waves_per_eu(2))) void moe_gemm_kernel(MoeGemmArgs a) {
    constexpr int NB = TM / 16;         // MFMA token blocks
    constexpr int CPS = SL / 128;       // 64-byte chunks per slab
    constexpr int LDR = SL + 8;         // halves per LDS row (16 B pad)
    constexpr int NI = TM * SL / 8 / kMoeThreads;
    constexpr int NM = GATED ? 2 : 1;
    static_assert(NI >= 1 && TM * SL == NI * 8 * kMoeThreads, "staging geometry");
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][TM * LDR];

    const int e = blockIdx.y;
    const int beg = a.off[e], n_e = a.off[e + 1] - beg;
    if (n_e <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane >> 4, r = lane & 15;
    const titan_nvfp4_expert ex = a.experts[e];
    const uint8_t* W[2] = {(const uint8_t*)(GATED ? ex.gate : ex.down), (const uint8_t*)ex.up};
    const float gsc[2] = {GATED ? ex.gate_scale : ex.down_scale, ex.up_scale};
    const Geo geo = make_geo(TITAN_NVFP4, a.N, a.K, 16);
    // tile q of this wave: rows [row0(q), row0(q) + 16)
    auto row0 = [&](int q) { return blockIdx.x * (kMoeRowsPerWg * RT) + q * kMoeRowsPerWg + wave * 16; };
    uint32_t code_off[RT], sc_off[RT];
#pragma unroll
    for (int q = 0; q < RT; q++) {
        code_off[q] = (uint32_t)tiled_code_off(geo, row0(q) + r, 0, j);
        sc_off[q] = (uint32_t)tiled_nvs_off(geo, row0(q) + r, 0);
    }
    const int nslab = a.K / SL;
    // bytes of the lane's scales in its chunk scale word (see e4m3x4_scaled)
    const uint32_t jj = (uint32_t)(j >> 1);
    const uint32_t ssel = jj | ((2 + jj) << 8) | ((4 + jj) << 16) | ((6 + jj) << 24);

    for (int t0 = 0; t0 < n_e; t0 += TM) {
        const int nt = min(TM, n_e - t0), nb = (nt + 15) >> 4;
        // staging sources: item it covers row rr, columns [8 cg, 8 cg + 8) of the slab
        int64_t src[NI];
        int ldsi[NI];
#pragma unroll
        for (int it = 0; it < NI; it++) {
            const int idx = it * kMoeThreads + tid, rr = idx / (SL / 8), cg = idx % (SL / 8);
            ldsi[it] = rr * LDR + cg * 8;
            int64_t srow = -1;
            if (rr < nt) srow = a.pair_at ? a.pair_at[beg + t0 + rr] / a.k : beg + t0 + rr;
            src[it] = srow < 0 ? -1 : srow * a.ldx + cg * 8;
        }
        auto load_x = [&](int s, XItem<XDT>* xr) {
#pragma unroll
            for (int it = 0; it < NI; it++) {
                if (src[it] >= 0) xr[it].load(a.x, src[it] + (int64_t)s * SL);
                else xr[it].zero();
            }
        };
        struct WSet { uint4 c[NM][RT][CPS]; uint2 s[NM][RT][CPS]; };
        auto load_w = [&](int s, WSet& w) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int q = 0; q < RT; q++)
#pragma unroll
                    for (int c = 0; c < CPS; c++) {
                        const uint32_t ch = (uint32_t)(s * CPS + c);
                        w.c[m][q][c] = ld_stream_u128(W[m] + code_off[q] + ch * 1024u);
                        w.s[m][q][c] = *(const uint2*)(W[m] + sc_off[q] + ch * 128u);
                    }
        };

        mf4 acc[NM][RT][NB];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int q = 0; q < RT; q++)
#pragma unroll
                for (int b = 0; b < NB; b++) acc[m][q][b] = mf4{0, 0, 0, 0};

        // Software pipeline over K slabs: weights two slabs ahead in three
        // register sets (no copies), activations one slab ahead.  Issue order
        // per slab -- activations, then weights -- lets the wait for the
        // activations of slab s leave the weights of slabs s+1, s+2 in flight.
        XItem<XDT> xr[NI];
        WSet w0, w1, w2;
        load_x(0, xr);
        load_w(0, w0);
        if (nslab > 1) load_w(1, w1);
        auto step = [&](int s, const WSet& wc, WSet& wnext2) {
            _Float16* buf = xs[s & 1];
#pragma unroll
            for (int it = 0; it < NI; it++) *(uint4*)(buf + ldsi[it]) = xr[it].h();
            if (s + 1 < nslab) load_x(s + 1, xr);
            if (s + 2 < nslab) load_w(s + 2, wnext2);
            __syncthreads();
#pragma unroll
            for (int c = 0; c < CPS; c++) {
                mh2 scw[NM][RT][2];  // word i's scale: half i % 2 of scw[.][.][i / 2]
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int q = 0; q < RT; q++) e4m3x4_scaled(wc.s[m][q][c], ssel, scw[m][q][0], scw[m][q][1]);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    mh8 B[NM][RT];
#pragma unroll
                    for (int m = 0; m < NM; m++)
#pragma unroll
                        for (int q = 0; q < RT; q++) {
                            const uint4 cw = wc.c[m][q][c];
                            const uint32_t w = i == 0 ? cw.x : i == 1 ? cw.y : i == 2 ? cw.z : cw.w;
                            B[m][q] = nvfp4_b8(w, scw[m][q][i >> 1][i & 1]);
                        }
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        if (b < nb) {
                            const mh8 A = *(const mh8*)(buf + (b * 16 + r) * LDR + c * 128 + 32 * i + 8 * j);
#pragma unroll
                            for (int m = 0; m < NM; m++)
#pragma unroll
                                for (int q = 0; q < RT; q++)
                                    acc[m][q][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                        A, B[m][q], acc[m][q][b], 0, 0, 0);
                        }
                    }
                }
            }
        };
        for (int s = 0; s < nslab; s += 3) {
            step(s, w0, w2);
            if (s + 1 < nslab) step(s + 1, w1, w0);
            if (s + 2 < nslab) step(s + 2, w2, w1);
        }

        // epilogue: lane holds weight row row0(q) + r for tokens 16 b + 4 j + v
#pragma unroll
        for (int q = 0; q < RT; q++) {
            const int row = row0(q) + r;
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (b >= nb) break;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int tok = b * 16 + 4 * j + v;
                    if (tok >= nt) continue;
                    const int64_t o = (int64_t)(beg + t0 + tok) * a.ldo + row;
                    if constexpr (GATED) {
                        const float g = acc[0][q][b][v] * gsc[0], u = acc[1][q][b][v] * gsc[1];
                        const float act = (g * (1.0f / (1.0f + expf(-g)))) * u;
                        ((_Float16*)a.out)[o] = (_Float16)act;
                    } else {
                        ((float*)a.out)[o] = acc[0][q][b][v] * gsc[0];
                    }
                }
            }
        }
        __syncthreads();  // the next token pass rewrites both LDS buffers
    }
}

// bf16 / fp32 activations -> fp16 once, 8 elements per thread (every
// workgroup of every selected expert stages these rows again).
template <int XDT>
__global__ __launch_bounds__(256) void to_f16_kernel(const void* __restrict__ x, int64_t n8,
                                                     _Float16* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    XItem<XDT> v;
    v.load(x, i * 8);
    *(uint4*)(out + i * 8) = v.h();
}

// Counting sort of the (token, slot) pairs by expert.  One workgroup; the
// order of pairs inside an expert is irrelevant to the results (each token is
// its own row of the GEMMs and the combine reads positions through `inv`).
__global__ __launch_bounds__(1024) void moe_permute_kernel(const int* __restrict__ idx, int P,
                                                           int E, int* __restrict__ off,
                                                           int* __restrict__ pair_at,
                                                           int* __restrict__ inv) {
    __shared__ int cnt[kMoeMaxExperts];
    __shared__ int part[1024];
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = idx[p];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scan: thread t owns experts [4t, 4t + 4)
    int loc[4], s = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = 4 * tid + q;
        loc[q] = s;
        s += e < E ? cnt[e] : 0;
    }
    part[tid] = s;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int v = tid >= d ? part[tid - d] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    const int base = part[tid] - s;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int e = 4 * tid + q;
        if (e < E) {
            off[e] = base + loc[q];
            cnt[e] = base + loc[q];
        }
    }
    if (tid == 1023) off[E] = part[1023];
    __syncthreads();
    for (int p = tid; p < P; p += 1024) {
        const int e = idx[p];
        if (e >= 0 && e < E) {
            const int pos = atomicAdd(&cnt[e], 1);
            pair_at[pos] = p;
            inv[p] = pos;
        } else {
            inv[p] = -1;
        }
    }
}

// activation.cu:111-139 per token: c = sum_j y_j * w_j (fused multiply-add in
// slot order), + shared * w_s, out = residual + c.
__global__ __launch_bounds__(256) void moe_combine_rows_kernel(
    const float* __restrict__ y, const int* __restrict__ inv, const float* __restrict__ w,
    int k, int dim, const float* __restrict__ residual, const float* __restrict__ shared,
    float sw, void* __restrict__ out, int out_dtype) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= dim) return;
    float c = 0.0f;
    for (int q = 0; q < k; q++) {
        const int pos = inv[(int64_t)t * k + q];
        if (pos >= 0) c = __builtin_fmaf(y[(int64_t)pos * dim + i], w[(int64_t)t * k + q], c);
    }
    if (shared) c = __builtin_fmaf(shared[(int64_t)t * dim + i], sw, c);
    const float v = (residual ? residual[(int64_t)t * dim + i] : 0.0f) + c;
    store_out(out, (int64_t)t * dim + i, out_dtype, v);
}

// The same with four consecutive elements per thread (dim % 4 == 0, 16-byte
// aligned rows): one 16-byte load per expert row.
__global__ __launch_bounds__(256) void moe_combine_rows4_kernel(
    const float* __restrict__ y, const int* __restrict__ inv, const float* __restrict__ w,
    int k, int dim, const float* __restrict__ residual, const float* __restrict__ shared,
    float sw, void* __restrict__ out, int out_dtype) {
    const int t = blockIdx.y, i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= dim) return;
    float4 c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int q = 0; q < k; q++) {
        const int pos = inv[(int64_t)t * k + q];
        if (pos >= 0) {
            const float wq = w[(int64_t)t * k + q];
            const float4 v = *(const float4*)(y + (int64_t)pos * dim + i);
            c.x = __builtin_fmaf(v.x, wq, c.x);
            c.y = __builtin_fmaf(v.y, wq, c.y);
            c.z = __builtin_fmaf(v.z, wq, c.z);
            c.w = __builtin_fmaf(v.w, wq, c.w);
        }
    }
    if (shared) {
        const float4 v = *(const float4*)(shared + (int64_t)t * dim + i);
        c.x = __builtin_fmaf(v.x, sw, c.x);
        c.y = __builtin_fmaf(v.y, sw, c.y);
        c.z = __builtin_fmaf(v.z, sw, c.z);
        c.w = __builtin_fmaf(v.w, sw, c.w);
    }
    float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (residual) r = *(const float4*)(residual + (int64_t)t * dim + i);
    const int64_t o = (int64_t)t * dim + i;
    store_out(out, o, out_dtype, r.x + c.x);
    store_out(out, o + 1, out_dtype, r.y + c.y);
    store_out(out, o + 2, out_dtype, r.z + c.z);
    store_out(out, o + 3, out_dtype, r.w + c.w);
}

}  // namespace tq

namespace {

using namespace tq;

struct MoeWs {
    int* off;
    int* pair_at;
    int* inv;
    _Float16* act;
    float* y;
    _Float16* xh;  // the tokens' activations as fp16 (bf16 / fp32 input)
    size_t bytes;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

MoeWs carve(void* base, int tokens, int k, int E, int hidden, int inter) {
    const size_t P = (size_t)tokens * k;
    MoeWs w;
    size_t o = 0;
    auto take = [&](size_t n) { size_t at = o; o = align256(o + n); return at; };
    const size_t o_off = take((size_t)(E + 1) * 4), o_pair = take(P * 4), o_inv = take(P * 4),
                 o_act = take(P * inter * 2), o_y = take(P * hidden * 4),
                 o_xh = take((size_t)tokens * hidden * 2);
    char* b = (char*)base;
    w.off = (int*)(b + o_off);
    w.pair_at = (int*)(b + o_pair);
    w.inv = (int*)(b + o_inv);
    w.act = (_Float16*)(b + o_act);
    w.y = (float*)(b + o_y);
    w.xh = (_Float16*)(b + o_xh);
    w.bytes = o;
    return w;
}

template <int TM, int SL, int RT, bool GATED>
int launch_moe(const MoeGemmArgs& a, int x_dtype, int E, hipStream_t st) {
    if (a.N % (kMoeRowsPerWg * RT)) return TITAN_ERR_UNSUPPORTED;
    dim3 grid(a.N / (kMoeRowsPerWg * RT), E);
    // Activations always arrive as fp16: the forward converts other types once.
    if (x_dtype != TITAN_FP16) return TITAN_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((moe_gemm_kernel<TM, SL, RT, GATED, TITAN_FP16>), grid, dim3(kMoeThreads), 0,
                       st, a);
    return tqh::launch_status();
}

// Tokens per pass from the mean load per expert; more rows per workgroup as
// the token tile grows, so that the activation staging stays small next to
// the weight stream.
// (tokens per pass, LDS slab columns, row tiles per wave) per token tile
#ifndef TQ_MOE_G16
#define TQ_MOE_G16 16, 128, 2
#endif
#ifndef TQ_MOE_D16
#define TQ_MOE_D16 16, 128, 2
#endif
#ifndef TQ_MOE_G32
#define TQ_MOE_G32 32, 128, 2
#endif
#ifndef TQ_MOE_D32
#define TQ_MOE_D32 32, 128, 2
#endif
#ifndef TQ_MOE_G48
#define TQ_MOE_G48 48, 128, 2
#endif
#ifndef TQ_MOE_D48
#define TQ_MOE_D48 48, 128, 4
#endif
#ifndef TQ_MOE_G64
#define TQ_MOE_G64 64, 128, 2
#endif
#ifndef TQ_MOE_D64
#define TQ_MOE_D64 64, 128, 4
#endif
#ifndef TQ_MOE_T32
#define TQ_MOE_T32 8   // mean tokens per expert above which 32-token passes are used
#endif
#ifndef TQ_MOE_T48
#define TQ_MOE_T48 24  // ... 48-token passes
#endif
#ifndef TQ_MOE_T64
#define TQ_MOE_T64 40  // ... and 64-token passes
#endif

template <bool GATED>
int launch_moe_tm(int tm, const MoeGemmArgs& a, int x_dtype, int E, hipStream_t st) {
    if constexpr (GATED) {
        if (tm == 16) return launch_moe<TQ_MOE_G16, true>(a, x_dtype, E, st);
        if (tm == 32) return launch_moe<TQ_MOE_G32, true>(a, x_dtype, E, st);
        if (tm == 48) return launch_moe<TQ_MOE_G48, true>(a, x_dtype, E, st);
        return launch_moe<TQ_MOE_G64, true>(a, x_dtype, E, st);
    } else {
        if (tm == 16) return launch_moe<TQ_MOE_D16, false>(a, x_dtype, E, st);
        if (tm == 32) return launch_moe<TQ_MOE_D32, false>(a, x_dtype, E, st);
        if (tm == 48) return launch_moe<TQ_MOE_D48, false>(a, x_dtype, E, st);
        return launch_moe<TQ_MOE_D64, false>(a, x_dtype, E, st);
    }
}

}  // namespace

extern "C" size_t titan_moe_nvfp4_workspace_bytes(int tokens, int k, int num_experts, int hidden,
                                                 int inter) {
    if (tokens <= 0 || k <= 0 || num_experts <= 0 || hidden <= 0 || inter <= 0) return 0;
    return carve(nullptr, tokens, k, num_experts, hidden, inter).bytes;
}

extern "C" int titan_moe_nvfp4_forward(const titan_nvfp4_expert* experts, int num_experts,
                                       int hidden, int inter, const void* x, int x_dtype,
                                       int tokens, const int* indices, const float* weights,
                                       int k, const float* residual, const float* shared,
                                       float shared_weight, void* out, int out_dtype,
                                       void* workspace, size_t workspace_bytes,
                                       hipStream_t stream) {
    if (!experts || !x || !indices || !weights || !out || !workspace) return TITAN_ERR_INVALID_ARG;
    if (tokens <= 0 || k <= 0 || num_experts <= 0 || num_experts > kMoeMaxExperts)
        return TITAN_ERR_INVALID_ARG;
    if (!tqh::act_dtype_ok(x_dtype) || !tqh::act_dtype_ok(out_dtype)) return TITAN_ERR_INVALID_ARG;
    // shapes: 64-row blocks of both projections, 512-column K slabs, tileable NVFP4
    if (hidden % 512 || inter % 512) return TITAN_ERR_UNSUPPORTED;
    if ((int64_t)tokens * k > (1 << 30)) return TITAN_ERR_UNSUPPORTED;
    if (!tq::tiled_total_bytes(TITAN_NVFP4, inter, hidden, 16) ||
        !tq::tiled_total_bytes(TITAN_NVFP4, hidden, inter, 16))
        return TITAN_ERR_UNSUPPORTED;
    if (((uintptr_t)x & 15) || ((uintptr_t)workspace & 255)) return TITAN_ERR_INVALID_ARG;
    const MoeWs ws = carve(workspace, tokens, k, num_experts, hidden, inter);
    if (workspace_bytes < ws.bytes) return TITAN_ERR_WORKSPACE;

    const int P = tokens * k;
    hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(1024), 0, stream, indices, P,
                       num_experts, ws.off, ws.pair_at, ws.inv);
    if (int st = tqh::launch_status()) return st;

    // tokens per pass from the mean load per expert
    const int avg = (P + num_experts - 1) / num_experts;
    const int tm = avg <= TQ_MOE_T32 ? 16 : avg <= TQ_MOE_T48 ? 32 : avg <= TQ_MOE_T64 ? 48 : 64;

    MoeGemmArgs g{};
    g.experts = experts;
    g.x = x;
    int gx_dtype = x_dtype;
    if (x_dtype != TITAN_FP16) {
        const int64_t n8 = (int64_t)tokens * hidden / 8;
        const dim3 grid((unsigned)((n8 + 255) / 256));
        if (x_dtype == TITAN_BF16)
            hipLaunchKernelGGL(to_f16_kernel<TITAN_BF16>, grid, dim3(256), 0, stream, x, n8, ws.xh);
        else
            hipLaunchKernelGGL(to_f16_kernel<TITAN_FP32>, grid, dim3(256), 0, stream, x, n8, ws.xh);
        if (int st = tqh::launch_status()) return st;
        g.x = ws.xh;
        gx_dtype = TITAN_FP16;
    }
    g.ldx = hidden;
    g.pair_at = ws.pair_at;
    g.k = k;
    g.off = ws.off;
    g.N = inter;
    g.K = hidden;
    g.out = ws.act;
    g.ldo = inter;
    if (int st = launch_moe_tm<true>(tm, g, gx_dtype, num_experts, stream)) return st;

    MoeGemmArgs d{};
    d.experts = experts;
    d.x = ws.act;
    d.ldx = inter;
    d.pair_at = nullptr;
    d.k = k;
    d.off = ws.off;
    d.N = hidden;
    d.K = inter;
    d.out = ws.y;
    d.ldo = hidden;
    if (int st = launch_moe_tm<false>(tm, d, TITAN_FP16, num_experts, stream)) return st;

    const bool vec = hidden % 4 == 0 && ((uintptr_t)residual & 15) == 0 && ((uintptr_t)shared & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(moe_combine_rows4_kernel, dim3((hidden / 4 + 255) / 256, tokens), dim3(256), 0,
                           stream, ws.y, ws.inv, weights, k, hidden, residual, shared, shared_weight,
                           out, out_dtype);
    else
        hipLaunchKernelGGL(moe_combine_rows_kernel, dim3((hidden + 255) / 256, tokens), dim3(256), 0,
                           stream, ws.y, ws.inv, weights, k, hidden, residual, shared, shared_weight,
                           out, out_dtype);
    return tqh::launch_status();
}
