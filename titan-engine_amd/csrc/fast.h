// fast.h -- the GEMV/small-M GEMM view of each weight format.
//
// A wave covers 16 rows x one 64-byte chunk of codes per row.  Lane
// l = 16*j + r (r = row in the tile, j = 0..3) holds words j, 4+j, 8+j, 12+j
// of row r's chunk: word i of the lane covers chunk bytes [16i + 4j, +4), so
// the four lanes of a row together cover chunk bytes [16i, 16i + 16) at "word
// step" i -- a run of contiguous columns inside one scale group.
//
// Three ways to fold a chunk against activations (all fp32 accumulation):
//  * fold_f32  (fp32 / bf16 activations): codes to fp32, FMA with fp32 x held
//    in natural column order in LDS.
//  * fold_h    (fp16 activations): a code word masked to bits inside the fp16
//    mantissa is a pair of exact fp16 subnormals (code * 2^-24 * 2^shift);
//    v_dot2_f32_f16 multiplies it with an activation pair.  Activations sit
//    in LDS permuted per format (stage8) so one 128-bit read yields the
//    pairs that line up with the masked code pairs.
//  * issue / finish (fp16 activations, selected formats): the same fp16 code
//    operands feed v_mfma_f32_16x16x{16,32}_f16 with activations as the A
//    operand (16 tokens x k) and codes as B (k x 16 rows); lane (r, q) of the
//    accumulator holds row r, tokens 4q..4q+3, so the lane's own per-row
//    scales apply without data movement.  Bias / min terms use the sum of x
//    over the group, taken by an extra MFMA against a vector of ones.
// fold_f32 / fold_h return the lane's partial dot product for one token; the
// four lanes of a row are summed afterwards.  Bias-like terms (scale *
// sum(x over the group)) are added by lane j == 0 only, with the group's full
// activation sum from the per-16-column sums staged in LDS.
#pragma once

#include "formats.h"

namespace tq {

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// ---- fp16 helpers -------------------------------------------------------------
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
TQ_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
TQ_DEV float dot2(uint32_t codes, uint32_t x2, float acc) {
    return __builtin_amdgcn_fdot2(as_h2(codes), as_h2(x2), acc, false);
}
constexpr float kTwo24 = 16777216.0f;  // 2^24
constexpr float kTwo14 = 16384.0f;     // 2^14
constexpr uint32_t kOnes2 = 0x3C003C00u;  // fp16 pair (1, 1)

TQ_DEV h4_t h4_of(uint32_t a, uint32_t b) { return __builtin_bit_cast(h4_t, make_uint2(a, b)); }
TQ_DEV h8_t h8_of(uint4 v) { return __builtin_bit_cast(h8_t, v); }
TQ_DEV f4_t mfma16(h4_t a, h4_t b, f4_t c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
TQ_DEV f4_t mfma32(h8_t a, h8_t b, f4_t c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
TQ_DEV f4_t f4_zero() { return (f4_t){0.f, 0.f, 0.f, 0.f}; }

// Code-plane source of one wave (tiled layouts): the 1 KiB chunks of the
// wave's row tile that its workgroup folds (base, bytes) and the lane's
// 16-byte offset inside a chunk.  at(c) is a buffer resource starting at
// chunk c; reads at or past the end of the range return zeros without a
// memory access (the hardware's range check), so the loads a wave issues
// past its last group cost no bandwidth.
struct CodeSrc {
    const uint8_t* base;
    uint32_t bytes;
    uint32_t lane;
    TQ_DEV __amdgpu_buffer_rsrc_t at(int c) const {
        const uint32_t o = (uint32_t)c * 1024u;
        // signed max (a scalar instruction; an unsigned saturating subtraction
        // would be a vector one and make the resource a per-lane value);
        // a tile's chunk range is far below 2^31 bytes
        const int d = (int)bytes - (int)o;
        const uint32_t n = (uint32_t)(d > 0 ? d : 0);
        // 0x00020000: raw buffer, 32-bit data format (word 3 of the descriptor)
        return __builtin_amdgcn_make_buffer_rsrc((void*)(base + o), (short)0, (int)n, 0x00020000);
    }
};
// Chunk u of a group whose first chunk `rs` starts at (nontemporal: cache
// policy 2); the chunk offset is an immediate of the instruction.
template <bool NT>
TQ_DEV uint4 ld_code_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t lane, int u) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane + (uint32_t)u * 1024u, 0,
                                                                           NT ? 2 : 0));
}

// E2M1 codes of a word as fp16 pairs (value = lut * 2^-14): nibbles n and
// n + 4 of word w become the low / high halves of fp4_pair(w, n).
TQ_DEV uint32_t fp4_pair(uint32_t w, int n) {
    switch (n) {  // magnitude bits (e1 e0 m) -> fp16 bits 11..9, sign -> bit 15
        case 0: return ((w & 0x00070007u) << 9) | ((w & 0x00080008u) << 12);
        case 1: return ((w & 0x00700070u) << 5) | ((w & 0x00800080u) << 8);
        case 2: return ((w & 0x07000700u) << 1) | ((w & 0x08000800u) << 4);
        default: return ((w >> 3) & 0x0E000E00u) | (w & 0x80008000u);
    }
}

// fp32 dot product of 8 nibbles (column n in bits 4n) with x[0..7]
TQ_DEV float dot_nib8(uint32_t w, const float* x) {
    uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    float a = (float)(lo & 0xFF) * x[0];
    float b = (float)(hi & 0xFF) * x[1];
    a = __builtin_fmaf((float)((lo >> 8) & 0xFF), x[2], a);
    b = __builtin_fmaf((float)((hi >> 8) & 0xFF), x[3], b);
    a = __builtin_fmaf((float)((lo >> 16) & 0xFF), x[4], a);
    b = __builtin_fmaf((float)((hi >> 16) & 0xFF), x[5], b);
    a = __builtin_fmaf((float)(lo >> 24), x[6], a);
    b = __builtin_fmaf((float)(hi >> 24), x[7], b);
    return a + b;
}
TQ_DEV void ld_f8(const float* p, float* x) {
    float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
TQ_DEV void ld_f4(const float* p, float* x) {
    float4 a = *(const float4*)p;
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
}

// Group index of a column: the fast path only takes power-of-two groups.
TQ_DEV int group_of(const WDesc& w, int col) { return col >> w.gshift; }

// Staging helpers: 8 / 4 fp16 activations from a natural-order row.
TQ_DEV void ldh8(const _Float16* p, _Float16* h) {
    uint4 v = *(const uint4*)p;
    h8_t t = h8_of(v);
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = t[i];
}
TQ_DEV void ldh4(const _Float16* p, _Float16* h) {
    uint2 v = *(const uint2*)p;
    h4_t t = __builtin_bit_cast(h4_t, v);
#pragma unroll
    for (int i = 0; i < 4; i++) h[i] = t[i];
}
TQ_DEV uint4 pack8(const _Float16* o) {
    h8_t t;
#pragma unroll
    for (int i = 0; i < 8; i++) t[i] = o[i];
    return __builtin_bit_cast(uint4, t);
}

// ============================================================================
// INT4 affine (dequant.cu:23-104): word (4i+j) = columns 32i + 8j + n of the
// chunk (nibble n).  Word step i lies in group (128c + 32i) >> gshift.
// LDS activation order: per 8 columns [0,4,2,6,1,5,3,7].
// ============================================================================
template <int LAYOUT, bool IS_FP4 = false>
struct FxNib {
    static constexpr int FMT = IS_FP4 ? TITAN_FP4 : TITAN_INT4;
    static constexpr int CHUNK_COLS = 128;
    static constexpr bool HAS_MFMA = !IS_FP4, PIPE = true;
    // one token: 1536 waves aimed for (the 8B layer's 14336-column rows split
    // over two waves, not four): 22.6 -> 21.2 us on the layer; FP4 14336 x
    // 4096 13.4 -> 12.3 us (4096 x 14336 unchanged; several tokens measured
    // slower with it)
    static constexpr long long WAVES_TARGET_M1 = 1536;
    // FP4, five to eight tokens: groups of two chunks (4096 x 14336 53.3 ->
    // 49.9 us, 14336 x 4096 unchanged; one to four tokens gain on one shape
    // and lose on the other); INT4 never (U2_MIN_M above every token count:
    // its scale cells span four chunks)
    static constexpr int U2_MIN_M = IS_FP4 ? 8 : 64, U2_MAX_M = 8;
    // tiled INT4: the scales come in 16-byte cells, one load per GS chunks
    static constexpr bool SB_CELL = LAYOUT == TITAN_LAYOUT_TILED && !IS_FP4;
    struct Off { uint32_t c, s, b; };
    struct Raw { uint32_t w[4], s[4], b[4]; uint4 q; };
    struct Dec { float s[4], b[4]; };
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        const Geo& g = w.g;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            return {(uint32_t)row * (uint32_t)g.row_code_bytes + 4u * j,
                    (uint32_t)row * (uint32_t)(g.ngroups * 2), (uint32_t)row * (uint32_t)(g.ngroups * 2)};
        else if constexpr (IS_FP4)
            return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_fp4s_off(g, row, 0), 0u};
        else
            return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_sb_off(g, row, 0), 0u};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
#pragma unroll
            for (int i = 0; i < 4; i++) r.w[i] = ld_u32(w.codes + (o.c + (uint32_t)c * 64u + 16u * i));
        } else {
            uint4 q = ld_code_chunk<NT>(rs, lane, u);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        }
        if constexpr (SB_CELL) return;  // load_cell
#pragma unroll
        for (int i = GS - 1; i < 4; i += GS) {  // last word step of each group
            const uint32_t grp = (uint32_t)group_of(w, c * 128 + 32 * i);
            if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
                r.s[i] = ld_u16(w.scales + (o.s + grp * 2u));
                if constexpr (!IS_FP4) r.b[i] = ld_u16(w.biases + (o.b + grp * 2u));
            } else if constexpr (IS_FP4) {
                r.s[i] = ld_u16(w.codes + (o.s + grp * 32u));
            } else {
                r.s[i] = ld_u32(w.codes + (o.s + grp * 64u));
            }
        }
    }
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        Dec d;  // step i takes the scales loaded for the last step of its group
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = i | (GS - 1);
            if constexpr (LAYOUT == TITAN_LAYOUT_TILED && !IS_FP4) {
                d.s[i] = f16_to_f32(r.s[k] & 0xFFFF);
                d.b[i] = f16_to_f32(r.s[k] >> 16);
            } else {
                d.s[i] = f16_to_f32(r.s[k]);
                d.b[i] = IS_FP4 ? 0.0f : f16_to_f32(r.b[k]);
            }
        }
        return d;
    }
    // Scale cells (tiled INT4 / INT2): chunk c's groups sit in cell c / GS at
    // entries (c % GS) * (4 / GS) + (step / GS); the cell is loaded with the
    // first chunk of its GS chunks (the caller's chunk groups start at
    // multiples of 4).
    template <int GS>
    TQ_DEV static void load_cell(const WDesc& w, const Off& o, int c, Raw& r) {
        r.q = ld_u128((w.codes + (size_t)(((uint32_t)c / GS) * 256u)) + o.s);
    }
    template <int GS>
    TQ_DEV static Dec decode_cell(const uint4& q, int u) {
        const uint32_t e[4] = {q.x, q.y, q.z, q.w};
        Dec d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = e[(u % GS) * (4 / GS) + i / GS];
            d.s[i] = f16_to_f32(v & 0xFFFF);
            d.b[i] = f16_to_f32(v >> 16);
        }
        return d;
    }
    // bias: lane j == 0 adds b * sum(x) over the 32 columns of each step
    TQ_DEV static float bias(const Dec& d, const float* s16) {
        float t = 0.0f;
        if constexpr (!IS_FP4) {
#pragma unroll
            for (int i = 0; i < 4; i++) t = __builtin_fmaf(d.b[i], s16[2 * i] + s16[2 * i + 1], t);
        }
        return t;
    }
    TQ_DEV static float fold_f32(const Raw& r, const Dec& d, int j, const float* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x[8];
            ld_f8(xc + 32 * i + 8 * j, x);
            if constexpr (IS_FP4) {
                float a = 0.0f, b = 0.0f;
#pragma unroll
                for (int n = 0; n < 8; n += 2) {
                    a = __builtin_fmaf(fp4_to_f32((r.w[i] >> (4 * n)) & 0xF), x[n], a);
                    b = __builtin_fmaf(fp4_to_f32((r.w[i] >> (4 * n + 4)) & 0xF), x[n + 1], b);
                }
                t = __builtin_fmaf(d.s[i], a + b, t);
            } else {
                t = __builtin_fmaf(d.s[i], dot_nib8(r.w[i], x), t);
            }
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec& d, int j, const _Float16* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xv = *(const uint4*)(xc + 32 * i + 8 * j);
            const uint32_t w = r.w[i];
            if constexpr (IS_FP4) {
                float a = dot2(fp4_pair(w, 0), xv.x, 0.0f);
                float b = dot2(fp4_pair(w, 2), xv.y, 0.0f);
                a = dot2(fp4_pair(w, 1), xv.z, a);
                b = dot2(fp4_pair(w, 3), xv.w, b);
                t = __builtin_fmaf(d.s[i], (a + b) * kTwo14, t);
            } else {
                const uint32_t u = w >> 8;
                float lo = dot2(w & 0x000F000Fu, xv.x, 0.0f);  // (n0, n4)
                lo = dot2(u & 0x000F000Fu, xv.y, lo);          // (n2, n6)
                // (n1, n5) / (n3, n7) enter x16 against activations staged / 16
                float hi = dot2(w & 0x00F000F0u, xv.z, 0.0f);
                hi = dot2(u & 0x00F000F0u, xv.w, hi);
                t = __builtin_fmaf(d.s[i], (lo + hi) * kTwo24, t);
            }
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    // MFMA: per step one 16x16x32 for sum(q*x) and one against ones for
    // sum(x); folded into acc at the end of each group.
    // MFMA, two stages so that a chunk's MFMAs are in flight while the
    // previous chunk is scaled: issue() runs the MFMAs of every scale group
    // of the chunk (codes low / high nibble, and the activation sums against
    // ones unless SX), finish() applies the per-row scales.  SX: sum(x) per
    // 32 columns comes from LDS instead (M <= 4: only accumulator entries of
    // lanes q = 0 hold tokens).
    template <int NB, int GS, bool SX>
    struct Tmp { f4_t C[4 / GS][NB], O[SX ? 1 : 4 / GS][NB]; };
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw& r, int j, const _Float16* const* xt, Tmp<NB, GS, SX>& T) {
        // staged activations of a step: columns (0,4,2,6) and (1,5,3,7) / 16, so
        // the ones vector weighs the second half by 16 for sum(x)
        const h8_t ones = h8_of(make_uint4(kOnes2, kOnes2, 0x4C004C00u, 0x4C004C00u));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = i / GS;
            const uint32_t w = r.w[i], u = w >> 8;
            // (n0, n4, n2, n6) and 16 x (n1, n5, n3, n7), exact fp16 subnormals
            const h8_t b = h8_of(make_uint4(w & 0x000F000Fu, u & 0x000F000Fu, w & 0x00F000F0u, u & 0x00F000F0u));
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const h8_t xv = h8_of(*(const uint4*)(xt[n] + 32 * i + 8 * j));
                const bool first = i % GS == 0;
                T.C[g][n] = mfma32(xv, b, first ? f4_zero() : T.C[g][n]);
                if constexpr (!SX) T.O[g][n] = mfma32(xv, ones, first ? f4_zero() : T.O[g][n]);
            }
        }
    }
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>& T, const Dec& d, const float* sx, f4_t* acc) {
#pragma unroll
        for (int g = 0; g < 4 / GS; g++) {
            const int i = g * GS;
            const float s = d.s[i] * kTwo24, bb = d.b[i];
            float4 xs;
            if constexpr (SX) xs = *(const float4*)(sx + 4 * i);  // the group's column sums
#pragma unroll
            for (int n = 0; n < NB; n++)
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const float t = __builtin_fmaf(s, T.C[g][n][v], acc[n][v]);
                    const float o = SX ? (v == 0 ? xs.x : v == 1 ? xs.y : v == 2 ? xs.z : xs.w)
                                       : T.O[SX ? 0 : g][n][v];
                    acc[n][v] = __builtin_fmaf(bb, o, t);
                }
        }
    }
    // 8 staged activations starting at chunk column d0 (d0 % 8 == 0)
    // INT4 (matrix cores): the odd columns are pre-divided by 16 to meet their
    // codes, which enter 16x too large (exact for |x| >= 2^-10; below that the
    // quotient is an fp16 subnormal, off by at most 2^-25)
    static constexpr bool STAGE_LOCAL = true;  // stage8 reads only columns d0..d0+7
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) { return stage8_raw(*(const uint4*)(xr + d0)); }
    TQ_DEV static uint4 stage8_raw(uint4 raw) {
        _Float16 h[8], o[8];
        const h8_t t = h8_of(raw);
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = t[i];
        const _Float16 k = IS_FP4 ? (_Float16)1.0f : (_Float16)0.0625f;
        o[0] = h[0]; o[1] = h[4]; o[2] = h[2]; o[3] = h[6];
        o[4] = h[1] * k; o[5] = h[5] * k; o[6] = h[3] * k; o[7] = h[7] * k;
        return pack8(o);
    }
    TQ_DEV static int steps_per_group(const WDesc& w) { return w.g.gs >= 128 ? 4 : w.g.gs / 32; }
    // columns summed per activation-sum entry (SX): one scale group
    template <int GS> static constexpr int sx_cols() { return 32 * GS; }
};
template <int L> using FxInt4 = FxNib<L, false>;
template <int L> using FxFp4 = FxNib<L, true>;

// ============================================================================
// INT2 affine (dequant.cu:110-172): word (4i+j) = columns 64i + 16j + n of
// the chunk (code n in bits 2n); groups >= 64 columns.  The field at bits 2k
// of the two 16-bit halves holds codes (k, k+8); masked in place (k <= 4) or
// after one shift by 6 (k = 5..7) it is an exact fp16 subnormal times 4^k (or
// 4^(k-3)), and the staged activations are divided by the same power of two.
// ============================================================================
template <int LAYOUT>
struct FxInt2 {
    static constexpr int FMT = TITAN_INT2, CHUNK_COLS = 256;
    static constexpr bool HAS_MFMA = true, PIPE = true;
    // several tokens: fewer, longer waves than the default 2048 measured 22%
    // faster on 28672x8192 at four tokens (42.6 -> 33.2 us), the other shapes
    // unchanged; one token keeps 2048 (28672x8192 1.5% slower with 1536)
    static constexpr long long WAVES_TARGET = 1536, WAVES_TARGET_M1 = 2048;
    // several tokens, rows in several activation phases: at most two waves a
    // row tile (8192 x 28672 at four tokens 47.6-49.3 -> 45.2 us, 8192 x 8192
    // 17.4 -> 16.1 us; one token and small launches keep the wider split)
    static constexpr bool KS1_MULTI_PHASE = true;
    // the cross-workgroup K split from two tokens on: at one token it
    // measured no faster (128-512 x 8192: 6.6 -> 6.6-6.9 us)
    static constexpr int XS_MIN_M = 2;
    static constexpr bool SB_CELL = LAYOUT == TITAN_LAYOUT_TILED;
    struct Off { uint32_t c, s, b; };
    struct Raw { uint32_t w[4], s[4], b[4]; uint4 q; };
    struct Dec { float s[4], b[4]; };
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        const Geo& g = w.g;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            return {(uint32_t)row * (uint32_t)g.row_code_bytes + 4u * j,
                    (uint32_t)row * (uint32_t)(g.ngroups * 2), (uint32_t)row * (uint32_t)(g.ngroups * 2)};
        else
            return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_sb_off(g, row, 0), 0u};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
#pragma unroll
            for (int i = 0; i < 4; i++) r.w[i] = ld_u32(w.codes + (o.c + (uint32_t)c * 64u + 16u * i));
        } else {
            uint4 q = ld_code_chunk<NT>(rs, lane, u);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        }
        if constexpr (SB_CELL) return;  // load_cell
#pragma unroll
        for (int i = GS - 1; i < 4; i += GS) {  // last word step of each group
            const uint32_t grp = (uint32_t)group_of(w, c * 256 + 64 * i);
            if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
                r.s[i] = ld_u16(w.scales + (o.s + grp * 2u));
                r.b[i] = ld_u16(w.biases + (o.b + grp * 2u));
            } else {
                r.s[i] = ld_u32(w.codes + (o.s + grp * 64u));
            }
        }
    }
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        Dec d;  // step i takes the scales loaded for the last step of its group
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = i | (GS - 1);
            if constexpr (LAYOUT == TITAN_LAYOUT_TILED) {
                d.s[i] = f16_to_f32(r.s[k] & 0xFFFF);
                d.b[i] = f16_to_f32(r.s[k] >> 16);
            } else {
                d.s[i] = f16_to_f32(r.s[k]);
                d.b[i] = f16_to_f32(r.b[k]);
            }
        }
        return d;
    }
    // Scale cells (tiled INT4 / INT2): chunk c's groups sit in cell c / GS at
    // entries (c % GS) * (4 / GS) + (step / GS); the cell is loaded with the
    // first chunk of its GS chunks (the caller's chunk groups start at
    // multiples of 4).
    template <int GS>
    TQ_DEV static void load_cell(const WDesc& w, const Off& o, int c, Raw& r) {
        r.q = ld_u128(w.codes + (o.s + ((uint32_t)c / GS) * 256u));
    }
    template <int GS>
    TQ_DEV static Dec decode_cell(const uint4& q, int u) {
        const uint32_t e[4] = {q.x, q.y, q.z, q.w};
        Dec d;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = e[(u % GS) * (4 / GS) + i / GS];
            d.s[i] = f16_to_f32(v & 0xFFFF);
            d.b[i] = f16_to_f32(v >> 16);
        }
        return d;
    }
    TQ_DEV static float bias(const Dec& d, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
            t = __builtin_fmaf(d.b[i], (s16[4 * i] + s16[4 * i + 1]) + (s16[4 * i + 2] + s16[4 * i + 3]), t);
        return t;
    }
    TQ_DEV static float fold_f32(const Raw& r, const Dec& d, int j, const float* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x[16];
            ld_f8(xc + 64 * i + 16 * j, x);
            ld_f8(xc + 64 * i + 16 * j + 8, x + 8);
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const uint32_t v = (r.w[i] >> (2 * s)) & 0x03030303u;  // codes s, s+4, s+8, s+12
                a = __builtin_fmaf((float)(v & 0xFF), x[s], a);
                b = __builtin_fmaf((float)((v >> 8) & 0xFF), x[s + 4], b);
                a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[s + 8], a);
                b = __builtin_fmaf((float)(v >> 24), x[s + 12], b);
            }
            t = __builtin_fmaf(d.s[i], a + b, t);
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec& d, int j, const _Float16* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xa = *(const uint4*)(xc + 64 * i + 16 * j);
            const uint4 xb = *(const uint4*)(xc + 64 * i + 16 * j + 8);
            const uint32_t w = r.w[i], u = w >> 6;
            // fields in place (x 4^k), activations staged / 4^k: one scale
            float s0 = dot2(w & 0x00030003u, xa.x, 0.0f);  // (0, 8)
            float s1 = dot2(w & 0x000C000Cu, xa.y, 0.0f);  // (1, 9)
            s0 = dot2(w & 0x00300030u, xa.z, s0);          // (2, 10)
            s1 = dot2(w & 0x00C000C0u, xa.w, s1);          // (3, 11)
            s0 = dot2(w & 0x03000300u, xb.x, s0);          // (4, 12)
            s1 = dot2(u & 0x00300030u, xb.y, s1);          // (5, 13)
            s0 = dot2(u & 0x00C000C0u, xb.z, s0);          // (6, 14)
            s1 = dot2(u & 0x03000300u, xb.w, s1);          // (7, 15)
            const float v = (s0 + s1) * kTwo24;
            t = __builtin_fmaf(d.s[i], v, t);
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    template <int NB, int GS, bool SX>
    struct Tmp { f4_t C[4 / GS][NB], O[SX ? 1 : 4 / GS][NB]; };
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw& r, int j, const _Float16* const* xt, Tmp<NB, GS, SX>& T) {
        // the staged activations are divided by the field weights 4^k: the
        // ones vectors weigh them back for sum(x)
        const h8_t ones_a = h8_of(make_uint4(0x3C003C00u, 0x44004400u, 0x4C004C00u, 0x54005400u));
        const h8_t ones_b = h8_of(make_uint4(0x5C005C00u, 0x4C004C00u, 0x54005400u, 0x5C005C00u));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = i / GS;
            const uint32_t w = r.w[i], u = w >> 6;
            // fields 0..4 of each 16-bit half in place (exact subnormals x 4^k),
            // fields 5..7 after one shift: 9 operations for 16 codes
            const h8_t b0 = h8_of(make_uint4(w & 0x00030003u, w & 0x000C000Cu, w & 0x00300030u,
                                             w & 0x00C000C0u));
            const h8_t b1 = h8_of(make_uint4(w & 0x03000300u, u & 0x00300030u, u & 0x00C000C0u,
                                             u & 0x03000300u));
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const _Float16* p = xt[n] + 64 * i + 16 * j;
                const uint4 xa = *(const uint4*)p, xb = *(const uint4*)(p + 8);
                const bool first = i % GS == 0;
                T.C[g][n] = mfma32(h8_of(xa), b0, first ? f4_zero() : T.C[g][n]);
                T.C[g][n] = mfma32(h8_of(xb), b1, T.C[g][n]);
                if constexpr (!SX) {
                    T.O[g][n] = mfma32(h8_of(xa), ones_a, first ? f4_zero() : T.O[g][n]);
                    T.O[g][n] = mfma32(h8_of(xb), ones_b, T.O[g][n]);
                }
            }
        }
    }
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>& T, const Dec& d, const float* sx, f4_t* acc) {
#pragma unroll
        for (int g = 0; g < 4 / GS; g++) {
            const int i = g * GS;
            const float s = d.s[i] * kTwo24, bb = d.b[i];
            float4 xs;  // the group's column sums (a word step is 64 columns)
            if constexpr (SX) xs = *(const float4*)(sx + 4 * (2 * i));
#pragma unroll
            for (int n = 0; n < NB; n++)
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    const float t = __builtin_fmaf(s, T.C[g][n][v], acc[n][v]);
                    const float o = SX ? (v == 0 ? xs.x : v == 1 ? xs.y : v == 2 ? xs.z : xs.w)
                                       : T.O[SX ? 0 : g][n][v];
                    acc[n][v] = __builtin_fmaf(bb, o, t);
                }
        }
    }
    // 16 staged columns: d0 % 16 == 0 gives [0,8,1,9,2,10,3,11] / [1,1,4,4,16,16,64,64],
    // == 8 gives [4,12,5,13,6,14,7,15] / [256,256,16,16,64,64,256,256] -- the
    // field weights of the codes they meet (division by a power of two is
    // exact unless the quotient falls below 2^-14, where it is off by < 2^-25)
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) {
        const int u = d0 & ~15;
        _Float16 a[8], b[8], o[8];
        ldh8(xr + u, a);
        ldh8(xr + u + 8, b);
        if ((d0 & 8) == 0) {
            o[0] = a[0]; o[1] = b[0];
            o[2] = a[1] * (_Float16)0.25f; o[3] = b[1] * (_Float16)0.25f;
            o[4] = a[2] * (_Float16)0.0625f; o[5] = b[2] * (_Float16)0.0625f;
            o[6] = a[3] * (_Float16)0.015625f; o[7] = b[3] * (_Float16)0.015625f;
        } else {
            o[0] = a[4] * (_Float16)0.00390625f; o[1] = b[4] * (_Float16)0.00390625f;
            o[2] = a[5] * (_Float16)0.0625f; o[3] = b[5] * (_Float16)0.0625f;
            o[4] = a[6] * (_Float16)0.015625f; o[5] = b[6] * (_Float16)0.015625f;
            o[6] = a[7] * (_Float16)0.00390625f; o[7] = b[7] * (_Float16)0.00390625f;
        }
        return pack8(o);
    }
    TQ_DEV static int steps_per_group(const WDesc& w) { return w.g.gs >= 256 ? 4 : w.g.gs / 64; }
    template <int GS> static constexpr int sx_cols() { return 64 * GS; }
};

// ============================================================================
// NVFP4 (fp4.cu:187-238): word (4i+j) = columns 32i + 8j + n (nibble n; the
// low nibble of a byte is the even column); e4m3 scale per 16 columns, global
// fp32 scale applied after the row sum.  LDS order as INT4.
// ============================================================================
template <int LAYOUT>
struct FxNvfp4 {
    static constexpr int FMT = TITAN_NVFP4, CHUNK_COLS = 128;
    static constexpr bool HAS_MFMA = false, PIPE = true;
    // one token: 1536 waves aimed for (14336 x 4096 16.15 -> 15.4 us,
    // 4096 x 14336 unchanged; four and eight tokens slower with it)
    static constexpr long long WAVES_TARGET_M1 = 1536;
    // five to eight tokens: groups of two chunks (4096 x 14336 56.2 -> 51.5
    // us, 14336 x 4096 unchanged; one and four tokens lose on one shape)
    static constexpr int U2_MIN_M = 8, U2_MAX_M = 8;
    struct Off { uint32_t c, s; };
    struct Raw { uint32_t w[4]; uint32_t s0, s1; };
    struct Dec { float s[4]; };
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        const Geo& g = w.g;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            return {(uint32_t)row * (uint32_t)g.row_code_bytes + 4u * j, (uint32_t)row * (uint32_t)(g.cols / 16)};
        else
            return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_nvs_off(g, row, 0)};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
#pragma unroll
            for (int i = 0; i < 4; i++) r.w[i] = ld_u32(w.codes + (o.c + (uint32_t)c * 64u + 16u * i));
            const uint8_t* sp = w.scales + (o.s + (uint32_t)c * 8u);
            r.s0 = ld_u32(sp);
            r.s1 = ld_u32(sp + 4);
        } else {
            uint4 q = ld_code_chunk<NT>(rs, lane, u);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
            const uint8_t* sp = w.codes + (o.s + (uint32_t)c * 128u);
            r.s0 = ld_u32(sp);
            r.s1 = ld_u32(sp + 4);
        }
    }
    // word step i, lane j: scale byte 2i + (j >> 1) of the chunk's 8
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int j) {
        Dec d;
        const int sh = 8 * (j >> 1);
        d.s[0] = e4m3_ref_to_f32(r.s0 >> sh);
        d.s[1] = e4m3_ref_to_f32(r.s0 >> (16 + sh));
        d.s[2] = e4m3_ref_to_f32(r.s1 >> sh);
        d.s[3] = e4m3_ref_to_f32(r.s1 >> (16 + sh));
        return d;
    }
    TQ_DEV static float fold_f32(const Raw& r, const Dec& d, int j, const float* xc, const float*) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x[8];
            ld_f8(xc + 32 * i + 8 * j, x);
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int n = 0; n < 8; n += 2) {
                a = __builtin_fmaf(fp4_to_f32((r.w[i] >> (4 * n)) & 0xF), x[n], a);
                b = __builtin_fmaf(fp4_to_f32((r.w[i] >> (4 * n + 4)) & 0xF), x[n + 1], b);
            }
            t = __builtin_fmaf(d.s[i], a + b, t);
        }
        return t;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec& d, int j, const _Float16* xc, const float*) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xv = *(const uint4*)(xc + 32 * i + 8 * j);
            const uint32_t w = r.w[i];
            float a = dot2(fp4_pair(w, 0), xv.x, 0.0f);
            float b = dot2(fp4_pair(w, 2), xv.y, 0.0f);
            a = dot2(fp4_pair(w, 1), xv.z, a);
            b = dot2(fp4_pair(w, 3), xv.w, b);
            t = __builtin_fmaf(d.s[i], a + b, t);
        }
        return t * kTwo14;
    }
    template <int NB, int GS, bool SX> struct Tmp {};
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw&, int, const _Float16* const*, Tmp<NB, GS, SX>&) {}
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>&, const Dec&, const float*, f4_t*) {}
    static constexpr bool STAGE_LOCAL = true;
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) { return FxNib<LAYOUT, true>::stage8(xr, d0); }
    TQ_DEV static uint4 stage8_raw(uint4 raw) { return FxNib<LAYOUT, true>::stage8_raw(raw); }
    TQ_DEV static int steps_per_group(const WDesc&) { return 1; }
    template <int GS> static constexpr int sx_cols() { return 32; }
};

// ============================================================================
// Q4_K (ggml): chunk c = half (c & 1) of block c >> 1; word step i covers qs
// bytes 64(c&1) + 16i .. +15 = positions l = 16(i&1) + 4j + k of the 64-element
// group c4 = 2(c&1) + (i>>1): low nibbles are sub-block 2*c4 (column
// 64*c4' + l), high nibbles sub-block 2*c4 + 1 (column + 32), c4' = i >> 1
// inside the chunk.  LDS order per 64 columns: for each l4 = l/4:
// [A(l+0), A(l+2), A(l+1), A(l+3), B(l+0), B(l+2), B(l+1), B(l+3)] with
// A(x) = column x, B(x) = column 32 + x.
// ============================================================================
template <int LAYOUT>
struct FxQ4K {
    static constexpr int FMT = TITAN_Q4_K, CHUNK_COLS = 128;
    static constexpr bool HAS_MFMA = true, PIPE = true;
    // one token: fewer, longer waves (the 14336-column rows split over two
    // waves, not four) measured 2-5% faster on the Llama-3-8B layer (31.7 ->
    // 30.5 us); INT4 measured slower with the same target
    static constexpr long long WAVES_TARGET_M1 = 1536;
    // two to eight tokens: groups of two chunks (8B layer: 2 tokens 35.5-38.9
    // -> 31.1-32.3 us, 4 tokens 45.3-46.6 -> 40.1-41.8 us, 28672 x 8192 at 4
    // tokens 48.4-49.3 -> 43.0 us); one token about 1-2% slower and 16
    // tokens 35% slower with them
    static constexpr int U2_MIN_M = 2, U2_MAX_M = 8;
    struct Off { uint32_t c, h; };
    struct Raw { uint32_t w[4]; uint4 hdr; };
    // decode<GS>(w, raw, c, j) uses only the parity of c (which half block)
    static constexpr bool HALF_FROM_U = true;
    // [2*c4' + (0: low / 1: high nibbles)]: ds = d sc 2^24 (low) or
    // d sc 2^20 (high, whose codes sit x16), the MFMA fold's code scales;
    // dm = -dmin m
    struct Dec { float ds[4], dm[4]; };
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        const Geo& g = w.g;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            return {(uint32_t)row * (uint32_t)(g.nblk * 144) + 16u + 4u * j, (uint32_t)row * (uint32_t)(g.nblk * 144)};
        else
            return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_q4k_hdr_off(g, row, 0)};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        const uint32_t blk = (uint32_t)c >> 1;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.hdr = ld_u128(w.codes + (o.h + blk * 144u));
            const uint32_t q = o.c + blk * 144u + ((uint32_t)c & 1u) * 64u;
#pragma unroll
            for (int i = 0; i < 4; i++) r.w[i] = ld_u32(w.codes + (q + 16u * i));
        } else {
            r.hdr = ld_u128(w.codes + (o.h + blk * 256u));
            uint4 q = ld_code_chunk<NT>(rs, lane, u);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        }
    }
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int c, int) {
        const float d = f16_to_f32(r.hdr.x & 0xFFFF), dmin = f16_to_f32(r.hdr.x >> 16);
        // The four 6-bit scales and mins of this half block, one per byte,
        // without a branch on the half (ggml packing, scales bytes s[0..11]
        // in hdr.y/z/w): sub-blocks 0..3 are s[k] & 63 and s[4+k] & 63;
        // sub-blocks 4..7 take the low / high nibble of s[8+k] and bits 6..7
        // of s[k] / s[4+k] as their bits 4..5.  Both are (A & 0x0F) |
        // ((B >> 2) & 0x30) per byte for the right A, B.
        const uint32_t s0 = r.hdr.y, s1 = r.hdr.z, s2 = r.hdr.w;
        const bool hi = c & 1;
        const uint32_t a_sc = hi ? s2 : s0, b_sc = hi ? s0 : s0 << 2;
        const uint32_t a_m = hi ? s2 >> 4 : s1, b_m = hi ? s1 : s1 << 2;
        const uint32_t SC = (a_sc & 0x0F0F0F0Fu) | ((b_sc >> 2) & 0x30303030u);
        const uint32_t MN = (a_m & 0x0F0F0F0Fu) | ((b_m >> 2) & 0x30303030u);
        Dec o;
        const float dlo = d * kTwo24, dhi = d * (kTwo24 / 16.0f), nmin = -dmin;  // exact scalings
#pragma unroll
        for (int k = 0; k < 4; k++) {
            o.ds[k] = (k & 1 ? dhi : dlo) * (float)((SC >> (8 * k)) & 0xFFu);
            o.dm[k] = nmin * (float)((MN >> (8 * k)) & 0xFFu);
        }
        return o;
    }
    TQ_DEV static float bias(const Dec& d, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) t = __builtin_fmaf(d.dm[k], s16[2 * k] + s16[2 * k + 1], t);
        return t;
    }
    TQ_DEV static float fold_f32(const Raw& r, const Dec& d, int j, const float* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int base = 64 * (i >> 1) + 16 * (i & 1) + 4 * j;
            float xa[4], xb[4];
            ld_f4(xc + base, xa);
            ld_f4(xc + base + 32, xb);
            const uint32_t lo = r.w[i] & 0x0F0F0F0Fu, hi = (r.w[i] >> 4) & 0x0F0F0F0Fu;
            float a = (float)(lo & 0xFF) * xa[0];
            a = __builtin_fmaf((float)((lo >> 8) & 0xFF), xa[1], a);
            a = __builtin_fmaf((float)((lo >> 16) & 0xFF), xa[2], a);
            a = __builtin_fmaf((float)(lo >> 24), xa[3], a);
            float b = (float)(hi & 0xFF) * xb[0];
            b = __builtin_fmaf((float)((hi >> 8) & 0xFF), xb[1], b);
            b = __builtin_fmaf((float)((hi >> 16) & 0xFF), xb[2], b);
            b = __builtin_fmaf((float)(hi >> 24), xb[3], b);
            t = __builtin_fmaf(d.ds[2 * (i >> 1)] * (1.0f / kTwo24), a, t);  // d sc (exact)
            t = __builtin_fmaf(d.ds[2 * (i >> 1) + 1] * (16.0f / kTwo24), b, t);
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec& d, int j, const _Float16* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xv = *(const uint4*)(xc + 64 * (i >> 1) + 8 * (4 * (i & 1) + j));
            const uint32_t w = r.w[i], u = w >> 8;
            float a = dot2(w & 0x000F000Fu, xv.x, 0.0f);  // low nibbles, bytes (0, 2)
            a = dot2(u & 0x000F000Fu, xv.y, a);           // bytes (1, 3)
            float b = dot2(w & 0x00F000F0u, xv.z, 0.0f);  // high nibbles x16
            b = dot2(u & 0x00F000F0u, xv.w, b);
            t = __builtin_fmaf(d.ds[2 * (i >> 1)], a, t);
            t = __builtin_fmaf(d.ds[2 * (i >> 1) + 1], b, t);
        }
        return j == 0 ? t + bias(d, s16) : t;
    }
    template <int NB, int GS, bool SX>
    struct Tmp { f4_t CA[2][NB], CB[2][NB], OA[SX ? 1 : 2][NB], OB[SX ? 1 : 2][NB]; };
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw& r, int j, const _Float16* const* xt, Tmp<NB, GS, SX>& T) {
        // word steps i = 2h and 2h + 1 fold into the same sub-block tiles: one
        // 16x16x32 step over both (A and B take their columns in the same
        // order, so the products pair up as in two 16x16x16 steps)
        const h8_t ones = h8_of(make_uint4(kOnes2, kOnes2, kOnes2, kOnes2));
#pragma unroll
        for (int h = 0; h < 2; h++) {  // the two 64-element groups of the chunk
            const uint32_t w0 = r.w[2 * h], u0 = w0 >> 8, w1 = r.w[2 * h + 1], u1 = w1 >> 8;
            const h8_t blo = h8_of(make_uint4(w0 & 0x000F000Fu, u0 & 0x000F000Fu, w1 & 0x000F000Fu, u1 & 0x000F000Fu));
            const h8_t bhi = h8_of(make_uint4(w0 & 0x00F000F0u, u0 & 0x00F000F0u, w1 & 0x00F000F0u,
                                              u1 & 0x00F000F0u));  // x16
#pragma unroll
            for (int n = 0; n < NB; n++) {
                const uint4 x0 = *(const uint4*)(xt[n] + 64 * h + 8 * j);
                const uint4 x1 = *(const uint4*)(xt[n] + 64 * h + 8 * (4 + j));
                const h8_t xa = h8_of(make_uint4(x0.x, x0.y, x1.x, x1.y)), xb = h8_of(make_uint4(x0.z, x0.w, x1.z, x1.w));
                T.CA[h][n] = mfma32(xa, blo, f4_zero());
                T.CB[h][n] = mfma32(xb, bhi, f4_zero());
                if constexpr (!SX) {
                    T.OA[h][n] = mfma32(xa, ones, f4_zero());
                    T.OB[h][n] = mfma32(xb, ones, f4_zero());
                }
            }
        }
    }
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>& T, const Dec& d, const float* sx, f4_t* acc) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float sa = d.ds[2 * h], sb = d.ds[2 * h + 1];
            const float ma = d.dm[2 * h], mb = d.dm[2 * h + 1];
            float4 xa, xb;  // sub-block sums (32 columns each) for tokens 0..3
            if constexpr (SX) {
                xa = *(const float4*)(sx + 4 * (2 * h));
                xb = *(const float4*)(sx + 4 * (2 * h + 1));
            }
#pragma unroll
            for (int n = 0; n < NB; n++)
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    float t = __builtin_fmaf(sa, T.CA[h][n][v], acc[n][v]);
                    t = __builtin_fmaf(sb, T.CB[h][n][v], t);
                    const float oa = SX ? (v == 0 ? xa.x : v == 1 ? xa.y : v == 2 ? xa.z : xa.w)
                                        : T.OA[SX ? 0 : h][n][v];
                    const float ob = SX ? (v == 0 ? xb.x : v == 1 ? xb.y : v == 2 ? xb.z : xb.w)
                                        : T.OB[SX ? 0 : h][n][v];
                    t = __builtin_fmaf(ma, oa, t);
                    acc[n][v] = __builtin_fmaf(mb, ob, t);
                }
        }
    }
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) {
        const int g64 = d0 & ~63, l = ((d0 & 63) >> 3) * 4;
        _Float16 a[4], b[4], o[8];
        ldh4(xr + g64 + l, a);
        ldh4(xr + g64 + 32 + l, b);
        o[0] = a[0]; o[1] = a[2]; o[2] = a[1]; o[3] = a[3];
        o[4] = b[0]; o[5] = b[2]; o[6] = b[1]; o[7] = b[3];
        return pack8(o);
    }
    TQ_DEV static int steps_per_group(const WDesc&) { return 2; }
    template <int GS> static constexpr int sx_cols() { return 32; }
};

// ============================================================================
// Q3_K (ggml, tiled layout only): chunk c = block c; word step i covers qs
// bytes 16i + 4j + k: half h = i >> 1, position l = 16(i&1) + 4j + k; level
// jj (bits 2jj of the byte, hmask bit 4h + jj of hmask[l]) is column
// 128h + 32jj + l with sub-block scale 8h + 2jj + (i&1).  LDS order per
// 256 columns: for each (h, l4 = l/4) 16 halves [jj: l+0, l+2, l+1, l+3].
// ============================================================================
template <int LAYOUT>
struct FxQ3K {
    static constexpr int FMT = TITAN_Q3_K, CHUNK_COLS = 256;
    // 2048 waves aimed for (the default).  With four-chunk groups 1536
    // measured 11-13% faster (8B layer one token 40.8 -> 35.5-36.0 us);
    // with two-chunk groups 2048 is: 28672 x 8192 one token 32.6-34.6 ->
    // 30.5-30.6 us, 8B layer two tokens 42.4-42.7 -> 39.9-41.1 us, the layer
    // at one token within 1 us either way, 8192 x 28672 one token 1-2%
    // slower in one pair
    static constexpr long long WAVES_TARGET = 2048;
    // every token count: groups of two chunks (8B layer: one token 31.9-32.1
    // -> 29.9-30.1 us, 8 tokens 76.6-77.3 -> 73.6-73.7 us, 16 tokens 158.4
    // -> 130.8-131.1 us, 2-4 tokens 2-3% faster; 1024 x 8192 one token 9.6
    // -> 9.0 us)
    static constexpr int U2_MIN_M = 1, U2_MAX_M = 16;
    // the EXACT kernel of this fold holds ~290 VGPRs against ~155 (one wave
    // per SIMD instead of three): Q3_K keeps the general kernel
    static constexpr bool NO_EXACT = true;
    // matrix cores: one 16x16x16 step per (word, level) = one 16-column
    // sub-block, folded at once with its scale (PIPE = false: issue and
    // finish of a chunk run back to back)
    static constexpr bool HAS_MFMA = true, PIPE = false;
    // one or two tokens: codes folded in place and the -4 offset applied
    // from 16-column activation sums (SX); more tokens: codes moved to bit 0
    // and offset in fp16
    static constexpr int SX_MAX_M = 2;
    struct Off { uint32_t c, h, s, d; };
    struct Raw { uint32_t w[4]; uint32_t hm0, hm1, s0, s1, s2, dh; };
    struct Dec { float dsc[4][4], m4[4][4]; };  // [i][jj]: d (sc - 32), -4 d (sc - 32)
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        const Geo& g = w.g;
        return {(uint32_t)tiled_code_off(g, row, 0, j), (uint32_t)tiled_q3k_hmask_off(g, row, 0, j),
                (uint32_t)tiled_q3k_sc_off(g, row, 0), (uint32_t)tiled_q3k_d_off(g, row, 0)};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        const uint32_t b = (uint32_t)c;
        uint4 q = ld_code_chunk<NT>(rs, lane, u);
        r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        const uint8_t* hp = w.codes + (o.h + b * 512u);
        r.hm0 = ld_u32(hp);
        r.hm1 = ld_u32(hp + 4);
        const uint8_t* sp = w.codes + (o.s + b * 192u);
        r.s0 = ld_u32(sp);
        r.s1 = ld_u32(sp + 4);
        r.s2 = ld_u32(sp + 8);
        r.dh = ld_u16(w.codes + (o.d + b * 32u));
    }
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        // the 16 six-bit scales, four per register as bytes (ggml packing:
        // low nibbles from bytes 0..7, high 2 bits from bytes 8..11), then
        // d * (sc - 32) as one fused multiply-add per scale
        const uint32_t L[4] = {
            (r.s0 & 0x0F0F0F0Fu) | ((r.s2 & 0x03030303u) << 4),          // k = 0..3
            (r.s1 & 0x0F0F0F0Fu) | (((r.s2 >> 2) & 0x03030303u) << 4),   // 4..7
            ((r.s0 >> 4) & 0x0F0F0F0Fu) | (((r.s2 >> 4) & 0x03030303u) << 4),  // 8..11
            ((r.s1 >> 4) & 0x0F0F0F0Fu) | (((r.s2 >> 6) & 0x03030303u) << 4)}; // 12..15
        Dec o;
        const float d = f16_to_f32(r.dh), d32 = -32.0f * d, dm4 = -4.0f * d, d128 = 128.0f * d;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int k = 8 * (i >> 1) + 2 * jj + (i & 1);
                const float sc = (float)((L[k >> 2] >> (8 * (k & 3))) & 0xFFu);
                o.dsc[i][jj] = __builtin_fmaf(sc, d, d32);
                o.m4[i][jj] = __builtin_fmaf(sc, dm4, d128);  // exact: -4 is a power of two
            }
        return o;
    }
    // the hmask bits of word step i in the tiled order (see tiled_q3k_hmask_off):
    // half h = i >> 1 rotated down to the h = 0 positions
    TQ_DEV static uint32_t hbits(const Raw& r, int i) {
        const uint32_t p = (i & 1) ? r.hm1 : r.hm0;
        return (i >> 1) ? __builtin_amdgcn_alignbit(p, p, 8) : p;
    }
    // 3-bit code u = q2 + 4 * hbit of the 4 bytes of word step i at level jj
    // (bytes 0, 2: hmask bit 2jj + 2 (+16) -> bit 2; bytes 1, 3: 2jj + 3 (+16))
    TQ_DEV static uint32_t code3(const Raw& r, int i, int jj) {
        const uint32_t x = hbits(r, i);
        return ((r.w[i] >> (2 * jj)) & 0x03030303u) | ((x >> (2 * jj)) & 0x00040004u) |
               ((x << (7 - 2 * jj)) & 0x04000400u);
    }
    TQ_DEV static uint32_t code3x(const Raw& r, int i, int jj) { return code3(r, i, jj); }
    TQ_DEV static float bias(const Dec& d, const float* s16) {
        // value = d*sc*(u - 4): the -4 term is -4 d sc sum(x) per sub-block
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                t = __builtin_fmaf(-4.0f * d.dsc[i][jj], s16[8 * (i >> 1) + 2 * jj + (i & 1)], t);
        return t;
    }
    TQ_DEV static float fold_f32(const Raw& r, const Dec& d, int j, const float* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                float x[4];
                ld_f4(xc + 128 * (i >> 1) + 32 * jj + 16 * (i & 1) + 4 * j, x);
                const uint32_t v = code3(r, i, jj);
                float a = (float)(v & 0xFF) * x[0];
                a = __builtin_fmaf((float)((v >> 8) & 0xFF), x[1], a);
                a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[2], a);
                a = __builtin_fmaf((float)(v >> 24), x[3], a);
                t = __builtin_fmaf(d.dsc[i][jj], a, t);
            }
        return j == 0 ? t + bias(d, s16) : t;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec& d, int j, const _Float16* xc, const float* s16) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16* p = xc + 16 * (8 * (i >> 1) + 4 * (i & 1) + j);
            const uint4 x01 = *(const uint4*)p, x23 = *(const uint4*)(p + 8);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const uint32_t v = code3(r, i, jj);
                const uint32_t xa = jj == 0 ? x01.x : jj == 1 ? x01.z : jj == 2 ? x23.x : x23.z;
                const uint32_t xb = jj == 0 ? x01.y : jj == 1 ? x01.w : jj == 2 ? x23.y : x23.w;
                float a = dot2(v & 0x00070007u, xa, 0.0f);
                a = dot2((v >> 8) & 0x00070007u, xb, a);
                t = __builtin_fmaf(d.dsc[i][jj], a, t);
            }
        }
        t *= kTwo24;
        return j == 0 ? t + bias(d, s16) : t;
    }
    template <int NB, int GS, bool SX> struct Tmp { f4_t C[16][NB]; };
    // SX: the codes u of level jj in place as fp16 subnormals, u * 2^(2jj-24):
    // bits 2jj, 2jj+1 of the byte from the 2-bit word, bit 2jj+2 from the
    // hmask; the halves hold bytes (0, 2) and (1, 3) of the word
    // (the tiled hmask order puts the high bit of level jj of bytes 0, 2 at
    // bit 2jj + 2 of the word and of bytes 1, 3 one bit higher: no shift per
    // level)
    TQ_DEV static h4_t codes_in_place(const Raw& r, int i, int jj) {
        const uint32_t w = r.w[i], w8 = w >> 8;
        const uint32_t x = hbits(r, i), x1 = x >> 1;
        const uint32_t mq = 0x00030003u << (2 * jj), mh = 0x00040004u << (2 * jj);
        return h4_of((w & mq) | (x & mh), (w8 & mq) | (x1 & mh));
    }
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw& r, int j, const _Float16* const* xt, Tmp<NB, GS, SX>& T) {
        if constexpr (SX) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const h4_t b = codes_in_place(r, i, jj);
#pragma unroll
                    for (int n = 0; n < NB; n++) {
                        const _Float16* p = xt[n] + 16 * (8 * (i >> 1) + 4 * (i & 1) + j) + 4 * jj;
                        const uint2 xv = *(const uint2*)p;
                        T.C[4 * i + jj][n] = mfma16(h4_of(xv.x, xv.y), b, f4_zero());
                    }
                }
            return;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                // codes u = q2 + 4 hbit as exact fp16 subnormals, minus 4
                // (exact): the sub-block's weights are d * sc * b
                const uint32_t v = code3x(r, i, jj);
                typedef _Float16 q3h2 __attribute__((ext_vector_type(2)));
                const q3h2 m4 = __builtin_bit_cast(q3h2, 0x80048004u);
                const q3h2 b01 = __builtin_bit_cast(q3h2, v & 0x00070007u) + m4;
                const q3h2 b23 = __builtin_bit_cast(q3h2, (v >> 8) & 0x00070007u) + m4;
                const h4_t b = h4_of(__builtin_bit_cast(uint32_t, b01), __builtin_bit_cast(uint32_t, b23));
#pragma unroll
                for (int n = 0; n < NB; n++) {
                    const _Float16* p = xt[n] + 16 * (8 * (i >> 1) + 4 * (i & 1) + j) + 4 * jj;
                    const uint2 xv = *(const uint2*)p;
                    T.C[4 * i + jj][n] = mfma16(h4_of(xv.x, xv.y), b, f4_zero());
                }
            }
    }
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>& T, const Dec& d, const float* sx, f4_t* acc) {
        if constexpr (SX) {
            // sub-block k = 8(i>>1) + 2jj + (i&1): d sc * (C 2^(24-2jj) - 4 sum(x))
            // = (-4 d sc) * (sum(x) - C 2^(22-2jj)); sums at sx[2k + token]
            static_assert(NB == 1 && NV <= 2, "SX folds at most two tokens");
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const int k = 8 * (i >> 1) + 2 * jj + (i & 1);
                    const float2 s2 = *(const float2*)(sx + 2 * k);
                    const float m4 = d.m4[i][jj], kc = -(float)(1u << (22 - 2 * jj));
#pragma unroll
                    for (int v = 0; v < NV; v++) {
                        const float t = __builtin_fmaf(T.C[4 * i + jj][0][v], kc, v == 0 ? s2.x : s2.y);
                        acc[0][v] = __builtin_fmaf(m4, t, acc[0][v]);
                    }
                }
            return;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float sc = d.dsc[i][jj] * kTwo24;
#pragma unroll
                for (int n = 0; n < NB; n++)
#pragma unroll
                    for (int v = 0; v < NV; v++)
                        acc[n][v] = __builtin_fmaf(sc, T.C[4 * i + jj][n][v], acc[n][v]);
            }
    }
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) {
        // d0 = 16 * (8h + l4) + 8 * p: levels jj = 2p, 2p+1 of positions l..l+3
        const int e = d0 >> 4, h = e >> 3, l = (e & 7) * 4, jj = (d0 & 8) ? 2 : 0;
        _Float16 a[4], b[4], o[8];
        ldh4(xr + 128 * h + 32 * jj + l, a);
        ldh4(xr + 128 * h + 32 * (jj + 1) + l, b);
        o[0] = a[0]; o[1] = a[2]; o[2] = a[1]; o[3] = a[3];
        o[4] = b[0]; o[5] = b[2]; o[6] = b[1]; o[7] = b[3];
        return pack8(o);
    }
    TQ_DEV static int steps_per_group(const WDesc&) { return 1; }
    template <int GS> static constexpr int sx_cols() { return 16; }
};

// ============================================================================
// FP8 E4M3 with a per-row fp32 scale applied after the row sum: word (4i+j) =
// columns 16i + 4j + k.  LDS order per 4 columns [0, 2, 1, 3].
// ============================================================================
template <int LAYOUT>
struct FxFp8 {
    static constexpr int FMT = TITAN_FP8_E4M3, CHUNK_COLS = 64;
    static constexpr bool HAS_MFMA = false, PIPE = true;
    // one token: 1536 waves aimed for (14336 x 4096 14.1-14.3 -> 13.0-13.3
    // us, 4096 x 14336 unchanged; eight tokens slower with it)
    static constexpr long long WAVES_TARGET_M1 = 1536;
    // three or four tokens: groups of two chunks (4096 x 14336 35.3-35.5 ->
    // 28.9-29.0 us, 14336 x 4096 24.0 -> 23.5 us; one token 20% and eight
    // tokens 10% slower on one shape)
    static constexpr int U2_MIN_M = 4, U2_MAX_M = 4;
    struct Off { uint32_t c; };
    struct Raw { uint32_t w[4]; };
    struct Dec {};
    TQ_DEV static Off base(const WDesc& w, int row, int j) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            return {(uint32_t)row * (uint32_t)w.g.row_code_bytes + 4u * j};
        else
            return {(uint32_t)tiled_code_off(w.g, row, 0, j)};
    }
    template <int GS, bool NT = true>
    TQ_DEV static void load(const WDesc& w, const Off& o, int c, int, Raw& r, __amdgpu_buffer_rsrc_t rs,
                            uint32_t lane, int u) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
#pragma unroll
            for (int i = 0; i < 4; i++) r.w[i] = ld_u32(w.codes + (o.c + (uint32_t)c * 64u + 16u * i));
        } else {
            uint4 q = ld_code_chunk<NT>(rs, lane, u);
            r.w[0] = q.x; r.w[1] = q.y; r.w[2] = q.z; r.w[3] = q.w;
        }
    }
    template <int GS>
    TQ_DEV static Dec decode(const WDesc&, const Raw&, int, int) { return {}; }
    TQ_DEV static float fold_f32(const Raw& r, const Dec&, int j, const float* xc, const float*) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float x[4];
            ld_f4(xc + 16 * i + 4 * j, x);
            a = __builtin_fmaf(e4m3_ocp_to_f32(r.w[i]), x[0], a);
            b = __builtin_fmaf(e4m3_ocp_to_f32(r.w[i] >> 8), x[1], b);
            a = __builtin_fmaf(e4m3_ocp_to_f32(r.w[i] >> 16), x[2], a);
            b = __builtin_fmaf(e4m3_ocp_to_f32(r.w[i] >> 24), x[3], b);
        }
        return a + b;
    }
    TQ_DEV static float fold_h(const Raw& r, const Dec&, int j, const _Float16* xc, const float*) {
        // e4m3 byte -> fp16 bits by shifting: value * 2^-8, exact (the NaN
        // codes are not produced by quantizers and are not special-cased)
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint2 xv = *(const uint2*)(xc + 16 * i + 4 * j);
            const uint32_t w = r.w[i], u = w >> 8;
            a = dot2(((w & 0x007F007Fu) << 7) | ((w & 0x00800080u) << 8), xv.x, a);
            b = dot2(((u & 0x007F007Fu) << 7) | ((u & 0x00800080u) << 8), xv.y, b);
        }
        return (a + b) * 256.0f;
    }
    template <int NB, int GS, bool SX> struct Tmp {};
    template <int NB, int GS, bool SX>
    TQ_DEV static void issue(const Raw&, int, const _Float16* const*, Tmp<NB, GS, SX>&) {}
    template <int NB, int NV, int GS, bool SX>
    TQ_DEV static void finish(const Tmp<NB, GS, SX>&, const Dec&, const float*, f4_t*) {}
    static constexpr bool STAGE_LOCAL = true;
    TQ_DEV static uint4 stage8(const _Float16* xr, int d0) { return stage8_raw(*(const uint4*)(xr + d0)); }
    TQ_DEV static uint4 stage8_raw(uint4 raw) {
        const h8_t h = h8_of(raw);
        _Float16 o[8];
        o[0] = h[0]; o[1] = h[2]; o[2] = h[1]; o[3] = h[3];
        o[4] = h[4]; o[5] = h[6]; o[6] = h[5]; o[7] = h[7];
        return pack8(o);
    }
    TQ_DEV static int steps_per_group(const WDesc&) { return 1; }
    template <int GS> static constexpr int sx_cols() { return 32; }
};

}  // namespace tq
