// formats.h -- device-side decoders of every weight format, both layouts.
//
// Two views of each format:
//  * elem<FMT, LAYOUT>(w, row, col): the exact fp32 dequantized value, one
//    element at a time (dequant kernel, generic GEMV for ragged shapes).
//  * Fmt* structs: the fast GEMV view.  A wave covers 16 rows x one 64-byte
//    chunk of codes; lane l = 16*j + r owns row r's 16-byte slot j.  Each
//    struct loads a lane's slot ("Raw") and folds it against activations in
//    SEGS segments of SEGW contiguous columns: contribution = scale * sum(q*x)
//    (+ offset * sum(x) for affine formats), which equals sum(w*x) with w the
//    exact dequantized weight up to fp32 reassociation.
#pragma once

#include "common.h"
#include "layout.h"

namespace tq {

// Device view of one weight matrix.
struct WDesc {
    const uint8_t* codes;
    const uint8_t* scales;
    const uint8_t* biases;
    Geo g;
    float gscale;
    int gshift;  // log2(group size) for power-of-two groups, else -1
};

TQ_DEV uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }
TQ_DEV uint32_t ld_u32(const uint8_t* p) { return *(const uint32_t*)p; }
TQ_DEV uint4 ld_u128(const uint8_t* p) { return *(const uint4*)p; }
TQ_DEV uint32_t byte_of(uint4 v, int i) {
    uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xFF;
}

// ---- K-quant scale unpacking (ggml block formats) ----------------------------
// Q4_K sub-block j (0..7) 6-bit scale/min from the 12 scale bytes s[0..11]
// held as three little-endian words.
TQ_DEV uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    uint32_t w = i < 4 ? s0 : i < 8 ? s1 : s2;
    return (w >> (8 * (i & 3))) & 0xFF;
}
TQ_DEV void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t& sc,
                          uint32_t& m) {
    if (j < 4) {
        sc = sbyte(s0, s1, s2, j) & 63;
        m = sbyte(s0, s1, s2, j + 4) & 63;
    } else {
        sc = (sbyte(s0, s1, s2, j + 4) & 0xF) | ((sbyte(s0, s1, s2, j - 4) >> 6) << 4);
        m = (sbyte(s0, s1, s2, j + 4) >> 4) | ((sbyte(s0, s1, s2, j) >> 6) << 4);
    }
}
// Q3_K signed 6-bit scale k (0..15).
TQ_DEV int q3k_scale(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
    uint32_t lo = k < 8 ? (sbyte(s0, s1, s2, k) & 0xF) : (sbyte(s0, s1, s2, k - 8) >> 4);
    uint32_t hi = (sbyte(s0, s1, s2, 8 + (k & 3)) >> (2 * (k >> 2))) & 3;
    return (int)(lo | (hi << 4)) - 32;
}

// ============================================================================
// Exact element values.
// ============================================================================
template <int FMT, int LAYOUT>
TQ_DEV float elem(const WDesc& w, int row, int col) {
    const Geo& g = w.g;
    if constexpr (FMT == TITAN_INT4 || FMT == TITAN_INT2 || FMT == TITAN_FP4) {
        constexpr int BITS = FMT == TITAN_INT2 ? 2 : 4;
        constexpr int PER = 32 / BITS;
        uint32_t word;
        int grp = (col & ~(PER - 1)) / g.gs;  // dequant.cu:63: group of the word's base column
        float s, b = 0.0f;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            word = ((const uint32_t*)w.codes)[(size_t)row * (g.cols / PER) + col / PER];
            s = f16_to_f32(((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp]);
            if constexpr (FMT != TITAN_FP4)
                b = f16_to_f32(((const uint16_t*)w.biases)[(size_t)row * g.ngroups + grp]);
        } else {
            int bi = (col / PER) * 4;  // byte index of the word in the row's code bytes
            word = ld_u32(w.codes + tiled_code_off(g, row, bi >> 6, (bi >> 4) & 3) + (bi & 15));
            if constexpr (FMT == TITAN_FP4) {
                s = f16_to_f32(ld_u16(w.codes + tiled_fp4s_off(g, row, grp)));
            } else {
                uint32_t sb = ld_u32(w.codes + tiled_sb_off(g, row, grp));
                s = f16_to_f32(sb & 0xFFFF);
                b = f16_to_f32(sb >> 16);
            }
        }
        uint32_t q = (word >> (BITS * (col % PER))) & ((1u << BITS) - 1);
        if constexpr (FMT == TITAN_FP4) return fp4_to_f32(q) * s;
        else return (float)q * s + b;  // q*s is exact: one rounding, as the reference
    } else if constexpr (FMT == TITAN_NVFP4) {
        uint32_t byte, sc;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            byte = w.codes[(size_t)row * (g.cols / 2) + col / 2];
            sc = w.scales[(size_t)row * (g.cols / 16) + col / 16];
        } else {
            int bi = col / 2;
            byte = w.codes[tiled_code_off(g, row, bi >> 6, (bi >> 4) & 3) + (bi & 15)];
            int c = col / 128, j = (col % 128) / 32;
            sc = (ld_u16(w.codes + tiled_nvs_off(g, row, c, j)) >> (8 * ((col / 16) & 1))) & 0xFF;
        }
        uint32_t q = (col & 1) ? (byte >> 4) : (byte & 0xF);
        float s0 = e4m3_ref_to_f32(sc) * w.gscale;  // fp4.cu:211-212
        return fp4_to_f32(q) * s0;
    } else if constexpr (FMT == TITAN_Q4_K) {
        int b = col / 256, e = col % 256, c4 = e / 64, l = e % 32, hi = (e % 64) >= 32;
        uint4 hdr;
        uint32_t qb;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            const uint8_t* blk = w.codes + ((size_t)row * g.nblk + b) * 144;
            hdr = ld_u128(blk);
            qb = blk[16 + 32 * c4 + l];
        } else {
            hdr = ld_u128(w.codes + tiled_q4k_hdr_off(g, row, b));
            int bi = b * 128 + 32 * c4 + l;
            qb = w.codes[tiled_code_off(g, row, bi >> 6, (bi >> 4) & 3) + (bi & 15)];
        }
        float d = f16_to_f32(hdr.x & 0xFFFF), dmin = f16_to_f32(hdr.x >> 16);
        uint32_t sc, m;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * c4 + hi, sc, m);
        float q = (float)(hi ? (qb >> 4) : (qb & 0xF));
        return (d * (float)sc) * q - dmin * (float)m;
    } else if constexpr (FMT == TITAN_Q3_K) {
        int b = col / 256, e = col % 256, h = e / 128, jj = (e % 128) / 32, l = e % 32;
        uint32_t qb, hb, s0, s1, s2, dh;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            const uint8_t* blk = w.codes + ((size_t)row * g.nblk + b) * 110;
            qb = blk[32 + 32 * h + l];
            hb = blk[l];
            const uint8_t* sp = blk + 96;
            s0 = sp[0] | (sp[1] << 8) | (sp[2] << 16) | ((uint32_t)sp[3] << 24);
            s1 = sp[4] | (sp[5] << 8) | (sp[6] << 16) | ((uint32_t)sp[7] << 24);
            s2 = sp[8] | (sp[9] << 8) | (sp[10] << 16) | ((uint32_t)sp[11] << 24);
            dh = blk[108] | (blk[109] << 8);
        } else {
            int bi = b * 64 + 32 * h + l;
            qb = w.codes[tiled_code_off(g, row, bi >> 6, (bi >> 4) & 3) + (bi & 15)];
            hb = w.codes[tiled_q3k_hmask_off(g, row, b, l >> 4) + (l & 15)];
            const uint8_t* sp = w.codes + tiled_q3k_sc_off(g, row, b);
            s0 = ld_u32(sp);
            s1 = ld_u32(sp + 4);
            s2 = ld_u32(sp + 8);
            dh = ld_u16(w.codes + tiled_q3k_d_off(g, row, b));
        }
        int k = 8 * h + 2 * jj + (l >= 16);
        float dl = f16_to_f32(dh) * (float)q3k_scale(s0, s1, s2, k);
        int q = (int)((qb >> (2 * jj)) & 3) - (((hb >> (4 * h + jj)) & 1) ? 0 : 4);
        return dl * (float)q;
    } else {  // FP8 E4M3, per-row fp32 scale
        uint32_t byte;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            byte = w.codes[(size_t)row * g.cols + col];
        } else {
            byte = w.codes[tiled_code_off(g, row, col >> 6, (col >> 4) & 3) + (col & 15)];
        }
        return e4m3_ocp_to_f32(byte) * ((const float*)w.scales)[row];
    }
}

// ============================================================================
// Fast GEMV view.
// ============================================================================

// 16 consecutive nibbles / bytes helpers ------------------------------------
// Sum of q_i * x_i over the 8 nibbles of word w (column n in bits 4n).
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
// Sum over the 16 two-bit codes of w (column n in bits 2n).
TQ_DEV float dot_crumb16(uint32_t w, const float* x) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        uint32_t v = (w >> (2 * s)) & 0x03030303u;  // codes s, s+4, s+8, s+12
        a = __builtin_fmaf((float)(v & 0xFF), x[s], a);
        b = __builtin_fmaf((float)((v >> 8) & 0xFF), x[s + 4], b);
        a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[s + 8], a);
        b = __builtin_fmaf((float)(v >> 24), x[s + 12], b);
    }
    return a + b;
}


// ---- fp16 dot-product helpers for the fp16-activation path -----------------
// A packed-code word masked down to bits that lie inside the fp16 mantissa
// field is a pair of fp16 subnormals: value = code * 2^-24 (times 2^shift
// for a field starting at bit `shift`), exact.  v_dot2_f32_f16 multiplies
// such a pair with a pair of activations and accumulates in fp32.
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
TQ_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
TQ_DEV float dot2(uint32_t codes, uint32_t x2, float acc) {
    return __builtin_amdgcn_fdot2(as_h2(codes), as_h2(x2), acc, false);
}
constexpr float kTwo24 = 16777216.0f;   // 2^24
constexpr float kTwo14 = 16384.0f;      // 2^14

// E2M1 codes of a word as fp16 pairs (value = lut * 2^-14): nibble n and
// n + 4 of word w become the low / high halves of fp4_pair(w, n).
TQ_DEV uint32_t fp4_pair(uint32_t w, int n) {
    // magnitude bits (e1 e0 m) -> fp16 bits 11..9, sign -> bit 15
    switch (n) {
        case 0: return ((w & 0x00070007u) << 9) | ((w & 0x00080008u) << 12);
        case 1: return ((w & 0x00700070u) << 5) | ((w & 0x00800080u) << 8);
        case 2: return ((w & 0x07000700u) << 1) | ((w & 0x08000800u) << 4);
        default: return ((w >> 3) & 0x0E000E00u) | (w & 0x80008000u);
    }
}

// Group index of a column (power-of-two group sizes shift).
TQ_DEV int group_of(const WDesc& w, int col) {
    return w.gshift >= 0 ? (col >> w.gshift) : col / w.g.gs;
}

// Each format: load() only issues the slot's memory loads (no use of the
// loaded values, so the wave never waits on them there); decode() turns the
// scale bits into floats when the group is folded; seg_dot() folds one
// segment against activations.
template <int LAYOUT>
struct FmtInt4 {
    static constexpr int FMT = TITAN_INT4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 1, SEGW = 32;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q; uint32_t s, b; };
    struct Dec { float s, b; };
    TQ_DEV static int seg_col(int j, int) { return 32 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = group_of(w, c * 128 + 32 * j);
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = ((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp];
            r.b = ((const uint16_t*)w.biases)[(size_t)row * g.ngroups + grp];
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            r.s = ld_u32(w.codes + tiled_sb_off(g, row, grp));
        }
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) return {f16_to_f32(r.s), f16_to_f32(r.b)};
        else return {f16_to_f32(r.s & 0xFFFF), f16_to_f32(r.s >> 16)};
    }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int, const float* x, float sx) {
        float v = dot_nib8(r.q.x, x) + dot_nib8(r.q.y, x + 8) +
                  dot_nib8(r.q.z, x + 16) + dot_nib8(r.q.w, x + 24);
        return __builtin_fmaf(d.s, v, d.b * sx);
    }
    // fp16 activations, permuted in LDS in groups of 8 (see stage_x_h)
    static constexpr int PERM = 8;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        // word i: nibbles (n, n+4) pair with x (8i+n, 8i+n+4); nibbles in
        // bits 4..7 of a half (n odd) read as 16x their code
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float lo = 0.0f, hi = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xv = xh[i];
            const uint32_t w = ws[i], t = w >> 8;
            lo = dot2(w & 0x000F000Fu, xv.x, lo);
            hi = dot2(w & 0x00F000F0u, xv.y, hi);
            lo = dot2(t & 0x000F000Fu, xv.z, lo);
            hi = dot2(t & 0x00F000F0u, xv.w, hi);
        }
        const float v = __builtin_fmaf(hi, 0.0625f, lo) * kTwo24;
        return __builtin_fmaf(d.s, v, d.b * sx);
    }
};

template <int LAYOUT>
struct FmtFp4 {
    static constexpr int FMT = TITAN_FP4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 1, SEGW = 32;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; uint32_t s; };
    struct Dec { float s; };
    TQ_DEV static int seg_col(int j, int) { return 32 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = group_of(w, c * 128 + 32 * j);
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = ((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp];
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            r.s = ld_u16(w.codes + tiled_fp4s_off(g, row, grp));
        }
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) { return {f16_to_f32(r.s)}; }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int, const float* x, float) {
        float a = 0.0f, b = 0.0f;
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int n = 0; n < 8; n += 2) {
                a = __builtin_fmaf(fp4_to_f32((ws[i] >> (4 * n)) & 0xF), x[8 * i + n], a);
                b = __builtin_fmaf(fp4_to_f32((ws[i] >> (4 * n + 4)) & 0xF), x[8 * i + n + 1], b);
            }
        return d.s * (a + b);
    }
    // fp16 activations, permuted in LDS in groups of 8 (see stage_x_h)
    static constexpr int PERM = 8;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 xv = xh[i];
            a = dot2(fp4_pair(ws[i], 0), xv.x, a);
            b = dot2(fp4_pair(ws[i], 1), xv.y, b);
            a = dot2(fp4_pair(ws[i], 2), xv.z, a);
            b = dot2(fp4_pair(ws[i], 3), xv.w, b);
        }
        return d.s * ((a + b) * kTwo14);
    }
};

template <int LAYOUT>
struct FmtInt2 {
    static constexpr int FMT = TITAN_INT2, CHUNK_COLS = 256, SLOT_COLS = 64;
    static constexpr int SEGS = 2, SEGW = 32;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q; uint32_t s, b; };
    struct Dec { float s, b; };
    TQ_DEV static int seg_col(int j, int seg) { return 64 * j + 32 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = group_of(w, c * 256 + 64 * j);
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = ((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp];
            r.b = ((const uint16_t*)w.biases)[(size_t)row * g.ngroups + grp];
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            r.s = ld_u32(w.codes + tiled_sb_off(g, row, grp));
        }
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) return {f16_to_f32(r.s), f16_to_f32(r.b)};
        else return {f16_to_f32(r.s & 0xFFFF), f16_to_f32(r.s >> 16)};
    }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int seg, const float* x, float sx) {
        uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        float v = dot_crumb16(w0, x) + dot_crumb16(w1, x + 16);
        return __builtin_fmaf(d.s, v, d.b * sx);
    }
    // fp16 activations, permuted in LDS in groups of 16 (see stage_x_h)
    static constexpr int PERM = 16;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        // word: codes (n, n+8) pair with x (n, n+8); the field at bit 2n
        // reads as 4^n times its code
        const uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        float s1 = 0.0f, s4 = 0.0f, s16 = 0.0f, s64 = 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t w = i ? w1 : w0, t = w >> 8;
            const uint4 xa = xh[2 * i], xb = xh[2 * i + 1];
            s1 = dot2(w & 0x00030003u, xa.x, s1);
            s4 = dot2(w & 0x000C000Cu, xa.y, s4);
            s16 = dot2(w & 0x00300030u, xa.z, s16);
            s64 = dot2(w & 0x00C000C0u, xa.w, s64);
            s1 = dot2(t & 0x00030003u, xb.x, s1);
            s4 = dot2(t & 0x000C000Cu, xb.y, s4);
            s16 = dot2(t & 0x00300030u, xb.z, s16);
            s64 = dot2(t & 0x00C000C0u, xb.w, s64);
        }
        const float v = (__builtin_fmaf(s4, 0.25f, s1) + __builtin_fmaf(s64, 0.25f, s16) * 0.0625f) * kTwo24;
        return __builtin_fmaf(d.s, v, d.b * sx);
    }
};

template <int LAYOUT>
struct FmtNvfp4 {
    static constexpr int FMT = TITAN_NVFP4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 2, SEGW = 16;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; uint32_t sc; };
    struct Dec { float s0, s1; };
    TQ_DEV static int seg_col(int j, int seg) { return 32 * j + 16 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.sc = ld_u16(w.scales + (size_t)row * (g.cols / 16) + c * 8 + 2 * j);
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            r.sc = ld_u16(w.codes + tiled_nvs_off(g, row, c, j));
        }
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int) {
        return {e4m3_ref_to_f32(r.sc & 0xFF), e4m3_ref_to_f32(r.sc >> 8)};
    }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int seg, const float* x, float) {
        uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int n = 0; n < 8; n += 2) {
            a = __builtin_fmaf(fp4_to_f32((w0 >> (4 * n)) & 0xF), x[n], a);
            b = __builtin_fmaf(fp4_to_f32((w0 >> (4 * n + 4)) & 0xF), x[n + 1], b);
            a = __builtin_fmaf(fp4_to_f32((w1 >> (4 * n)) & 0xF), x[8 + n], a);
            b = __builtin_fmaf(fp4_to_f32((w1 >> (4 * n + 4)) & 0xF), x[8 + n + 1], b);
        }
        return (seg ? d.s1 : d.s0) * (a + b);
    }
    // fp16 activations, permuted in LDS in groups of 8 (see stage_x_h)
    static constexpr int PERM = 8;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        const uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        const uint4 xa = xh[0], xb = xh[1];
        float a = 0.0f, b = 0.0f;
        a = dot2(fp4_pair(w0, 0), xa.x, a);
        b = dot2(fp4_pair(w0, 1), xa.y, b);
        a = dot2(fp4_pair(w0, 2), xa.z, a);
        b = dot2(fp4_pair(w0, 3), xa.w, b);
        a = dot2(fp4_pair(w1, 0), xb.x, a);
        b = dot2(fp4_pair(w1, 1), xb.y, b);
        a = dot2(fp4_pair(w1, 2), xb.z, a);
        b = dot2(fp4_pair(w1, 3), xb.w, b);
        return (seg ? d.s1 : d.s0) * ((a + b) * kTwo14);
    }
};

template <int LAYOUT>
struct FmtQ4K {
    static constexpr int FMT = TITAN_Q4_K, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 2, SEGW = 16;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q, hdr; };
    struct Dec { float ds0, dm0, ds1, dm1; };
    // Chunk c is half-block c&1 of block c>>1; slot j holds qs bytes
    // [64(c&1) + 16j, +16): 64-element group c4 = 2(c&1) + (j>>1), elements
    // l0 = 16(j&1) .. +15 (low nibbles, sub-block 2*c4) and 32 + l0 ..
    // (high nibbles, sub-block 2*c4 + 1).
    TQ_DEV static int seg_col(int j, int seg) { return 64 * (j >> 1) + 16 * (j & 1) + 32 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int blk = c >> 1;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            const uint8_t* bp = w.codes + ((size_t)row * g.nblk + blk) * 144;
            r.hdr = ld_u128(bp);
            r.q = ld_u128(bp + 16 + 64 * (c & 1) + 16 * j);
        } else {
            r.hdr = ld_u128(w.codes + tiled_q4k_hdr_off(g, row, blk));
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
        }
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int c, int j) {
        float d = f16_to_f32(r.hdr.x & 0xFFFF), dmin = f16_to_f32(r.hdr.x >> 16);
        int c4 = 2 * (c & 1) + (j >> 1);
        uint32_t sc, m;
        Dec o;
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * c4, sc, m);
        o.ds0 = d * (float)sc;
        o.dm0 = dmin * (float)m;
        q4k_scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * c4 + 1, sc, m);
        o.ds1 = d * (float)sc;
        o.dm1 = dmin * (float)m;
        return o;
    }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int seg, const float* x, float sx) {
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float a = 0.0f, b = 0.0f;
        int sh = seg ? 4 : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t v = (ws[i] >> sh) & 0x0F0F0F0Fu;
            a = __builtin_fmaf((float)(v & 0xFF), x[4 * i], a);
            b = __builtin_fmaf((float)((v >> 8) & 0xFF), x[4 * i + 1], b);
            a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[4 * i + 2], a);
            b = __builtin_fmaf((float)(v >> 24), x[4 * i + 3], b);
        }
        float ds = seg ? d.ds1 : d.ds0, dm = seg ? d.dm1 : d.dm0;
        return __builtin_fmaf(ds, a + b, -dm * sx);
    }
    // fp16 activations, permuted in LDS in groups of 4 (see stage_x_h)
    static constexpr int PERM = 4;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        // word i = bytes 4i..4i+3 (elements 4i..4i+3 of the run): bytes
        // (0, 2) and (1, 3) pair with x (0, 2) / (1, 3); high nibbles x16
        const uint32_t mask = seg ? 0x00F000F0u : 0x000F000Fu;
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const uint4 xv = xh[i >> 1];
            a = dot2(ws[i] & mask, xv.x, a);
            b = dot2((ws[i] >> 8) & mask, xv.y, b);
            a = dot2(ws[i + 1] & mask, xv.z, a);
            b = dot2((ws[i + 1] >> 8) & mask, xv.w, b);
        }
        const float v = (a + b) * (seg ? kTwo24 / 16.0f : kTwo24);
        const float ds = seg ? d.ds1 : d.ds0, dm = seg ? d.dm1 : d.dm0;
        return __builtin_fmaf(ds, v, -dm * sx);
    }
};

template <int LAYOUT>
struct FmtQ3K {
    // Tiled layout only (110-byte ggml blocks are not 16-byte aligned).
    static constexpr int FMT = TITAN_Q3_K, CHUNK_COLS = 256, SLOT_COLS = 64;
    static constexpr int SEGS = 4, SEGW = 16;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q, hm; uint32_t s0, s1, s2, dh; };
    struct Dec { float dsc[4]; int hsh; };
    // Chunk c = block c; slot j holds qs bytes [16j, +16): half h = j>>1,
    // positions l = 16(j&1) + i; segment jj (shift 2jj) covers elements
    // 128h + 32jj + l, scale index 8h + 2jj + (j&1), hmask bit 4h + jj of
    // hmask[l].
    TQ_DEV static int seg_col(int j, int jj) { return 128 * (j >> 1) + 32 * jj + 16 * (j & 1); }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
        r.hm = ld_u128(w.codes + tiled_q3k_hmask_off(g, row, c, j & 1));
        const uint8_t* sp = w.codes + tiled_q3k_sc_off(g, row, c);
        r.s0 = ld_u32(sp);
        r.s1 = ld_u32(sp + 4);
        r.s2 = ld_u32(sp + 8);
        r.dh = ld_u16(w.codes + tiled_q3k_d_off(g, row, c));
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw& r, int, int j) {
        Dec o;
        float d = f16_to_f32(r.dh);
        int h = j >> 1;
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
            o.dsc[jj] = d * (float)q3k_scale(r.s0, r.s1, r.s2, 8 * h + 2 * jj + (j & 1));
        o.hsh = 4 * h;
        return o;
    }
    TQ_DEV static float seg_dot(const Raw& r, const Dec& d, int jj, const float* x, float sx) {
        uint32_t qs[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t hs[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w};
        float a = 0.0f, b = 0.0f;
        int hb = d.hsh + jj;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // 3-bit code u = q2 + 4*hbit; value = u - 4
            uint32_t v = ((qs[i] >> (2 * jj)) & 0x03030303u) | (((hs[i] >> hb) & 0x01010101u) << 2);
            a = __builtin_fmaf((float)(v & 0xFF), x[4 * i], a);
            b = __builtin_fmaf((float)((v >> 8) & 0xFF), x[4 * i + 1], b);
            a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[4 * i + 2], a);
            b = __builtin_fmaf((float)(v >> 24), x[4 * i + 3], b);
        }
        return d.dsc[jj] * ((a + b) - 4.0f * sx);
    }
    // fp16 activations, permuted in LDS in groups of 4 (see stage_x_h)
    static constexpr int PERM = 4;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        uint32_t qs[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t hs[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w};
        const int hb = d.hsh + seg;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const uint4 xv = xh[i >> 1];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                // 3-bit code u = q2 + 4*hbit per byte; value = u - 4
                const uint32_t u = ((qs[i + k] >> (2 * seg)) & 0x03030303u) |
                                   (((hs[i + k] >> hb) & 0x01010101u) << 2);
                a = dot2(u & 0x00070007u, k ? xv.z : xv.x, a);
                b = dot2((u >> 8) & 0x00070007u, k ? xv.w : xv.y, b);
            }
        }
        return d.dsc[seg] * __builtin_fmaf(a + b, kTwo24, -4.0f * sx);
    }
};

template <int LAYOUT>
struct FmtFp8 {
    static constexpr int FMT = TITAN_FP8_E4M3, CHUNK_COLS = 64, SLOT_COLS = 16;
    static constexpr int SEGS = 1, SEGW = 16;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; };
    struct Dec {};
    TQ_DEV static int seg_col(int j, int) { return 16 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            r.q = ld_u128(w.codes + (size_t)row * w.g.row_code_bytes + c * 64 + j * 16);
        else
            r.q = ld_u128(w.codes + tiled_code_off(w.g, row, c, j));
    }
    TQ_DEV static Dec decode(const WDesc&, const Raw&, int, int) { return {}; }
    TQ_DEV static float seg_dot(const Raw& r, const Dec&, int, const float* x, float) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            a = __builtin_fmaf(e4m3_ocp_to_f32(byte_of(r.q, i)), x[i], a);
            b = __builtin_fmaf(e4m3_ocp_to_f32(byte_of(r.q, i + 1)), x[i + 1], b);
        }
        return a + b;
    }
    // fp16 activations, permuted in LDS in groups of 4 (see stage_x_h)
    static constexpr int PERM = 4;
    TQ_DEV static float seg_dot_h(const Raw& r, const Dec& d, int seg, const uint4* xh, float sx) {
        // e4m3 byte -> fp16 bits by shifting: value * 2^-8, exact (the two
        // NaN codes are not produced by quantizers and are not special-cased)
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const uint4 xv = xh[i >> 1];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const uint32_t w = ws[i + k], t = w >> 8;
                const uint32_t p0 = ((w & 0x007F007Fu) << 7) | ((w & 0x00800080u) << 8);
                const uint32_t p1 = ((t & 0x007F007Fu) << 7) | ((t & 0x00800080u) << 8);
                a = dot2(p0, k ? xv.z : xv.x, a);
                b = dot2(p1, k ? xv.w : xv.y, b);
            }
        }
        return (a + b) * 256.0f;
    }
};

}  // namespace tq
