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

template <int LAYOUT>
struct FmtInt4 {
    static constexpr int FMT = TITAN_INT4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 1, SEGW = 32;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q; float s, b; };
    TQ_DEV static int seg_col(int j, int) { return 32 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = (c * 128 + 32 * j) / g.gs;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = f16_to_f32(((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp]);
            r.b = f16_to_f32(((const uint16_t*)w.biases)[(size_t)row * g.ngroups + grp]);
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            uint32_t sb = ld_u32(w.codes + tiled_sb_off(g, row, grp));
            r.s = f16_to_f32(sb & 0xFFFF);
            r.b = f16_to_f32(sb >> 16);
        }
    }
    TQ_DEV static float seg_dot(const Raw& r, int, const float* x, float sx) {
        float d = dot_nib8(r.q.x, x) + dot_nib8(r.q.y, x + 8) +
                  dot_nib8(r.q.z, x + 16) + dot_nib8(r.q.w, x + 24);
        return __builtin_fmaf(r.s, d, r.b * sx);
    }
};

template <int LAYOUT>
struct FmtFp4 {
    static constexpr int FMT = TITAN_FP4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 1, SEGW = 32;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; float s; };
    TQ_DEV static int seg_col(int j, int) { return 32 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = (c * 128 + 32 * j) / g.gs;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = f16_to_f32(((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp]);
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            r.s = f16_to_f32(ld_u16(w.codes + tiled_fp4s_off(g, row, grp)));
        }
    }
    TQ_DEV static float seg_dot(const Raw& r, int, const float* x, float) {
        float a = 0.0f, b = 0.0f;
        uint32_t ws[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int n = 0; n < 8; n += 2) {
                a = __builtin_fmaf(fp4_to_f32((ws[i] >> (4 * n)) & 0xF), x[8 * i + n], a);
                b = __builtin_fmaf(fp4_to_f32((ws[i] >> (4 * n + 4)) & 0xF), x[8 * i + n + 1], b);
            }
        return r.s * (a + b);
    }
};

template <int LAYOUT>
struct FmtInt2 {
    static constexpr int FMT = TITAN_INT2, CHUNK_COLS = 256, SLOT_COLS = 64;
    static constexpr int SEGS = 2, SEGW = 32;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q; float s, b; };
    TQ_DEV static int seg_col(int j, int seg) { return 64 * j + 32 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int grp = (c * 256 + 64 * j) / g.gs;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            r.s = f16_to_f32(((const uint16_t*)w.scales)[(size_t)row * g.ngroups + grp]);
            r.b = f16_to_f32(((const uint16_t*)w.biases)[(size_t)row * g.ngroups + grp]);
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            uint32_t sb = ld_u32(w.codes + tiled_sb_off(g, row, grp));
            r.s = f16_to_f32(sb & 0xFFFF);
            r.b = f16_to_f32(sb >> 16);
        }
    }
    TQ_DEV static float seg_dot(const Raw& r, int seg, const float* x, float sx) {
        uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        float d = dot_crumb16(w0, x) + dot_crumb16(w1, x + 16);
        return __builtin_fmaf(r.s, d, r.b * sx);
    }
};

template <int LAYOUT>
struct FmtNvfp4 {
    static constexpr int FMT = TITAN_NVFP4, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 2, SEGW = 16;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; float s0, s1; };
    TQ_DEV static int seg_col(int j, int seg) { return 32 * j + 16 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        uint32_t sc;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            r.q = ld_u128(w.codes + (size_t)row * g.row_code_bytes + c * 64 + j * 16);
            sc = ld_u16(w.scales + (size_t)row * (g.cols / 16) + c * 8 + 2 * j);
        } else {
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
            sc = ld_u16(w.codes + tiled_nvs_off(g, row, c, j));
        }
        r.s0 = e4m3_ref_to_f32(sc & 0xFF);
        r.s1 = e4m3_ref_to_f32(sc >> 8);
    }
    TQ_DEV static float seg_dot(const Raw& r, int seg, const float* x, float) {
        uint32_t w0 = seg ? r.q.z : r.q.x, w1 = seg ? r.q.w : r.q.y;
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int n = 0; n < 8; n += 2) {
            a = __builtin_fmaf(fp4_to_f32((w0 >> (4 * n)) & 0xF), x[n], a);
            b = __builtin_fmaf(fp4_to_f32((w0 >> (4 * n + 4)) & 0xF), x[n + 1], b);
            a = __builtin_fmaf(fp4_to_f32((w1 >> (4 * n)) & 0xF), x[8 + n], a);
            b = __builtin_fmaf(fp4_to_f32((w1 >> (4 * n + 4)) & 0xF), x[8 + n + 1], b);
        }
        return (seg ? r.s1 : r.s0) * (a + b);
    }
};

template <int LAYOUT>
struct FmtQ4K {
    static constexpr int FMT = TITAN_Q4_K, CHUNK_COLS = 128, SLOT_COLS = 32;
    static constexpr int SEGS = 2, SEGW = 16;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q; float ds0, dm0, ds1, dm1; };
    // Chunk c is half-block c&1 of block c>>1; slot j holds qs bytes
    // [64(c&1) + 16j, +16): 64-element group c4 = 2(c&1) + (j>>1), elements
    // l0 = 16(j&1) .. +15 (low nibbles, sub-block 2*c4) and 32 + l0 ..
    // (high nibbles, sub-block 2*c4 + 1).
    TQ_DEV static int seg_col(int j, int seg) { return 64 * (j >> 1) + 16 * (j & 1) + 32 * seg; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        const Geo& g = w.g;
        int blk = c >> 1;
        uint4 hdr;
        if constexpr (LAYOUT == TITAN_LAYOUT_REF) {
            const uint8_t* bp = w.codes + ((size_t)row * g.nblk + blk) * 144;
            hdr = ld_u128(bp);
            r.q = ld_u128(bp + 16 + 64 * (c & 1) + 16 * j);
        } else {
            hdr = ld_u128(w.codes + tiled_q4k_hdr_off(g, row, blk));
            r.q = ld_u128(w.codes + tiled_code_off(g, row, c, j));
        }
        float d = f16_to_f32(hdr.x & 0xFFFF), dmin = f16_to_f32(hdr.x >> 16);
        int c4 = 2 * (c & 1) + (j >> 1);
        uint32_t sc, m;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * c4, sc, m);
        r.ds0 = d * (float)sc;
        r.dm0 = dmin * (float)m;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * c4 + 1, sc, m);
        r.ds1 = d * (float)sc;
        r.dm1 = dmin * (float)m;
    }
    TQ_DEV static float seg_dot(const Raw& r, int seg, const float* x, float sx) {
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
        float ds = seg ? r.ds1 : r.ds0, dm = seg ? r.dm1 : r.dm0;
        return __builtin_fmaf(ds, a + b, -dm * sx);
    }
};

template <int LAYOUT>
struct FmtQ3K {
    // Tiled layout only (110-byte ggml blocks are not 16-byte aligned).
    static constexpr int FMT = TITAN_Q3_K, CHUNK_COLS = 256, SLOT_COLS = 64;
    static constexpr int SEGS = 4, SEGW = 16;
    static constexpr bool NEEDS_SX = true;
    struct Raw { uint4 q, hm; float dsc[4]; int hsh; };
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
        uint32_t s0 = ld_u32(sp), s1 = ld_u32(sp + 4), s2 = ld_u32(sp + 8);
        float d = f16_to_f32(ld_u16(w.codes + tiled_q3k_d_off(g, row, c)));
        int h = j >> 1;
#pragma unroll
        for (int jj = 0; jj < 4; jj++) r.dsc[jj] = d * (float)q3k_scale(s0, s1, s2, 8 * h + 2 * jj + (j & 1));
        r.hsh = 4 * h;
    }
    TQ_DEV static float seg_dot(const Raw& r, int jj, const float* x, float sx) {
        uint32_t qs[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        uint32_t hs[4] = {r.hm.x, r.hm.y, r.hm.z, r.hm.w};
        float a = 0.0f, b = 0.0f;
        int hb = r.hsh + jj;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // 3-bit code u = q2 + 4*hbit; value = u - 4
            uint32_t v = ((qs[i] >> (2 * jj)) & 0x03030303u) | (((hs[i] >> hb) & 0x01010101u) << 2);
            a = __builtin_fmaf((float)(v & 0xFF), x[4 * i], a);
            b = __builtin_fmaf((float)((v >> 8) & 0xFF), x[4 * i + 1], b);
            a = __builtin_fmaf((float)((v >> 16) & 0xFF), x[4 * i + 2], a);
            b = __builtin_fmaf((float)(v >> 24), x[4 * i + 3], b);
        }
        return r.dsc[jj] * ((a + b) - 4.0f * sx);
    }
};

template <int LAYOUT>
struct FmtFp8 {
    static constexpr int FMT = TITAN_FP8_E4M3, CHUNK_COLS = 64, SLOT_COLS = 16;
    static constexpr int SEGS = 1, SEGW = 16;
    static constexpr bool NEEDS_SX = false;
    struct Raw { uint4 q; };
    TQ_DEV static int seg_col(int j, int) { return 16 * j; }
    TQ_DEV static void load(const WDesc& w, int row, int c, int j, Raw& r) {
        if constexpr (LAYOUT == TITAN_LAYOUT_REF)
            r.q = ld_u128(w.codes + (size_t)row * w.g.row_code_bytes + c * 64 + j * 16);
        else
            r.q = ld_u128(w.codes + tiled_code_off(w.g, row, c, j));
    }
    TQ_DEV static float seg_dot(const Raw& r, int, const float* x, float) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            a = __builtin_fmaf(e4m3_ocp_to_f32(byte_of(r.q, i)), x[i], a);
            b = __builtin_fmaf(e4m3_ocp_to_f32(byte_of(r.q, i + 1)), x[i + 1], b);
        }
        return a + b;
    }
};

}  // namespace tq
