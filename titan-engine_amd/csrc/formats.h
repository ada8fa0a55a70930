// formats.h -- device-side decoders of every weight format, both layouts.
//
// Two views of each format:
//  * elem<FMT, LAYOUT>(w, row, col): the exact fp32 dequantized value, one
//    element at a time (dequant kernel, generic GEMV for ragged shapes).
//  * the fast GEMV view lives in fast.h.
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
    int gshift;  // log2(group size) (fast path: power-of-two groups only)
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
            word = ld_u32(w.codes + tiled_code_byte(g, row, (col / PER) * 4));
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
            byte = w.codes[tiled_code_byte(g, row, col / 2)];
            sc = w.codes[tiled_nvs_off(g, row, col / 128) + (col % 128) / 16];
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
            qb = w.codes[tiled_code_byte(g, row, b * 128 + 32 * c4 + l)];
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
            qb = w.codes[tiled_code_byte(g, row, b * 64 + 32 * h + l)];
            // hmask byte l: word l/4 = 4*hi + j  ->  plane entry j, half hi; its
            // bit 4h + jj at q3k_hpos(l % 4, jj, h) of the tiled word
            const uint32_t hw = ld_u32(w.codes + tiled_q3k_hmask_off(g, row, b, (l >> 2) & 3) + 4 * (l >> 4));
            hb = ((hw >> q3k_hpos(l & 3, jj, h)) & 1u) << (4 * h + jj);
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
            byte = w.codes[tiled_code_byte(g, row, col)];
        }
        return e4m3_ocp_to_f32(byte) * ((const float*)w.scales)[row];
    }
}

}  // namespace tq
