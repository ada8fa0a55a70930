// repack.cpp -- loader-side repack between the reference byte layout and the
// gfx950 tiled layout (host only; a byte permutation, exactly invertible).
//
// Hook point in the reference: between the pread of a tensor and its H2D copy
// (loader.cpp:434-472 read_tensor_gpu, gguf_loader.cpp:321-342, and the NVFP4
// expert staging of moe.cpp:613-724).
#include <string.h>

#include <vector>

#include "common.h"
#include "layout.h"

namespace {

using tq::Geo;

// Pointer to row r's code bytes [64c .. 64c+63] in the REF layout, copied into
// `tmp` for K-quants (whose qs arrays are interleaved with block headers).
struct RefRowCodes {
    const Geo& g;
    const uint8_t* codes;
    std::vector<uint8_t> tmp;
    explicit RefRowCodes(const Geo& geo, const void* c)
        : g(geo), codes((const uint8_t*)c), tmp((size_t)geo.row_code_bytes) {}
    const uint8_t* row(int r) {
        if (g.fmt == TITAN_Q4_K || g.fmt == TITAN_Q3_K) {
            int bb = tq::kquant_block_bytes(g.fmt), qsb = g.fmt == TITAN_Q4_K ? 128 : 64,
                qso = g.fmt == TITAN_Q4_K ? 16 : 32;
            for (int b = 0; b < g.nblk; b++)
                memcpy(&tmp[(size_t)b * qsb], codes + ((size_t)r * g.nblk + b) * bb + qso, qsb);
            return tmp.data();
        }
        return codes + (size_t)r * g.row_code_bytes;
    }
};

int check(int fmt, int rows, int cols, int gs, size_t* need) {
    *need = tq::tiled_total_bytes(fmt, rows, cols, gs);
    return *need ? TITAN_OK : TITAN_ERR_UNSUPPORTED;
}

}  // namespace

extern "C" size_t titan_tiled_bytes(int format, int rows, int cols, int group_size) {
    return tq::tiled_total_bytes(format, rows, cols, group_size);
}

extern "C" int titan_repack_host(int fmt, int rows, int cols, int gs, const void* codes,
                                 const void* scales, const void* biases, void* tiled,
                                 size_t tiled_bytes) {
    size_t need;
    if (!codes || !tiled) return TITAN_ERR_INVALID_ARG;
    if (int st = check(fmt, rows, cols, gs, &need)) return st;
    if (tiled_bytes < need) return TITAN_ERR_INVALID_ARG;
    bool needs_s = fmt == TITAN_INT4 || fmt == TITAN_INT2 || fmt == TITAN_FP4 || fmt == TITAN_NVFP4;
    bool needs_b = fmt == TITAN_INT4 || fmt == TITAN_INT2;
    if ((needs_s && !scales) || (needs_b && !biases)) return TITAN_ERR_INVALID_ARG;

    Geo g = tq::make_geo(fmt, rows, cols, gs);
    uint8_t* out = (uint8_t*)tiled;
    memset(out, 0, need);  // padding slots read as zero
    RefRowCodes rc(g, codes);
    for (int r = 0; r < rows; r++) {
        const uint8_t* src = rc.row(r);
        for (int b = 0; b < g.row_code_bytes; b += 4)
            memcpy(out + tq::tiled_code_byte(g, r, b), src + b, 4);
    }
    const uint16_t* s16 = (const uint16_t*)scales;
    const uint16_t* b16 = (const uint16_t*)biases;
    const uint8_t* s8 = (const uint8_t*)scales;
    const uint8_t* blocks = (const uint8_t*)codes;
    for (int r = 0; r < rows; r++) {
        switch (fmt) {
            case TITAN_INT4:
            case TITAN_INT2:
                for (int q = 0; q < g.ngroups; q++) {
                    uint32_t v = (uint32_t)s16[(size_t)r * g.ngroups + q] |
                                 ((uint32_t)b16[(size_t)r * g.ngroups + q] << 16);
                    const int s0 = tq::tiled_sb_slot_of(g, q), n = tq::tiled_sb_copies(g);
                    for (int k = 0; k < n; k++) memcpy(out + tq::tiled_sb_slot_off(g, r, s0 + k), &v, 4);
                }
                break;
            case TITAN_FP4:
                for (int q = 0; q < g.ngroups; q++)
                    memcpy(out + tq::tiled_fp4s_off(g, r, q), &s16[(size_t)r * g.ngroups + q], 2);
                break;
            case TITAN_NVFP4:
                for (int c = 0; c < g.nchunks; c++)
                    memcpy(out + tq::tiled_nvs_off(g, r, c), s8 + (size_t)r * (cols / 16) + c * 8, 8);
                break;
            case TITAN_Q4_K:
                for (int b = 0; b < g.nblk; b++)
                    memcpy(out + tq::tiled_q4k_hdr_off(g, r, b),
                           blocks + ((size_t)r * g.nblk + b) * 144, 16);
                break;
            case TITAN_Q3_K:
                for (int b = 0; b < g.nblk; b++) {
                    const uint8_t* blk = blocks + ((size_t)r * g.nblk + b) * 110;
                    for (int j = 0; j < 4; j++)
                        for (int hi = 0; hi < 2; hi++) {  // hmask words j, 4 + j
                            uint32_t w;
                            memcpy(&w, blk + 16 * hi + 4 * j, 4);
                            w = tq::q3k_hm_pack(w);
                            memcpy(out + tq::tiled_q3k_hmask_off(g, r, b, j) + 4 * hi, &w, 4);
                        }
                    memcpy(out + tq::tiled_q3k_sc_off(g, r, b), blk + 96, 12);
                    memcpy(out + tq::tiled_q3k_d_off(g, r, b), blk + 108, 2);
                }
                break;
            default:
                break;
        }
    }
    return TITAN_OK;
}

extern "C" int titan_unpack_host(int fmt, int rows, int cols, int gs, const void* tiled,
                                 void* codes, void* scales, void* biases) {
    size_t need;
    if (!codes || !tiled) return TITAN_ERR_INVALID_ARG;
    if (int st = check(fmt, rows, cols, gs, &need)) return st;
    bool needs_s = fmt == TITAN_INT4 || fmt == TITAN_INT2 || fmt == TITAN_FP4 || fmt == TITAN_NVFP4;
    bool needs_b = fmt == TITAN_INT4 || fmt == TITAN_INT2;
    if ((needs_s && !scales) || (needs_b && !biases)) return TITAN_ERR_INVALID_ARG;

    Geo g = tq::make_geo(fmt, rows, cols, gs);
    const uint8_t* in = (const uint8_t*)tiled;
    uint8_t* c8 = (uint8_t*)codes;
    std::vector<uint8_t> row((size_t)g.row_code_bytes);
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < g.row_code_bytes; b += 4)
            memcpy(&row[(size_t)b], in + tq::tiled_code_byte(g, r, b), 4);
        if (fmt == TITAN_Q4_K || fmt == TITAN_Q3_K) {
            int bb = tq::kquant_block_bytes(fmt), qsb = fmt == TITAN_Q4_K ? 128 : 64,
                qso = fmt == TITAN_Q4_K ? 16 : 32;
            for (int b = 0; b < g.nblk; b++)
                memcpy(c8 + ((size_t)r * g.nblk + b) * bb + qso, &row[(size_t)b * qsb], qsb);
        } else {
            memcpy(c8 + (size_t)r * g.row_code_bytes, row.data(), g.row_code_bytes);
        }
    }
    uint16_t* s16 = (uint16_t*)scales;
    uint16_t* b16 = (uint16_t*)biases;
    uint8_t* s8 = (uint8_t*)scales;
    for (int r = 0; r < rows; r++) {
        switch (fmt) {
            case TITAN_INT4:
            case TITAN_INT2:
                for (int q = 0; q < g.ngroups; q++) {
                    uint32_t v;
                    memcpy(&v, in + tq::tiled_sb_off(g, r, q), 4);
                    s16[(size_t)r * g.ngroups + q] = (uint16_t)(v & 0xFFFF);
                    b16[(size_t)r * g.ngroups + q] = (uint16_t)(v >> 16);
                }
                break;
            case TITAN_FP4:
                for (int q = 0; q < g.ngroups; q++)
                    memcpy(&s16[(size_t)r * g.ngroups + q], in + tq::tiled_fp4s_off(g, r, q), 2);
                break;
            case TITAN_NVFP4:
                for (int c = 0; c < g.nchunks; c++)
                    memcpy(s8 + (size_t)r * (cols / 16) + c * 8, in + tq::tiled_nvs_off(g, r, c), 8);
                break;
            case TITAN_Q4_K:
                for (int b = 0; b < g.nblk; b++)
                    memcpy(c8 + ((size_t)r * g.nblk + b) * 144, in + tq::tiled_q4k_hdr_off(g, r, b), 16);
                break;
            case TITAN_Q3_K:
                for (int b = 0; b < g.nblk; b++) {
                    uint8_t* blk = c8 + ((size_t)r * g.nblk + b) * 110;
                    for (int j = 0; j < 4; j++)
                        for (int hi = 0; hi < 2; hi++) {
                            uint32_t w;
                            memcpy(&w, in + tq::tiled_q3k_hmask_off(g, r, b, j) + 4 * hi, 4);
                            w = tq::q3k_hm_unpack(w);
                            memcpy(blk + 16 * hi + 4 * j, &w, 4);
                        }
                    memcpy(blk + 96, in + tq::tiled_q3k_sc_off(g, r, b), 12);
                    memcpy(blk + 108, in + tq::tiled_q3k_d_off(g, r, b), 2);
                }
                break;
            default:
                break;
        }
    }
    return TITAN_OK;
}
