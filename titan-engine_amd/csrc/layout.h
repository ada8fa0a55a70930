// layout.h -- geometry of every weight format in both layouts.
//
// Shared by the host repack (repack.cpp) and the device kernels so that the
// two can never disagree about where a byte lives.
//
// TILED layout (one buffer, all planes back to back; the same byte count as
// REF except for INT4 / INT2 scale slots, padded to whole 16-byte cells and
// repeated for groups longer than one chunk):
//   code plane   row r's code bytes (K-quants: the concatenated qs arrays of
//                its blocks) cut into 64-byte chunks of 16 words; tile t = rows
//                16t..16t+15; chunk c of tile t is 1 KiB at
//                ((t*nchunks + c) * 64 + lane) * 16, lane = 16*j + (r % 16)
//                holding words j, 4+j, 8+j, 12+j of row r's chunk (word i of
//                the lane = chunk bytes [16i + 4j, +4)).  A wave's 64 lanes
//                read one chunk of 16 rows as 1 KiB of contiguous memory, and
//                word i of the four lanes of a row covers chunk bytes
//                [16i, 16i + 16): one matrix-core k-step over contiguous
//                columns.
//   aux planes   per format, also 16-row interleaved (see tiled_* below).
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifndef TQ_HD
#define TQ_HD __host__ __device__ __forceinline__
#endif

namespace tq {

struct Geo {
    int fmt;
    int rows, cols, gs;
    int row_code_bytes;  // bytes of the code plane per row
    int nchunks;         // 64-byte chunks per row (tiled)
    int chunk_cols;      // columns covered by one 64-byte chunk
    int slot_cols;       // columns covered by one lane's 16 bytes
    int nblk;            // K-quant blocks per row
    int ngroups;         // INT4/INT2/FP4 scale groups per row
};

TQ_HD int code_bits(int fmt) {
    switch (fmt) {
        case TITAN_INT4: case TITAN_FP4: case TITAN_NVFP4: case TITAN_Q4_K: return 4;
        case TITAN_INT2: case TITAN_Q3_K: return 2;
        case TITAN_FP8_E4M3: return 8;
        default: return 0;
    }
}

TQ_HD Geo make_geo(int fmt, int rows, int cols, int gs) {
    Geo g;
    g.fmt = fmt;
    g.rows = rows;
    g.cols = cols;
    g.gs = gs;
    int bits = code_bits(fmt);
    g.row_code_bytes = bits ? (int)(((int64_t)cols * bits) / 8) : 0;
    g.nchunks = g.row_code_bytes / 64;
    g.chunk_cols = bits ? 512 / bits : 0;
    g.slot_cols = bits ? 128 / bits : 0;
    g.nblk = (fmt == TITAN_Q4_K || fmt == TITAN_Q3_K) ? cols / 256 : 0;
    g.ngroups = (gs > 0 && (fmt == TITAN_INT4 || fmt == TITAN_INT2 || fmt == TITAN_FP4))
                    ? cols / gs : 0;
    return g;
}

// Bytes per K-quant block in the REF (ggml) layout.
TQ_HD int kquant_block_bytes(int fmt) { return fmt == TITAN_Q4_K ? 144 : 110; }

// ---- TILED code plane ------------------------------------------------------
TQ_HD size_t tiled_code_off(const Geo& g, int row, int chunk, int j) {
    int t = row >> 4, r = row & 15;
    return (((size_t)t * g.nchunks + chunk) * 64 + (size_t)(j * 16 + r)) * 16;
}
TQ_HD size_t tiled_code_plane_bytes(const Geo& g) {
    return (size_t)g.rows * g.row_code_bytes;
}
// Offset of byte b (0 <= b < row_code_bytes) of row `row`'s code bytes.
TQ_HD size_t tiled_code_byte(const Geo& g, int row, int b) {
    const int c = b >> 6, w = (b & 63) >> 2;
    return tiled_code_off(g, row, c, w & 3) + 4 * (w >> 2) + (b & 3);
}

// ---- TILED aux planes (offsets from the start of the buffer) ----------------
// INT4 / INT2: u32 words (scale | bias << 16) in "slots", four slots of one
// row in one 16-byte cell at [t][slot / 4][r][slot % 4], so that a lane reads
// the scales of four chunks (groups of at least one chunk) or of one chunk
// (smaller groups) with a single 16-byte load.  Groups of at least one chunk
// have one slot per chunk (slot c = the group of chunk c; a group of n chunks
// is stored n times); smaller groups have one slot per group.
TQ_HD int tiled_sb_slots(const Geo& g) { return g.gs >= g.chunk_cols ? g.nchunks : g.ngroups; }
TQ_HD int tiled_sb_cells(const Geo& g) { return (tiled_sb_slots(g) + 3) >> 2; }
TQ_HD size_t tiled_sb_slot_off(const Geo& g, int row, int slot) {
    return tiled_code_plane_bytes(g) +
           ((((size_t)(row >> 4) * tiled_sb_cells(g) + (slot >> 2)) * 16 + (row & 15)) * 4 + (slot & 3)) * 4;
}
// first slot holding group grp, and how many slots hold it
TQ_HD int tiled_sb_slot_of(const Geo& g, int grp) {
    return g.gs >= g.chunk_cols ? grp * (g.gs / g.chunk_cols) : grp;
}
TQ_HD int tiled_sb_copies(const Geo& g) { return g.gs >= g.chunk_cols ? g.gs / g.chunk_cols : 1; }
TQ_HD size_t tiled_sb_off(const Geo& g, int row, int grp) {
    return tiled_sb_slot_off(g, row, tiled_sb_slot_of(g, grp));
}
// FP4: u16 scale at [t][group][r].
TQ_HD size_t tiled_fp4s_off(const Geo& g, int row, int grp) {
    return tiled_code_plane_bytes(g) +
           (((size_t)(row >> 4) * g.ngroups + grp) * 16 + (row & 15)) * 2;
}
// NVFP4: the 8 e4m3 scales of chunk c (128 columns) at [t][c][r] (8 bytes).
TQ_HD size_t tiled_nvs_off(const Geo& g, int row, int chunk) {
    return tiled_code_plane_bytes(g) +
           (((size_t)(row >> 4) * g.nchunks + chunk) * 16 + (row & 15)) * 8;
}
// Q4_K: 16-byte block header {d, dmin, scales[12]} at [t][blk][r].
TQ_HD size_t tiled_q4k_hdr_off(const Geo& g, int row, int blk) {
    return tiled_code_plane_bytes(g) +
           (((size_t)(row >> 4) * g.nblk + blk) * 16 + (row & 15)) * 16;
}
// Q3_K: hmask words (j, 4+j) (8 B) at [t][blk][j][r]; scales (12 B) at
// [t][blk][r]; d (2 B) at [t][blk][r].  Each tiled hmask word holds the 32
// bits of one ggml hmask word (bytes k = 0..3 of four positions, bit 4h + jj
// of byte k: half h, level jj) re-ordered for the decoder: bit (h, jj, k) at
// q3k_hpos(k, jj, h).  For h = 0, bytes 0 and 2 of level jj sit at bits
// 2jj + 2 and 2jj + 18 -- where the 3-bit code of level jj needs its high
// bit inside the fp16 halves of bytes (0, 2) -- and bytes 1, 3 one bit
// higher; h = 1 is the same pattern rotated by 8 bits.
TQ_HD int q3k_hpos(int k, int jj, int h) { return (2 * jj + 2 + (k & 1) + 16 * (k >> 1) + 8 * h) & 31; }
TQ_HD uint32_t q3k_hm_pack(uint32_t w) {
    uint32_t o = 0;
    for (int k = 0; k < 4; k++)
        for (int h = 0; h < 2; h++)
            for (int jj = 0; jj < 4; jj++) o |= ((w >> (8 * k + 4 * h + jj)) & 1u) << q3k_hpos(k, jj, h);
    return o;
}
TQ_HD uint32_t q3k_hm_unpack(uint32_t p) {
    uint32_t w = 0;
    for (int k = 0; k < 4; k++)
        for (int h = 0; h < 2; h++)
            for (int jj = 0; jj < 4; jj++) w |= ((p >> q3k_hpos(k, jj, h)) & 1u) << (8 * k + 4 * h + jj);
    return w;
}
TQ_HD size_t tiled_q3k_hmask_off(const Geo& g, int row, int blk, int j) {
    return tiled_code_plane_bytes(g) +
           ((((size_t)(row >> 4) * g.nblk + blk) * 4 + j) * 16 + (row & 15)) * 8;
}
TQ_HD size_t tiled_q3k_sc_off(const Geo& g, int row, int blk) {
    return tiled_code_plane_bytes(g) + (size_t)g.rows * g.nblk * 32 +
           (((size_t)(row >> 4) * g.nblk + blk) * 16 + (row & 15)) * 12;
}
TQ_HD size_t tiled_q3k_d_off(const Geo& g, int row, int blk) {
    return tiled_code_plane_bytes(g) + (size_t)g.rows * g.nblk * 44 +
           (((size_t)(row >> 4) * g.nblk + blk) * 16 + (row & 15)) * 2;
}

// Total bytes of the TILED buffer, or 0 if the format/shape has no tiled
// form.  Tiled weights are always served by the fast GEMV kernel, so the
// group size must also be a power of two that keeps each lane's 16-byte slot
// inside one group, and the buffer must stay below 4 GiB.
TQ_HD size_t tiled_total_bytes(int fmt, int rows, int cols, int gs) {
    if (rows <= 0 || cols <= 0 || (rows & 15)) return 0;
    Geo g = make_geo(fmt, rows, cols, gs);
    if (!g.row_code_bytes || (g.row_code_bytes & 63)) return 0;
    size_t codes = tiled_code_plane_bytes(g);
    // groups: a power of two no smaller than one lane's 16-byte slot
    const bool gs_ok = gs > 0 && cols % gs == 0 && gs % g.slot_cols == 0 && (gs & (gs - 1)) == 0;
    size_t total = 0;
    switch (fmt) {
        case TITAN_INT4:
        case TITAN_INT2:
            if (gs_ok) total = codes + (size_t)rows * tiled_sb_cells(g) * 16;
            break;
        case TITAN_FP4:
            if (gs_ok) total = codes + (size_t)rows * g.ngroups * 2;
            break;
        case TITAN_NVFP4:
            if (cols % 128 == 0) total = codes + (size_t)rows * (cols / 16);
            break;
        case TITAN_Q4_K:
            if (cols % 256 == 0) total = codes + (size_t)rows * g.nblk * 16;
            break;
        case TITAN_Q3_K:
            if (cols % 256 == 0) total = codes + (size_t)rows * g.nblk * 46;
            break;
        case TITAN_FP8_E4M3:
            total = codes;
            break;
        default:
            break;
    }
    // the kernels address the buffer with 32-bit per-lane offsets
    return total < (1ull << 32) ? total : 0;
}

}  // namespace tq
