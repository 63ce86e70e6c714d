// rlq_layout.hpp - device layout of weights kept in HBM.
//
// Rows are grouped into tiles of 16 (the N dimension of one
// v_mfma_i32_16x16x64_i8); the last tile is zero-padded.  For every
// (tile, block) the sixteen rows' GGUF blocks are rearranged into one
// contiguous chunk whose 16-byte pieces sit in the order the 64 lanes of a
// wave load them, so each load instruction of the decode kernels reads 1 KB
// (or 256 B for per-row headers) of consecutive bytes.  Lane l of a wave
// works on row n = l % 16 and K quarter kq = l / 16 of the chunk.
//
// Q4_K, chunk of 2304 B per (tile, block):
//   [P*1024 + l*16, +16)  qs bytes 32g + q45_pos_of_slot(16h + s), s = 0..15, of
//                         row n, where P = 0, 1, g = 2P + kq/2, h = kq%2 (low
//                         nibbles: sub-block 2g, high nibbles: sub-block
//                         2g+1).  Slot 16h + 4k + i holds position
//                         4h + k + 8i of the sub-block, so each 4-byte word
//                         of a lane holds the four values of one lane class
//                         j % 8 = 4h + k (the reference's eight accumulators,
//                         matvec_extra.rs:223-294)
//   [2048 + n*16, +16)    d, dmin, scales[12] of row n (GGUF bytes 0..15)
// Q6_K, chunk of 3360 B per (tile, block):
//   [h*1024 + l*16, +16)  ql bytes 32kq + 16h .. +15 of row n
//   [2048 + n*64, +64)    qh[64] of row n
//   [3072 + n*16, +16)    scales[16] of row n
//   [3328 + n*2, +2)      d of row n
// Q5_K, chunk of 2816 B per (tile, block): the Q4_K pieces plus qh
//   [P*1024 + l*16, +16)  qs bytes of row n (GGUF bytes 48..) with the Q4_K
//                         mapping of P, g, h and slots
//   [2048 + n*32, +32)    qh[32] of row n (GGUF bytes 16..47), byte p at slot
//                         q45_slot_of_pos(p)
//   [2560 + n*16, +16)    d, dmin, scales[12] of row n (GGUF bytes 0..15)
// Q3_K, chunk of 1760 B per (tile, block):
//   [l*16, +16)           qs bytes 16kq .. +15 of row n (GGUF bytes 32..95)
//   [1024 + n*32, +32)    hmask[32] of row n (GGUF bytes 0..31)
//   [1536 + n*12, +12)    scales[12] of row n (GGUF bytes 96..107)
//   [1728 + n*2, +2)      d of row n (GGUF bytes 108..109)
// Q2_K, chunk of 1344 B per (tile, block):
//   [l*16, +16)           qs bytes 16kq .. +15 of row n (GGUF bytes 16..79)
//   [1024 + n*16, +16)    scales[16] of row n (GGUF bytes 0..15)
//   [1280 + n*4, +4)      d, dmin of row n (GGUF bytes 80..83)
// Q8_0, chunk of 1088 B per (tile, block pair p):
//   [l*16, +16)           qs bytes 16(kq%2) .. +15 of block 2p + kq/2, row n
//   [1024 + n*4, +4)      d of blocks 2p and 2p+1 of row n (a missing
//                         block 2p+1, when the row has an odd block count,
//                         is all zero)
#pragma once

#include <stdint.h>

namespace rlq {

constexpr uint32_t kTileRows = 16;
constexpr uint32_t kQ4KChunk = 2304;
constexpr uint32_t kQ6KChunk = 3360;
constexpr uint32_t kQ80Chunk = 1088;
constexpr uint32_t kQ5KChunk = 2816;
constexpr uint32_t kQ3KChunk = 1760;
constexpr uint32_t kQ2KChunk = 1344;

__host__ __device__ inline uint64_t layout_tiles(uint64_t rows) { return (rows + kTileRows - 1) / kTileRows; }

// Q4_K / Q5_K slot order within a 32-value sub-block: slot 16h + 4k + i
// holds position 4h + k + 8i (h, k, i = the lane half, the word, the byte).
__host__ __device__ constexpr uint32_t q45_pos_of_slot(uint32_t w) {
    return 4 * (w >> 4) + ((w >> 2) & 3u) + 8 * (w & 3u);
}
__host__ __device__ constexpr uint32_t q45_slot_of_pos(uint32_t p) {
    return 16 * ((p >> 2) & 1u) + 4 * (p & 3u) + (p >> 3);
}

// Chunks per tile (blocks, or block pairs for Q8_0) and chunk size.
__host__ __device__ inline uint64_t layout_chunks_per_tile(uint32_t t, uint64_t cols) {
    return t == 8 ? (cols / 32 + 1) / 2 : cols / 256;
}
__host__ __device__ inline uint64_t layout_chunk_bytes(uint32_t t) {
    switch (t) {
        case 10: return kQ2KChunk;
        case 11: return kQ3KChunk;
        case 12: return kQ4KChunk;
        case 13: return kQ5KChunk;
        case 14: return kQ6KChunk;
        default: return kQ80Chunk;
    }
}
__host__ __device__ inline uint64_t layout_bytes(uint32_t t, uint64_t rows, uint64_t cols) {
    return layout_tiles(rows) * layout_chunks_per_tile(t, cols) * layout_chunk_bytes(t);
}

// Offset in the device layout of byte `byte` of GGUF block `blk` of row `row`
// (nb = GGUF blocks per row).
__host__ __device__ inline uint64_t layout_offset(uint32_t t, uint64_t row, uint64_t blk, uint32_t byte,
                                                  uint64_t nb) {
    const uint64_t tile = row / kTileRows;
    const uint32_t n = (uint32_t)(row % kTileRows);
    if (t == 12) {
        const uint64_t base = (tile * nb + blk) * kQ4KChunk;
        if (byte < 16) return base + 2048 + n * 16 + byte;
        const uint32_t q = byte - 16, g = q / 32, w = q45_slot_of_pos(q % 32), h = w / 16, i = w % 16;
        const uint32_t P = g / 2, kq = 2 * (g % 2) + h;
        return base + P * 1024 + (16 * kq + n) * 16 + i;
    }
    if (t == 13) {
        const uint64_t base = (tile * nb + blk) * kQ5KChunk;
        if (byte < 16) return base + 2560 + n * 16 + byte;
        if (byte < 48) return base + 2048 + n * 32 + q45_slot_of_pos(byte - 16);
        const uint32_t q = byte - 48, g = q / 32, w = q45_slot_of_pos(q % 32), h = w / 16, i = w % 16;
        const uint32_t P = g / 2, kq = 2 * (g % 2) + h;
        return base + P * 1024 + (16 * kq + n) * 16 + i;
    }
    if (t == 11) {
        const uint64_t base = (tile * nb + blk) * kQ3KChunk;
        if (byte < 32) return base + 1024 + n * 32 + byte;
        if (byte < 96) {
            const uint32_t q = byte - 32;
            return base + (16 * (q / 16) + n) * 16 + q % 16;
        }
        if (byte < 108) return base + 1536 + n * 12 + (byte - 96);
        return base + 1728 + n * 2 + (byte - 108);
    }
    if (t == 10) {
        const uint64_t base = (tile * nb + blk) * kQ2KChunk;
        if (byte < 16) return base + 1024 + n * 16 + byte;
        if (byte < 80) {
            const uint32_t q = byte - 16;
            return base + (16 * (q / 16) + n) * 16 + q % 16;
        }
        return base + 1280 + n * 4 + (byte - 80);
    }
    if (t == 14) {
        const uint64_t base = (tile * nb + blk) * kQ6KChunk;
        if (byte < 128) {
            const uint32_t kq = byte / 32, w = byte % 32, h = w / 16, i = w % 16;
            return base + h * 1024 + (16 * kq + n) * 16 + i;
        }
        if (byte < 192) return base + 2048 + n * 64 + (byte - 128);
        if (byte < 208) return base + 3072 + n * 16 + (byte - 192);
        return base + 3328 + n * 2 + (byte - 208);
    }
    const uint64_t np = (nb + 1) / 2, p = blk / 2;
    const uint32_t which = (uint32_t)(blk % 2);
    const uint64_t base = (tile * np + p) * kQ80Chunk;
    if (byte < 2) return base + 1024 + n * 4 + 2 * which + byte;
    const uint32_t j = byte - 2, kq = 2 * which + j / 16, i = j % 16;
    return base + (16 * kq + n) * 16 + i;
}

}  // namespace rlq
