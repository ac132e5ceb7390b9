// Resident layout of K-quant and IQ rows, shared by host and device code.
//
// A ggml row of these types is B superblocks of 256 values, each a packed
// struct of a few fields (codes, high bits, signs, scales, fp16 d).  The
// resident row keeps the same bytes, regrouped into field planes:
//   [field 0 of blocks 0..B-1][field 1 of blocks 0..B-1]...
// with the planes ordered by decreasing record size, so a lane reading one
// block's field finds it at a naturally aligned address and the lanes of a
// wavefront reading consecutive blocks read one contiguous span.  Types whose
// block size is 2 mod 4 (Q3_K, Q6_K, IQ3_S, IQ3_XXS, IQ2_S) give rows that
// start 2 mod 4 when B is odd; on such rows the 2-byte fp16 plane (always the
// last plane) moves to the front, which realigns every other plane to 4.
// The map is a row-local byte permutation, so any byte range of the ggml
// encoding can be scattered or gathered on its own.
//
// Block structs (field offsets in bytes) follow ggml's block_q*_K / block_iq*
// as restated in the reference (include/xdna/kquants.h:53-160).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MI355X_HD __host__ __device__
#else
#define MI355X_HD
#endif

namespace mi355x {

struct KqField {
    uint8_t off;  // offset of the field inside the ggml block
    uint8_t len;  // bytes per block
};

struct KqLayout {
    int type;
    int block_bytes;
    int nfields;
    KqField f[5];  // resident plane order; a 2-byte last plane flips on misaligned rows
};

// Plane order per type (largest records first).
//   Q4_K   144: qs[128]@16, head[16]@0 (d, dmin, scales[12])
//   Q5_K   176: qs[128]@48, qh[32]@16, head[16]@0
//   Q3_K   110: qs[64]@32, hmask[32]@0, scales[12]@96, d[2]@108
//   Q6_K   210: ql[128]@0, qh[64]@128, scales[16]@192, d[2]@208
//   IQ4_XS 136: qs[128]@8, head[8]@0 (d, scales_h, scales_l[4])
//   IQ3_S  110: qs[64]@2, signs[32]@74, qh[8]@66, scales[4]@106, d[2]@0
//   IQ3_XXS 98: qs[64]@2, scales_and_signs[32]@66, d[2]@0
//   IQ2_S   82: qs[32]@2, signs[32]@34, qh[8]@66, scales[8]@74, d[2]@0
MI355X_HD constexpr KqLayout kq_layout(int type) {
    switch (type) {
    case 12: return {12, 144, 2, {{16, 128}, {0, 16}}};
    case 13: return {13, 176, 3, {{48, 128}, {16, 32}, {0, 16}}};
    case 11: return {11, 110, 4, {{32, 64}, {0, 32}, {96, 12}, {108, 2}}};
    case 14: return {14, 210, 4, {{0, 128}, {128, 64}, {192, 16}, {208, 2}}};
    case 23: return {23, 136, 2, {{8, 128}, {0, 8}}};
    case 21: return {21, 110, 5, {{2, 64}, {74, 32}, {66, 8}, {106, 4}, {0, 2}}};
    case 18: return {18, 98, 3, {{2, 64}, {66, 32}, {0, 2}}};
    case 22: return {22, 82, 5, {{2, 32}, {34, 32}, {66, 8}, {74, 8}, {0, 2}}};
    default: return {0, 0, 0, {}};
    }
}

// A row flips when its first byte sits at an address that is 2 mod 4; the
// tensor base is at least 4-aligned, so this depends only on the row index.
MI355X_HD constexpr bool kq_row_flipped(uint64_t row_addr) { return (row_addr & 3) == 2; }

// Start of plane i inside a row of B blocks.
MI355X_HD constexpr uint64_t kq_plane_start(const KqLayout &L, int i, uint64_t B, bool flipped) {
    const bool has_d = L.f[L.nfields - 1].len == 2;
    if (flipped && has_d) {
        if (i == L.nfields - 1) return 0;
        uint64_t s = 2 * B;
        for (int j = 0; j < i; ++j) s += L.f[j].len * B;
        return s;
    }
    uint64_t s = 0;
    for (int j = 0; j < i; ++j) s += L.f[j].len * B;
    return s;
}

// Offset inside the row of ggml byte `e` of block `blk`.
MI355X_HD constexpr uint64_t kq_row_offset(const KqLayout &L, uint64_t blk, int e, uint64_t B, bool flipped) {
    for (int i = 0; i < L.nfields; ++i) {
        const int off = L.f[i].off, len = L.f[i].len;
        if (e >= off && e < off + len) return kq_plane_start(L, i, B, flipped) + blk * len + (e - off);
    }
    return 0;  // unreachable for a valid layout (fields tile the block)
}

}  // namespace mi355x
