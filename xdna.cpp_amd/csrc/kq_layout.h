// Resident layout of K-quant and IQ rows, shared by host and device code.
//
// A ggml row of these types is B superblocks of 256 values, each a packed
// struct of a few fields (codes, high bits, signs, scales, fp16 d).  The
// resident row keeps the same bytes in another order; the map is a row-local
// byte permutation, so any byte range of the ggml encoding can be scattered
// or gathered on its own.  The GEMV kernels give each superblock 8 lanes
// (slice s = 0..7 of its 256 values) and a wavefront 8 superblocks per step,
// and what costs is the number of load instructions per lane, so the layout
// is chosen per type to minimise them:
//
//  * plane layout (Q4_K, Q5_K, IQ4_XS: one 16-byte field per lane already):
//      [field 0 of blocks 0..B-1][field 1 of blocks 0..B-1]...
//    planes ordered by decreasing record size;
//  * group layout (Q3_K, Q6_K, IQ3_S, IQ3_XXS, IQ2_S): the row in groups of
//    up to 8 superblocks (g in the last group), each group a run of
//    sections: first the lane records -- for slice s of superblock bl the
//    bytes that lane alone reads, R bytes at R * (s * g + bl), so the 64
//    lanes of a step read one contiguous span with one load -- then
//    per-superblock sections (scales), then the fp16 d of the g superblocks.
//
// Rows are B * block_bytes long; for the group types the block size is
// 2 mod 4, so with B odd every other row starts 2 mod 4.  On such rows the
// d section of the last group (2g bytes, g odd) moves to the front of the
// row, which realigns every other section to 4 (the plane layout does the
// same with the whole d plane, always its last plane).
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
    KqField f[5];  // plane types: resident plane order; group types: ggml fields
    bool grouped;  // group layout (kq_group_offset) instead of planes
};

// Plane order per type (largest records first).
//   Q4_K   144: qs[128]@16, head[16]@0 (d, dmin, scales[12])
//   Q5_K   176: qs[128]@48, qh[32]@16, head[16]@0
//   IQ4_XS 136: qs[128]@8, head[8]@0 (d, scales_h, scales_l[4])
// The group types list their ggml fields here (f[] tiles the block); their
// resident order is kq_group_offset below.
//   Q3_K   110: hmask[32]@0, qs[64]@32, scales[12]@96, d[2]@108
//   Q6_K   210: ql[128]@0, qh[64]@128, scales[16]@192, d[2]@208
//   IQ3_S  110: d[2]@0, qs[64]@2, qh[8]@66, signs[32]@74, scales[4]@106
//   IQ3_XXS 98: d[2]@0, qs[64]@2, scales_and_signs[32]@66
//   IQ2_S   82: d[2]@0, qs[32]@2, signs[32]@34, qh[8]@66, scales[8]@74
MI355X_HD constexpr KqLayout kq_layout(int type) {
    switch (type) {
    case 12: return {12, 144, 2, {{16, 128}, {0, 16}}, false};
    case 13: return {13, 176, 3, {{48, 128}, {16, 32}, {0, 16}}, false};
    case 23: return {23, 136, 2, {{8, 128}, {0, 8}}, false};
    case 11: return {11, 110, 4, {{0, 32}, {32, 64}, {96, 12}, {108, 2}}, true};
    case 14: return {14, 210, 4, {{0, 128}, {128, 64}, {192, 16}, {208, 2}}, true};
    case 21: return {21, 110, 5, {{0, 2}, {2, 64}, {66, 8}, {74, 32}, {106, 4}}, true};
    case 18: return {18, 98, 3, {{0, 2}, {2, 64}, {66, 32}}, true};
    case 22: return {22, 82, 5, {{0, 2}, {2, 32}, {34, 32}, {66, 8}, {74, 8}}, true};
    default: return {0, 0, 0, {}, false};
    }
}

// ---- group layout ----------------------------------------------------------
// Sections of a group of g superblocks, in order (offsets from the group):
//   Q3_K    lane records of 12 B: qs[8s..8s+7] (the 8 codes bytes slice s =
//             4hh + k reads), hmask[8k + 4hh .. +3] (half of the 8 high-bit
//             bytes the slice pair (k, hh = 0/1) shares); 96g
//           scales[12] per superblock at 96g + 12 bl, the low-nibble bytes
//             as two words, word kk = scales[kk], [kk + 4], [kk + 2],
//             [kk + 6] (the four scales of slices 2kk, 2kk + 1, 4 + 2kk,
//             5 + 2kk, in the order their high bits sit in scales[8..11]),
//             then scales[8..11]; d at 108g + 2 bl
//   Q6_K    lane records of 24 B: ql[64hh + 8k ..+7], ql[64hh + 32 + 8k ..+7],
//             qh[32hh + 8k ..+7]; 192g
//           scale words per superblock at 192g + 16 bl: word 2hh + kk holds
//             scales[8hh + kk + 2j], j = 0..3 (the four scales of slices
//             4hh + 2kk, 4hh + 2kk + 1); d at 208g + 2 bl
//   IQ3_S   lane records of 12 B: qs[8s..8s+7], signs[4s..4s+3]; 96g
//           qh[s] at 96g + (s g + bl); scales[4] at 104g + 4 bl;
//           d at 108g + 2 bl
//   IQ3_XXS lane records of 12 B: qs[8s..8s+7], scales_and_signs[4s..4s+3];
//           d at 96g + 2 bl
//   IQ2_S   lane records of 8 B: qs[4s..4s+3], signs[4s..4s+3]; 64g
//           lane pairs of 2 B: qh[s], scales[s] at 64g + 2 (s g + bl);
//           d at 80g + 2 bl
// Superblock blk sits in group blk / 8 at bl = blk % 8.

// Group geometry of superblock `blk` in a row of B superblocks.
struct KqGroupPos {
    uint64_t base;  // start of the group's sections in the row
    uint32_t g;     // superblocks in the group
    uint32_t bl;    // superblock inside the group
    uint64_t d;     // offset of the superblock's fp16 d
};

MI355X_HD constexpr KqGroupPos kq_group_pos(int block_bytes, uint64_t blk, uint64_t B, bool flipped) {
    const uint64_t t = blk >> 3;
    const uint64_t ng = (B + 7) >> 3;
    const uint32_t last_g = static_cast<uint32_t>(B - 8 * (ng - 1));
    const uint32_t g = t + 1 == ng ? last_g : 8u;
    const uint32_t bl = static_cast<uint32_t>(blk & 7);
    const uint64_t base = (flipped ? 2u * last_g : 0u) + t * 8u * static_cast<uint64_t>(block_bytes);
    const uint64_t d = flipped && t + 1 == ng ? 2u * bl : base + static_cast<uint64_t>(block_bytes - 2) * g + 2u * bl;
    return {base, g, bl, d};
}

// Offset inside the row of ggml byte `e` of block `blk` (group types).
MI355X_HD constexpr uint64_t kq_group_offset(int type, uint64_t blk, int e, uint64_t B, bool flipped) {
    const int bb = type == 11 || type == 21 ? 110 : type == 14 ? 210 : type == 18 ? 98 : 82;
    const KqGroupPos q = kq_group_pos(bb, blk, B, flipped);
    const uint64_t g = q.g, bl = q.bl;
    auto lane = [&](int s) -> uint64_t { return static_cast<uint64_t>(s) * g + bl; };
    switch (type) {
    case 11:  // Q3_K
        if (e < 32) {  // hmask: byte 8k + 4hh + j of slice 4hh + k
            const int k = e >> 3, hh = (e >> 2) & 1, j = e & 3;
            return q.base + 12 * lane(4 * hh + k) + 8 + j;
        }
        if (e < 96) return q.base + 12 * lane((e - 32) >> 3) + ((e - 32) & 7);
        if (e < 104) {  // low-nibble byte kk + 2j: word kk, byte 0, 2, 1, 3 for j = 0..3
            const int i = e - 96, kk = i & 1, j = i >> 1;
            return q.base + 96 * g + 12 * bl + 4 * kk + ((j & 1) << 1) + (j >> 1);
        }
        if (e < 108) return q.base + 96 * g + 12 * bl + (e - 96);
        return q.d + (e - 108);
    case 14:  // Q6_K
        if (e < 128) {
            const int hh = e >> 6, w = e & 63, half = w >> 5, k = (w & 31) >> 3, j = w & 7;
            return q.base + 24 * lane(4 * hh + k) + 8 * half + j;
        }
        if (e < 192) {
            const int p = e - 128, hh = p >> 5, k = (p & 31) >> 3, j = p & 7;
            return q.base + 24 * lane(4 * hh + k) + 16 + j;
        }
        if (e < 208) {
            const int i = e - 192, hh = i >> 3, kk = i & 1, j = (i & 7) >> 1;
            return q.base + 192 * g + 16 * bl + 4 * (2 * hh + kk) + j;
        }
        return q.d + (e - 208);
    case 21:  // IQ3_S
        if (e < 2) return q.d + e;
        if (e < 66) return q.base + 12 * lane((e - 2) >> 3) + ((e - 2) & 7);
        if (e < 74) return q.base + 96 * g + lane(e - 66);
        if (e < 106) return q.base + 12 * lane((e - 74) >> 2) + 8 + ((e - 74) & 3);
        return q.base + 104 * g + 4 * bl + (e - 106);
    case 18:  // IQ3_XXS
        if (e < 2) return q.d + e;
        if (e < 66) return q.base + 12 * lane((e - 2) >> 3) + ((e - 2) & 7);
        return q.base + 12 * lane((e - 66) >> 2) + 8 + ((e - 66) & 3);
    default:  // IQ2_S
        if (e < 2) return q.d + e;
        if (e < 34) return q.base + 8 * lane((e - 2) >> 2) + ((e - 2) & 3);
        if (e < 66) return q.base + 8 * lane((e - 34) >> 2) + 4 + ((e - 34) & 3);
        if (e < 74) return q.base + 64 * g + 2 * lane(e - 66);
        return q.base + 64 * g + 2 * lane(e - 74) + 1;
    }
}

// A row flips when its first byte sits at an address that is 2 mod 4; the
// tensor base is at least 4-aligned, so this depends only on the row index.
MI355X_HD constexpr bool kq_row_flipped(uint64_t row_addr) { return (row_addr & 3) == 2; }

// Start of plane i inside a row of B blocks (plane types).
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
    if (L.grouped) return kq_group_offset(L.type, blk, e, B, flipped);
    for (int i = 0; i < L.nfields; ++i) {
        const int off = L.f[i].off, len = L.f[i].len;
        if (e >= off && e < off + len) return kq_plane_start(L, i, B, flipped) + blk * len + (e - off);
    }
    return 0;  // unreachable for a valid layout (fields tile the block)
}

}  // namespace mi355x
