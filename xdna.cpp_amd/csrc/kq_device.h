// Device-side pieces of the K-quant and IQ GEMV kernels: resident-row loads,
// per-type decode (f32 and 16-bit digit arithmetic), activation staging in
// lane-major LDS records and codebook staging.  Included by the kernel
// sources; everything sits in an anonymous namespace, one copy per source.
#pragma once

#include "device_common.h"
#include "iq3s_grid.h"
#include "kq_layout.h"
#include "mi355x-gemv.h"

#include <cstdint>

namespace mi355x {
namespace {


constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kSlices = 8;  // lanes per superblock
constexpr int kBlocksPerStep = 64 / kSlices;
// Superblocks of x staged per pass: 60 (15360 values) keeps the LDS of an
// f32 workgroup within 80 KB with the largest codebook, so two fit on a CU.
constexpr int kChunkBlocks = 60;

struct KqArgs {
    const uint8_t *W;
    int64_t N;
    int64_t row_bytes;
    int B;   // superblocks per row
    int b0;  // first superblock of this chunk
    int nb;  // superblocks in this chunk
    const float *x;
    float *y;
    int accumulate;
    const uint32_t *grid;  // device codebook (IQ3_XXS, IQ2_S), else null
};

__device__ __forceinline__ float byte_f(uint32_t w, int t) { return static_cast<float>((w >> (8 * t)) & 0xFFu); }

__device__ __forceinline__ uint32_t byte_u(uint32_t w, int t) { return (w >> (8 * t)) & 0xFFu; }

// One DPP move of an int across lanes (all lanes active).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// sum_t byte_t(codes) * x[t] for the 4 bytes of one dword
__device__ __forceinline__ float dot4(uint32_t codes, const float *x, float acc) {
    acc = fmaf(byte_f(codes, 0), x[0], acc);
    acc = fmaf(byte_f(codes, 1), x[1], acc);
    acc = fmaf(byte_f(codes, 2), x[2], acc);
    acc = fmaf(byte_f(codes, 3), x[3], acc);
    return acc;
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Row {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t P[5];  // plane types: plane starts in the row; group types: B, flip
};

__device__ __forceinline__ u32x4 ld128(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}
__device__ __forceinline__ u32x2 ld64(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}
__device__ __forceinline__ uint32_t ld32(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}
__device__ __forceinline__ uint32_t ld16(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}
__device__ __forceinline__ uint32_t ld8(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
__device__ __forceinline__ u32x3 ld96(const Row &r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b96(r.rsrc, static_cast<int>(off), 0, kNonTemporal);
}

// Buffer view of one row; rows at or past `lim` get an empty range.
template <int TYPE>
__device__ __forceinline__ Row make_row_pl(const KqArgs &a, int64_t row, int64_t lim) {
    constexpr KqLayout L = kq_layout(TYPE);
    const uint8_t *base = a.W + row * a.row_bytes;
    Row r;
    r.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0,
                                               row < lim ? static_cast<uint32_t>(a.row_bytes) : 0u, kBufferWord3);
    const bool flipped = kq_row_flipped(reinterpret_cast<uintptr_t>(base));
    if constexpr (L.grouped) {
        r.P[0] = static_cast<uint32_t>(a.B);
        r.P[1] = flipped ? 1u : 0u;
    } else {
#pragma unroll
        for (int i = 0; i < 5; ++i)
            r.P[i] = i < L.nfields ? static_cast<uint32_t>(kq_plane_start(L, i, a.B, flipped)) : 0u;
    }
    return r;
}

// Group-layout position of superblock b for slice s (kq_layout.h): the
// group's start, its size g, the lane record index s * g + bl and the fp16
// d's offset.  Row.P[0] holds B and P[1] the row's flip for these types.
struct GPos {
    uint32_t base, g, bl, m, d;
};
__device__ __forceinline__ GPos gpos(const Row &r, int bb, uint32_t b, int s) {
    const uint32_t B = r.P[0];
    const bool flipped = r.P[1] != 0;
    const uint32_t t = b >> 3;
    const uint32_t ng = (B + 7) >> 3;
    const uint32_t last_g = B - 8 * (ng - 1);
    const bool last = t + 1 == ng;
    const uint32_t g = last ? last_g : 8u;
    const uint32_t bl = b & 7;
    const uint32_t base = (flipped ? 2 * last_g : 0u) + t * 8 * static_cast<uint32_t>(bb);
    const uint32_t d = flipped && last ? 2 * bl : base + static_cast<uint32_t>(bb - 2) * g + 2 * bl;
    return {base, g, bl, static_cast<uint32_t>(s) * g + bl, d};
}

__device__ __forceinline__ float half_f(uint32_t bits) { return half_bits_to_float(static_cast<uint16_t>(bits)); }

// The activations of one lane slice: 32 values and the sums of its runs.
struct XSlice {
    float v[32];
    float s[4];
};

// ---- lane-major activation staging ---------------------------------------------
// At step t of a row, lane l = 8 s + bl works on slice s of superblock
// 8 t + bl.  Staging stores each (superblock, slice) record at position
// lm_chunk(l) of its superblock's 8-superblock group, in 16-byte slots laid
// out [slot][position]: every slot read of the row loops is one contiguous
// 1 KB per wavefront, which the LDS serves at its full rate whatever the
// slice shape.
// (A superblock-major layout, even padded, leaves the Q4_K and Q6_K slice
// shapes and the digit slices with 2- and 3-way bank conflicts, measured
// with SQ_LDS_BANK_CONFLICT on MI355X.)
// A slice is four 8-value runs; the shapes differ in which runs of the
// superblock they take, at positions p = 0..3 in the order the computes use:
//  * S32 (the IQ types): runs 4s + p, the 32-value block s;
//  * K4 (Q4_K, Q5_K; s = 2c + h): runs 8c + 2h + (p & 1) + 4 (p >> 1), i.e.
//    values [64c + 16h, +16) then [64c + 32 + 16h, +16) (the low and high
//    nibbles of code bytes [32c + 16h, +16); include/xdna/kquants.h:290-348);
//  * K6 (Q3_K, Q6_K; s = 4hh + k): runs 16hh + 4p + k, i.e. positions
//    [8k, 8k + 8) of the four 32-value groups of half hh
//    (include/xdna/kquants.h:350-419).
enum SliceShape { kS32 = 0, kK4 = 1, kK6 = 2 };
constexpr int slice_shape(int type) {
    return type == MI355X_TYPE_Q4_K || type == MI355X_TYPE_Q5_K   ? kK4
           : type == MI355X_TYPE_Q3_K || type == MI355X_TYPE_Q6_K ? kK6
                                                                  : kS32;
}
// run at position p of slice s
template <int SH>
__device__ __forceinline__ int run_of(int s, int p) {
    return SH == kS32 ? 4 * s + p
           : SH == kK4 ? 8 * (s >> 1) + 2 * (s & 1) + (p & 1) + 4 * (p >> 1)
                       : 16 * (s >> 2) + 4 * p + (s & 3);
}
constexpr int kLmSlot = 16 * 64;                // bytes of one slot row (64 records)
constexpr int kXGroupBytes = 9 * kLmSlot;       // f32: 8 value slots, the run sums
constexpr int kDgGroupBytes = 6 * kLmSlot;      // digits: 2 planes x 2, units, Z sums
// 16-byte position of record l = 8s + bl in its slot rows: l with bits 1-2
// XORed by bits 4-5.  Readers take one record per lane (a permutation of
// the 64 positions either way); the row kernels' staging stores (one 8-value
// run per lane, so a wavefront writes the records of two superblocks, all
// eight slices each) then fall on 16 distinct positions, i.e. every LDS
// bank, instead of 4.
__device__ __forceinline__ int lm_chunk(int l) { return l ^ (((l >> 4) & 3) << 1); }
// byte offset of the record of slice s of chunk superblock bc
__device__ __forceinline__ int lm_record(int group_bytes, int bc, int s) {
    return group_bytes * (bc >> 3) + 16 * lm_chunk(8 * s + (bc & 7));
}
constexpr size_t x_lds_bytes(int nb) { return static_cast<size_t>((nb + 7) / 8) * kXGroupBytes; }
constexpr size_t dg_lds_bytes(int nb) { return static_cast<size_t>((nb + 7) / 8) * kDgGroupBytes; }

// The pipelined and activation-stationary forms stage one record per
// thread: thread r stages record r & 63 of group r >> 6, i.e. slice s =
// (r & 63) >> 3 of chunk superblock 8 (r >> 6) + (r & 7), so each slot store
// of a wavefront is again one contiguous 1 KB (the row form stages one run
// per thread, further below).
// The record's four runs, from the chunk's activations xc (bc clamped into
// the chunk by the caller):
template <int SH>
__device__ __forceinline__ void load_record(const float *xc, int bc, int s, float4 (&v)[8]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const float4 *src = reinterpret_cast<const float4 *>(xc + 256 * bc + 8 * run_of<SH>(s, p));
        v[2 * p] = src[0];
        v[2 * p + 1] = src[1];
    }
}

// f32 record: slots 2p and 2p + 1 hold run p's 8 values, slot 8 the four
// run sums.
__device__ __forceinline__ void put_record_f32(uint8_t *rec, const float4 (&v)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<float4 *>(rec + kLmSlot * i) = v[i];
    float S[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const float4 a = v[2 * p], b = v[2 * p + 1];
        S[p] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    }
    *reinterpret_cast<float4 *>(rec + kLmSlot * 8) = make_float4(S[0], S[1], S[2], S[3]);
}

// The slice of a record: its 32 values and the sums the computes subtract
// (K6: each run's; K4: each 16-value half's; S32: the block's).
template <int SH>
__device__ __forceinline__ void x_slice_lm(const uint8_t *rec, XSlice &x) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 a = *reinterpret_cast<const float4 *>(rec + kLmSlot * i);
        x.v[4 * i + 0] = a.x;
        x.v[4 * i + 1] = a.y;
        x.v[4 * i + 2] = a.z;
        x.v[4 * i + 3] = a.w;
    }
    const float4 S = *reinterpret_cast<const float4 *>(rec + kLmSlot * 8);
    if constexpr (SH == kS32) {
        x.s[0] = (S.x + S.y) + (S.z + S.w);
    } else if constexpr (SH == kK4) {
        x.s[0] = S.x + S.y;
        x.s[1] = S.z + S.w;
    } else {
        x.s[0] = S.x;
        x.s[1] = S.y;
        x.s[2] = S.z;
        x.s[3] = S.w;
    }
}

template <int TYPE>
struct Kq;

// ---- Q4_K / Q5_K -------------------------------------------------------------
// Slice s = (chunk c = s/2, half h = s%2): code bytes [32c+16h, +16) of the
// chunk's 32; low nibbles are values 64c+16h+l (sub-block 2c), high nibbles
// 64c+32+16h+l (sub-block 2c+1) (include/xdna/kquants.h:290-348).

// 6-bit (scale, min) pair j of a Q4_K/Q5_K block from its 12 scale bytes
// (words w0 = bytes 0-3, w1 = 4-7, w2 = 8-11); include/xdna/kquants.h:204-212.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t w0, uint32_t w1, uint32_t w2, float &sc, float &m) {
    const int jj = j & 3;
    const uint32_t a = byte_u(w0, jj), b = byte_u(w1, jj), c = byte_u(w2, jj);
    const uint32_t sc_lo = a & 63, m_lo = b & 63;
    const uint32_t sc_hi = (c & 15) | ((a >> 6) << 4), m_hi = (c >> 4) | ((b >> 6) << 4);
    sc = static_cast<float>(j < 4 ? sc_lo : sc_hi);
    m = static_cast<float>(j < 4 ? m_lo : m_hi);
}

__device__ __forceinline__ float k4_finish(int s, const u32x4 &hd, float slo, float shi, const XSlice &x) {
    const int c = s >> 1;
    float sc0, m0, sc1, m1;
    scale_min_k4(2 * c, hd[1], hd[2], hd[3], sc0, m0);
    scale_min_k4(2 * c + 1, hd[1], hd[2], hd[3], sc1, m1);
    const float d = half_f(hd[0] & 0xFFFF), dmin = half_f(hd[0] >> 16);
    return (d * sc0) * slo - (dmin * m0) * x.s[0] + (d * sc1) * shi - (dmin * m1) * x.s[1];
}

template <>
struct Kq<MI355X_TYPE_Q4_K> {
    static constexpr int kGrid = 0;
    struct Regs {
        u32x4 q, hd;
    };
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const int c = s >> 1, h = s & 1;
        return {ld128(r, r.P[0] + 128 * b + 32 * c + 16 * h), ld128(r, r.P[1] + 16 * b)};
    }
    __device__ static float compute(const Regs &g, int s, const XSlice &x, const uint32_t *) {
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            slo = dot4(g.q[i] & 0x0F0F0F0Fu, &x.v[4 * i], slo);
            shi = dot4((g.q[i] >> 4) & 0x0F0F0F0Fu, &x.v[16 + 4 * i], shi);
        }
        return k4_finish(s, g.hd, slo, shi, x);
    }
};

template <>
struct Kq<MI355X_TYPE_Q5_K> {
    static constexpr int kGrid = 0;
    struct Regs {
        u32x4 q, qh, hd;
    };
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const int c = s >> 1, h = s & 1;
        return {ld128(r, r.P[0] + 128 * b + 32 * c + 16 * h), ld128(r, r.P[1] + 32 * b + 16 * h),
                ld128(r, r.P[2] + 16 * b)};
    }
    __device__ static float compute(const Regs &g, int s, const XSlice &x, const uint32_t *) {
        const int c = s >> 1;
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (g.q[i] & 0x0F0F0F0Fu) | (((g.qh[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((g.q[i] >> 4) & 0x0F0F0F0Fu) | (((g.qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            slo = dot4(lo, &x.v[4 * i], slo);
            shi = dot4(hi, &x.v[16 + 4 * i], shi);
        }
        return k4_finish(s, g.hd, slo, shi, x);
    }
};

// ---- Q3_K / Q6_K -------------------------------------------------------------
// Slice s = (half hh = s/4, k = s%4): positions l in [8k, 8k+8) of each of the
// four 32-value groups j of the half, values 128hh + 32j + l; every 8-value
// run lies inside one 16-value scale group (8hh + 2j + k/2).

// Q6_K: ql[128] (low nibbles), qh[64] (2 high bits), int8 scales[16], fp16 d;
// value = d * sc * (code6 - 32) (include/xdna/kquants.h:391-419).
template <>
struct Kq<MI355X_TYPE_Q6_K> {
    static constexpr int kGrid = 0;
    // sw4: the four scales of this slice, scales[8hh + kk + 2j] in byte j
    struct Regs {
        u32x2 qa, qb, qh;
        uint32_t sw4, d;
    };
    // lane record (ql, ql, qh runs), the slice pair's scale word, d
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const GPos q = gpos(r, 210, b, s);
        const u32x4 a = ld128(r, q.base + 24 * q.m);
        const u32x2 h = ld64(r, q.base + 24 * q.m + 16);
        const uint32_t w = ld32(r, q.base + 192 * q.g + 16 * q.bl + 4 * (s >> 1));
        return {u32x2{a[0], a[1]}, u32x2{a[2], a[3]}, h, w, ld16(r, q.d)};
    }
    __device__ static float compute(const Regs &g, int, const XSlice &x, const uint32_t *) {
        float sg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t A = g.qa[w], Bq = g.qb[w], H = g.qh[w];
            sg[0] = dot4((A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u), &x.v[0 + 4 * w], sg[0]);
            sg[1] = dot4((Bq & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u), &x.v[8 + 4 * w], sg[1]);
            sg[2] = dot4(((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u), &x.v[16 + 4 * w], sg[2]);
            sg[3] = dot4(((Bq >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u), &x.v[24 + 4 * w], sg[3]);
        }
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float sc = static_cast<float>(static_cast<int32_t>(g.sw4 << (24 - 8 * j)) >> 24);
            acc = fmaf(sc, sg[j] - 32.0f * x.s[j], acc);
        }
        return half_f(g.d) * acc;
    }
};

// Q3_K: hmask[32], qs[64] (2-bit codes), 12 bytes of sixteen 6-bit scales,
// fp16 d; value = d * (scale - 32) * (code2 + 4*hbit - 4)
// (include/xdna/kquants.h:350-389).
template <>
struct Kq<MI355X_TYPE_Q3_K> {
    static constexpr int kGrid = 0;
    struct Regs {
        u32x2 q;
        uint32_t h;
        u32x2 sw01;
        uint32_t sw2, d;
    };
    // lane record (8 code bytes, this slice's half h of the 8 hmask bytes it
    // shares with slice s ^ 4, whose lane is lane ^ 32), the 12 scale bytes
    // (sw01[kk]: the low-nibble bytes of scales kk, kk + 4, kk + 2, kk + 6;
    // sw2: scales[8..11]), d.  The loads return raw words; the exchange of h happens at decode
    // (hmask), so no load has to complete before the next one is issued.
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const GPos q = gpos(r, 110, b, s);
        const u32x3 rec = ld96(r, q.base + 12 * q.m);
        const u32x3 sc = ld96(r, q.base + 96 * q.g + 12 * q.bl);
        return {u32x2{rec[0], rec[1]}, rec[2], u32x2{sc[0], sc[1]}, sc[2], ld16(r, q.d)};
    }
    // The slice's 8 hmask bytes: one permlane32 swap of h returns, in every
    // lane, the lower lane's (slice hh = 0) half first and the upper lane's
    // second, i.e. the 8 bytes in order.  Every lane of the wavefront takes
    // part.
    __device__ static u32x2 hmask(const Regs &g) {
        const auto sw = __builtin_amdgcn_permlane32_swap(g.h, g.h, false, false);
        return u32x2{static_cast<uint32_t>(sw[0]), static_cast<uint32_t>(sw[1])};
    }
    // The byte whose nibble hh is the low 4 bits of scale 8hh + kk + 2j.
    __device__ static uint32_t lo_scale_byte(const Regs &g, int kk, int j) {
        return byte_u(kk ? g.sw01[1] : g.sw01[0], ((j & 1) << 1) | (j >> 1));
    }
    __device__ static float compute(const Regs &g, int s, const XSlice &x, const uint32_t *) {
        const int hh = s >> 2, k = s & 3;
        const u32x2 hm = hmask(g);
        float sg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t code =
                    ((g.q[w] >> (2 * j)) & 0x03030303u) | (((hm[w] >> (4 * hh + j)) & 0x01010101u) << 2);
                sg[j] = dot4(code, &x.v[8 * j + 4 * w], sg[j]);
            }
        }
        const int kk = k >> 1;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // scale index sidx = 8hh + 2j + kk: low nibble from byte sidx % 8
            // (nibble sidx / 8 = hh), high 2 bits from byte 8 + sidx % 4
            // (bit pair sidx / 4 = 2hh + j/2)
            const int lo_byte = 2 * j + kk;
            const uint32_t lo = (lo_scale_byte(g, kk, j) >> (4 * hh)) & 15u;
            const uint32_t hi = (byte_u(g.sw2, lo_byte & 3) >> (2 * (2 * hh + (j >> 1)))) & 3u;
            const float sc = static_cast<float>(static_cast<int>(lo | (hi << 4)) - 32);
            acc = fmaf(sc, sg[j] - 4.0f * x.s[j], acc);
        }
        return half_f(g.d) * acc;
    }
};

// ---- 32-value slices: IQ4_XS, IQ3_S, IQ3_XXS, IQ2_S ---------------------------

// IQ4_XS: d, scales_h, scales_l[4], qs[128]; sub-block ib has the 6-bit
// scale ls and 32 codebook indices (low nibbles first); value =
// d * (ls - 32) * kvalues_iq4nl[idx] (include/xdna/kquants.h:421-441).
// The codebook (biased by +128 into unsigned bytes) is looked up four
// indices at a time with byte permutes.
// Four 16-entry table lookups at once: nibble bytes n (each < 16) index the
// 16 bytes t0..t3.  Two v_perm read entry n & 7 of each 8-byte half; a third
// takes, per byte b, byte b of the first (selector b) or of the second half's
// result (selector b + 4, when bit 3 of the nibble is set).
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t n, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    return __builtin_amdgcn_perm(hi, lo, ((n >> 1) & 0x04040404u) | 0x03020100u);
}

template <>
struct Kq<MI355X_TYPE_IQ4_XS> {
    static constexpr int kGrid = 0;
    // kvalues_iq4nl + 128: {1, 24, 45, 63, 79, 93, 106, 118, 129, 141, 153, 166, 181, 197, 217, 241}
    static constexpr uint32_t kT0 = 0x3F2D1801u, kT1 = 0x766A5D4Fu, kT2 = 0xA6998D81u, kT3 = 0xF1D9C5B5u;
    struct Regs {
        u32x4 q;
        u32x2 hd;
    };
    __device__ static uint32_t lookup(uint32_t n) {
        return iq4_lookup(n, kT0, kT1, kT2, kT3);
    }
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        return {ld128(r, r.P[0] + 128 * b + 16 * s), ld64(r, r.P[1] + 8 * b)};
    }
    __device__ static float compute(const Regs &g, int s, const XSlice &x, const uint32_t *) {
        const float d = half_f(g.hd[0] & 0xFFFF);
        const uint32_t sh = g.hd[0] >> 16;
        const uint32_t ls = ((g.hd[1] >> (4 * s)) & 15u) | (((sh >> (2 * s)) & 3u) << 4);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = dot4(lookup(g.q[i] & 0x0F0F0F0Fu), &x.v[4 * i], acc);
            acc = dot4(lookup((g.q[i] >> 4) & 0x0F0F0F0Fu), &x.v[16 + 4 * i], acc);
        }
        return (d * static_cast<float>(static_cast<int>(ls) - 32)) * (acc - 128.0f * x.s[0]);
    }
};

// x with its sign flipped where bit `bit` of `signs` is set
__device__ __forceinline__ float signed_x(float x, uint32_t signs, int bit) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, x) ^ ((signs << (31 - bit)) & 0x80000000u));
}

// IQ3_S: d, qs[64], qh[8], signs[32], scales[4]; group g: 8 lookups of a
// 9-bit index (low byte qs[8g+k], bit k of qh[g]) into the 512-entry grid,
// sign bit 4k+j of the group's 4 sign bytes, scale d * (1 + 2 * nibble g)
// (include/xdna/kquants.h:443-490).
template <>
struct Kq<MI355X_TYPE_IQ3_S> {
    static constexpr int kGrid = kIq3sGridSize;  // u32 words
    struct Regs {
        u32x2 qs;
        uint32_t sg, qh, scb, d;
    };
    // lane record (qs, signs), qh byte, scale byte, d
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const GPos q = gpos(r, 110, b, s);
        const u32x3 rec = ld96(r, q.base + 12 * q.m);
        return {u32x2{rec[0], rec[1]}, rec[2], ld8(r, q.base + 96 * q.g + q.m),
                ld8(r, q.base + 104 * q.g + 4 * q.bl + (s >> 1)), ld16(r, q.d)};
    }
    __device__ static float compute(const Regs &g, int s, const XSlice &x, const uint32_t *grid) {
        const float db = half_f(g.d) * (1.0f + 2.0f * static_cast<float>((g.scb >> (4 * (s & 1))) & 15u));
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t idx = byte_u(g.qs[k >> 2], k & 3) | (((g.qh >> k) & 1u) << 8);
            const uint32_t gv = grid[idx];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = fmaf(byte_f(gv, j), signed_x(x.v[4 * k + j], g.sg, 4 * k + j), acc);
        }
        return db * acc;
    }
};

// 8 sign bits from a 7-bit index: bit 7 makes the count even (ksigns_iq2xs).
__device__ __forceinline__ uint32_t ksigns(uint32_t i7) { return i7 | ((__builtin_popcount(i7) & 1u) << 7); }

// IQ3_XXS (ggml): d, qs[64] grid indices, 8 words of [4 x 7-bit sign
// index | 4-bit scale << 28]; db = d * (0.5 + scale) * 0.5.  Grid from ggml.
template <>
struct Kq<MI355X_TYPE_IQ3_XXS> {
    static constexpr int kGrid = 256;
    struct Regs {
        u32x2 qs;
        uint32_t aux, d;
    };
    // lane record (qs, scales_and_signs word), d
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const GPos q = gpos(r, 98, b, s);
        const u32x3 rec = ld96(r, q.base + 12 * q.m);
        return {u32x2{rec[0], rec[1]}, rec[2], ld16(r, q.d)};
    }
    __device__ static float compute(const Regs &g, int, const XSlice &x, const uint32_t *grid) {
        const float db = half_f(g.d) * (0.5f + static_cast<float>(g.aux >> 28)) * 0.5f;
        float acc = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t sg = ksigns((g.aux >> (7 * l)) & 127u);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t gv = grid[byte_u(g.qs[l >> 1], 2 * (l & 1) + h)];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = fmaf(byte_f(gv, j), signed_x(x.v[8 * l + 4 * h + j], sg, 4 * h + j), acc);
            }
        }
        return db * acc;
    }
};

// IQ2_S (ggml): d, qs[32] index low bytes, signs[32], qh[8] (2 index bits per
// lookup), scales[8] (nibble per 16 values); db = d * (0.5 + s) * 0.25.
template <>
struct Kq<MI355X_TYPE_IQ2_S> {
    static constexpr int kGrid = 2048;  // 1024 x u64 as u32 pairs
    struct Regs {
        uint32_t qs, sg, qh, scb, d;
    };
    // lane record (qs, signs), the (qh, scale) byte pair, d
    __device__ static Regs load(const Row &r, uint32_t b, int s) {
        const GPos q = gpos(r, 82, b, s);
        const u32x2 rec = ld64(r, q.base + 8 * q.m);
        const uint32_t p = ld16(r, q.base + 64 * q.g + 2 * q.m);
        return {rec[0], rec[1], p & 0xFFu, p >> 8, ld16(r, q.d)};
    }
    __device__ static float compute(const Regs &g, int, const XSlice &x, const uint32_t *grid) {
        float part[2] = {0.f, 0.f};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = byte_u(g.qs, l) | (((g.qh >> (2 * l)) & 3u) << 8);
            const uint32_t g0 = grid[2 * idx], g1 = grid[2 * idx + 1];
            const uint32_t sb8 = byte_u(g.sg, l);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                part[l >> 1] = fmaf(byte_f(j < 4 ? g0 : g1, j & 3), signed_x(x.v[8 * l + j], sb8, j), part[l >> 1]);
        }
        const float d = half_f(g.d);
        const float db0 = d * (0.5f + static_cast<float>(g.scb & 15u)) * 0.25f;
        const float db1 = d * (0.5f + static_cast<float>(g.scb >> 4)) * 0.25f;
        return db0 * part[0] + db1 * part[1];
    }
};

// ---- digit path ---------------------------------------------------------------
// Activations as 16-bit fixed point: each 32-value block b of x has a scale
// c(b) = 32638 / m(b), m(b) its largest |x|, and x = Z * u(b) with
// Z = round(x * c(b)), |Z| <= 32638, u(b) = 1 / c(b); Z = z0 + 2^8 z1 in
// balanced signed bytes (z1 stays in [-128, 127] because |Z| <= 32639).  A
// staged slice record (lane-major, as the f32 records above) holds, per
// digit plane, the 4 runs' 8 bytes in position order (slots 2p, 2p + 1),
// then u of the block each run lies in (slot 4) and each run's sum of Z
// (slot 5); K4 records, whose computes take a unit and a Z sum per 16-value
// half, hold those four words in slot 4 (one full-width read).  Weight codes
// (small unsigned integers, or signed bytes for the signed codebooks) meet
// the digits in v_dot4_i32_i8: sum_i code_i * Z_i over a run is s0 + 2^8 s1
// with s_p = sum_i code_i * z_p,i, exact in int32.
// Error: rounding x to Z u moves each value by at most u / 2 = m / 65276
// (1.54e-5 m, with the reciprocals' rounding), so a row's result moves by at
// most 1.54e-5 * sum_b m(b) * sum_{i in b} |w_i| <= 1.54e-5 * sqrt(32) *
// |w_r| * |x| = 8.7e-5 |w_r| |x| (Cauchy-Schwarz twice: within a block, then
// over blocks with m(b) <= |x_b|), inside the GEMV tolerance of
// 1e-4 * |w_r| * |x|; for random data the error is orders of magnitude
// smaller.
struct XDig {
    uint32_t z[2][8];  // digit planes: 8 dwords (32 values) per plane
    float u[4];        // units of the 32-blocks the slice's runs lie in
    float zs[4];       // sum of Z over each run
};

// Scale c and unit u of a block whose largest |x| is m: m * c <= 32638
// (1 + 2^-22) < 32638.5, so |Z| <= 32638.  An all-zero (or denormal-small)
// block takes c = 2^126: its Z are 0 (or tiny) and u is a normal number.
__device__ __forceinline__ void dg_scale(float m, float &c, float &u) {
    c = fminf(32638.0f * __builtin_amdgcn_rcpf(m), 0x1p126f);
    u = __builtin_amdgcn_rcpf(c);
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// s0 + 2^8 s1 in f32: formed in int32 (exact: it is sum_i code_i * Z_i over
// at most 32 values, |code_i| <= 127, |Z_i| <= 32638) and rounded once.
__device__ __forceinline__ float combine(const int (&s)[2]) { return static_cast<float>(s[0] + s[1] * 256); }
// The same in f32, for sums up to 2^24 in magnitude whose s0 + 2^8 s1 may
// exceed int32 (one rounding: both converts are exact).
__device__ __forceinline__ float combine_f(const int (&s)[2]) {
    return fmaf(static_cast<float>(s[1]), 256.0f, static_cast<float>(s[0]));
}


// (scale, min) of sub-blocks 2c and 2c+1 of a Q4_K/Q5_K block at once: their
// bytes are adjacent in each of the three scale words (w0 = bytes 0-3,
// w1 = 4-7, w2 = 8-11), so both 6-bit pairs come out of 16-bit lanes
// (include/xdna/kquants.h:204-212 per sub-block).
__device__ __forceinline__ void scale_min_pair_k4(int c, uint32_t w0, uint32_t w1, uint32_t w2, float &sc0,
                                                  float &m0, float &sc1, float &m1) {
    const uint32_t sh = 16u * static_cast<uint32_t>(c & 1);
    const uint32_t a2 = (w0 >> sh) & 0xFFFFu, b2 = (w1 >> sh) & 0xFFFFu, c2 = (w2 >> sh) & 0xFFFFu;
    const uint32_t sc = c < 2 ? (a2 & 0x3F3Fu) : ((c2 & 0x0F0Fu) | ((a2 >> 2) & 0x3030u));
    const uint32_t mn = c < 2 ? (b2 & 0x3F3Fu) : (((c2 >> 4) & 0x0F0Fu) | ((b2 >> 2) & 0x3030u));
    sc0 = static_cast<float>(sc & 0xFFu);
    sc1 = static_cast<float>(sc >> 8);
    m0 = static_cast<float>(mn & 0xFFu);
    m1 = static_cast<float>(mn >> 8);
}

// sdot4(a, b, 0).  With the clamp bit the compiler selects the VOP3P form,
// which takes the zero as an inline constant, instead of the accumulating
// VOP2 form after a move of zero into the destination.  The clamp never
// acts: four products of signed bytes sum to at most 4 * 128 * 128 in
// magnitude.
__device__ __forceinline__ int sdot4_0(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), 0, true);
}

// Accumulates code dword `c` (4 values) against dword `i` of the 2 planes;
// with `first` (a compile-time constant at every call) the sums start here.
__device__ __forceinline__ void dot2(uint32_t c, const XDig &x, int i, int (&s)[2], bool first = false) {
    if (first) {
        s[0] = sdot4_0(c, x.z[0][i]);
        s[1] = sdot4_0(c, x.z[1][i]);
    } else {
        s[0] = sdot4(c, x.z[0][i], s[0]);
        s[1] = sdot4(c, x.z[1][i], s[1]);
    }
}

// The 4 codebook values of grid word g (magnitude bytes, each in 1..127, as
// every installed grid is) with the signs of nibble n (bit j set: value j
// negative; n < 16).  n * 0x810204 places copies of n at bits 2, 9, 16, 23
// (no two overlap, so no carries): bit j of n lands at bit 8j + 2, which
// with 0x03020100 makes a v_perm selector taking byte j of g (selector j) or
// of -g (j + 4); -g is 0x01010100 - g, exact per byte while no byte of g is
// zero.
__device__ __forceinline__ uint32_t sign_sel(uint32_t n) { return ((n * 0x810204u) & 0x04040404u) | 0x03020100u; }
__device__ __forceinline__ uint32_t signed4(uint32_t g, uint32_t n) {
    return __builtin_amdgcn_perm(0x01010100u - g, g, sign_sel(n));
}
// Two grid words with the low and high nibble of sign byte b.
__device__ __forceinline__ void signed8(uint32_t g_lo, uint32_t g_hi, uint32_t b, uint32_t &lo, uint32_t &hi) {
    lo = signed4(g_lo, b & 15u);
    hi = signed4(g_hi, (b >> 4) & 15u);
}

// The slice of a digit record (K4: units and Z sums per 16-value half; K6:
// per run; S32: the block's unit).
template <int SH>
__device__ __forceinline__ void dg_slice_lm(const uint8_t *rec, XDig &x) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const uint4 a = *reinterpret_cast<const uint4 *>(rec + kLmSlot * (2 * p));
        const uint4 b = *reinterpret_cast<const uint4 *>(rec + kLmSlot * (2 * p + 1));
        x.z[p][0] = a.x;
        x.z[p][1] = a.y;
        x.z[p][2] = a.z;
        x.z[p][3] = a.w;
        x.z[p][4] = b.x;
        x.z[p][5] = b.y;
        x.z[p][6] = b.z;
        x.z[p][7] = b.w;
    }
    if constexpr (SH == kS32) {
        x.u[0] = *reinterpret_cast<const float *>(rec + kLmSlot * 4);
    } else if constexpr (SH == kK4) {
        // slot 4 holds both halves' units and Z sums (put_record_dg)
        const float4 E = *reinterpret_cast<const float4 *>(rec + kLmSlot * 4);
        x.u[0] = E.x;
        x.u[1] = E.y;
        x.zs[0] = E.z;
        x.zs[1] = E.w;
    } else {
        const float4 E = *reinterpret_cast<const float4 *>(rec + kLmSlot * 4);
        const float4 Z = *reinterpret_cast<const float4 *>(rec + kLmSlot * 5);
        x.u[0] = E.x;
        x.u[1] = E.y;
        x.u[2] = E.z;
        x.u[3] = E.w;
        x.zs[0] = Z.x;
        x.zs[1] = Z.y;
        x.zs[2] = Z.z;
        x.zs[3] = Z.w;
    }
}

template <int TYPE>
struct KqDg;

template <>
struct KqDg<MI355X_TYPE_Q4_K> {
    __device__ static float compute(const Kq<MI355X_TYPE_Q4_K>::Regs &g, int s, const XDig &x, const uint32_t *) {
        int sa[2] = {0, 0}, sb[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dot2(g.q[i] & 0x0F0F0F0Fu, x, i, sa, i == 0);
            dot2((g.q[i] >> 4) & 0x0F0F0F0Fu, x, 4 + i, sb, i == 0);
        }
        const int c = s >> 1;
        float sc0, m0, sc1, m1;
        scale_min_pair_k4(c, g.hd[1], g.hd[2], g.hd[3], sc0, m0, sc1, m1);
        const float d = half_f(g.hd[0] & 0xFFFF), dmin = half_f(g.hd[0] >> 16);
        return ((d * sc0) * combine(sa) - (dmin * m0) * x.zs[0]) * x.u[0] +
               ((d * sc1) * combine(sb) - (dmin * m1) * x.zs[1]) * x.u[1];
    }
};

template <>
struct KqDg<MI355X_TYPE_Q5_K> {
    __device__ static float compute(const Kq<MI355X_TYPE_Q5_K>::Regs &g, int s, const XDig &x, const uint32_t *) {
        const int c = s >> 1;
        int sa[2] = {0, 0}, sb[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dot2((g.q[i] & 0x0F0F0F0Fu) | (((g.qh[i] >> (2 * c)) & 0x01010101u) << 4), x, i, sa, i == 0);
            dot2(((g.q[i] >> 4) & 0x0F0F0F0Fu) | (((g.qh[i] >> (2 * c + 1)) & 0x01010101u) << 4), x, 4 + i, sb,
                 i == 0);
        }
        float sc0, m0, sc1, m1;
        scale_min_pair_k4(c, g.hd[1], g.hd[2], g.hd[3], sc0, m0, sc1, m1);
        const float d = half_f(g.hd[0] & 0xFFFF), dmin = half_f(g.hd[0] >> 16);
        return ((d * sc0) * combine(sa) - (dmin * m0) * x.zs[0]) * x.u[0] +
               ((d * sc1) * combine(sb) - (dmin * m1) * x.zs[1]) * x.u[1];
    }
};

template <>
struct KqDg<MI355X_TYPE_Q6_K> {
    __device__ static float compute(const Kq<MI355X_TYPE_Q6_K>::Regs &g, int s, const XDig &x, const uint32_t *) {
        int sg[4][2] = {};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t A = g.qa[w], Bq = g.qb[w], H = g.qh[w];
            dot2((A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u), x, 0 + w, sg[0], w == 0);
            dot2((Bq & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u), x, 2 + w, sg[1], w == 0);
            dot2(((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u), x, 4 + w, sg[2], w == 0);
            dot2(((Bq >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u), x, 6 + w, sg[3], w == 0);
        }
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float sc = static_cast<float>(static_cast<int32_t>(g.sw4 << (24 - 8 * j)) >> 24);
            acc = fmaf(sc, (combine(sg[j]) - 32.0f * x.zs[j]) * x.u[j], acc);
        }
        return half_f(g.d) * acc;
    }
};

template <>
struct KqDg<MI355X_TYPE_Q3_K> {
    // Run j's 3-bit codes (2 code bits + the hmask bit) are formed in place,
    // scaled by 1, 4, 16, 16 for j = 0..3 -- code bits kept where they sit in
    // the byte (moved down two for j = 3, whose top bits would read as a
    // negative byte), the hmask bit ORed in above them -- so each costs a
    // mask and an OR.  Every scaled code is a multiple of its scale and below
    // 128, so the plane sums are exact multiples of it and combine_shr
    // divides it out exactly: the sums equal those of the unscaled codes.
    template <int SHR>
    __device__ static int combine_shr(const int (&s)[2]) {
        return (s[0] >> SHR) + s[1] * (1 << (8 - SHR));
    }
    __device__ static float compute(const Kq<MI355X_TYPE_Q3_K>::Regs &g, int s, const XDig &x, const uint32_t *) {
        const int hh = s >> 2, k = s & 3;
        const u32x2 hm = Kq<MI355X_TYPE_Q3_K>::hmask(g);
        int sg[4][2] = {};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t q = g.q[w];
            const uint32_t hs = hm[w] >> (4 * hh);  // bit j of each byte: run j's high bit
            dot2((q & 0x03030303u) | ((hs << 2) & 0x04040404u), x, 0 + w, sg[0], w == 0);
            dot2((q & 0x0C0C0C0Cu) | ((hs << 3) & 0x10101010u), x, 2 + w, sg[1], w == 0);
            dot2((q & 0x30303030u) | ((hs << 4) & 0x40404040u), x, 4 + w, sg[2], w == 0);
            dot2(((q >> 2) & 0x30303030u) | ((hs << 3) & 0x40404040u), x, 6 + w, sg[3], w == 0);
        }
        // The four 6-bit scales sidx = 8hh + kk + 2j (kk = k / 2) in one word,
        // bytes in run order 0, 2, 1, 3: low nibbles (nibble hh) from the
        // resident word sw01[kk], which holds scales[kk], [kk + 4], [kk + 2],
        // [kk + 6] in that order; high bit pairs from bytes kk (runs 0, 2)
        // and kk + 2 (runs 1, 3) of scales[8..11], pairs 2hh and 2hh + 1
        // (include/xdna/kquants.h:350-389).
        const int kk = k >> 1;
        const uint32_t L = kk ? g.sw01[1] : g.sw01[0];
        const uint32_t H = g.sw2 >> (8 * kk + 4 * hh);
        const uint32_t SC = ((L >> (4 * hh)) & 0x0F0F0F0Fu) | ((H & 0x00030003u) << 4) | ((H & 0x000C000Cu) << 10);
        // scale - 32 = the 6-bit scale with its top bit flipped, read as a
        // signed 6-bit field (one signed bitfield extract per scale)
        const int SX = static_cast<int>(SC ^ 0x20202020u);
        const float sc0 = static_cast<float>((SX << 26) >> 26);
        const float sc2 = static_cast<float>((SX << 18) >> 26);
        const float sc1 = static_cast<float>((SX << 10) >> 26);
        const float sc3 = static_cast<float>((SX << 2) >> 26);
        float acc = 0.f;
        acc = fmaf(sc0, (static_cast<float>(combine_shr<0>(sg[0])) - 4.0f * x.zs[0]) * x.u[0], acc);
        acc = fmaf(sc1, (static_cast<float>(combine_shr<2>(sg[1])) - 4.0f * x.zs[1]) * x.u[1], acc);
        acc = fmaf(sc2, (static_cast<float>(combine_shr<4>(sg[2])) - 4.0f * x.zs[2]) * x.u[2], acc);
        acc = fmaf(sc3, (static_cast<float>(combine_shr<4>(sg[3])) - 4.0f * x.zs[3]) * x.u[3], acc);
        return half_f(g.d) * acc;
    }
};

// IQ4_XS: the codebook as signed bytes, looked up four indices at a time.
template <>
struct KqDg<MI355X_TYPE_IQ4_XS> {
    // kvalues_iq4nl: {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}
    static constexpr uint32_t kT0 = 0xBFAD9881u, kT1 = 0xF6EADDCFu, kT2 = 0x26190D01u, kT3 = 0x71594535u;
    __device__ static uint32_t lookup(uint32_t n) {
        return iq4_lookup(n, kT0, kT1, kT2, kT3);
    }
    __device__ static float compute(const Kq<MI355X_TYPE_IQ4_XS>::Regs &g, int s, const XDig &x, const uint32_t *) {
        int sm[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dot2(lookup(g.q[i] & 0x0F0F0F0Fu), x, i, sm, i == 0);
            dot2(lookup((g.q[i] >> 4) & 0x0F0F0F0Fu), x, 4 + i, sm);
        }
        const float d = half_f(g.hd[0] & 0xFFFF);
        const uint32_t sh = g.hd[0] >> 16;
        const uint32_t ls = ((g.hd[1] >> (4 * s)) & 15u) | (((sh >> (2 * s)) & 3u) << 4);
        return (d * static_cast<float>(static_cast<int>(ls) - 32)) * (combine(sm) * x.u[0]);
    }
};

template <>
struct KqDg<MI355X_TYPE_IQ3_S> {
    __device__ static float compute(const Kq<MI355X_TYPE_IQ3_S>::Regs &g, int s, const XDig &x,
                                    const uint32_t *grid) {
        const uint2 *gt = reinterpret_cast<const uint2 *>(grid);
        const uint2 *st = gt + kIq3sGridSize;
        // The 9-bit grid indices two at a time, as the halfwords of one
        // word: bit k of qh spread to bit 0 of byte k % 4 of hb[k / 4]
        // (n * 0x204081 puts copies of the 4-bit n at bits 0, 7, 14, 21: no
        // two overlap, and bit j of copy j lands at bit 8j), then one v_perm
        // interleaves those bytes with the low index bytes.
        uint32_t hb[2] = {((g.qh & 15u) * 0x204081u) & 0x01010101u,
                          ((g.qh >> 4) * 0x204081u) & 0x01010101u};  // qh < 256
        // (opaque to the compiler, which otherwise narrows the low halfword's
        // mask to 0x1FF and loses the one-instruction halfword shift)
        asm("" : "+v"(hb[0]));
        asm("" : "+v"(hb[1]));
        int sm[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            constexpr uint32_t kSel[2] = {0x05010400u, 0x07030602u};
            const uint32_t pair = __builtin_amdgcn_perm(hb[k >> 2], g.qs[k >> 2], kSel[(k >> 1) & 1]);
            const uint32_t i0 = pair & 0xFFFFu, i1 = pair >> 16;
            const uint2 e0 = gt[i0], e1 = gt[i1], sl = st[byte_u(g.sg, k >> 1)];
            dot2(__builtin_amdgcn_perm(e0.y, e0.x, sl.x), x, k, sm, k == 0);
            dot2(__builtin_amdgcn_perm(e1.y, e1.x, sl.y), x, k + 1, sm);
        }
        const float db = half_f(g.d) * (1.0f + 2.0f * static_cast<float>((g.scb >> (4 * (s & 1))) & 15u));
        return db * (combine(sm) * x.u[0]);
    }
};

template <>
struct KqDg<MI355X_TYPE_IQ3_XXS> {
    __device__ static float compute(const Kq<MI355X_TYPE_IQ3_XXS>::Regs &g, int, const XDig &x,
                                    const uint32_t *grid) {
        const uint2 *gt = reinterpret_cast<const uint2 *>(grid);
        const uint2 *st = gt + 256;
        int sm[2] = {0, 0};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint2 e0 = gt[byte_u(g.qs[l >> 1], 2 * (l & 1))], e1 = gt[byte_u(g.qs[l >> 1], 2 * (l & 1) + 1)];
            const uint2 sl = st[(g.aux >> (7 * l)) & 127u];
            dot2(__builtin_amdgcn_perm(e0.y, e0.x, sl.x), x, 2 * l, sm, l == 0);
            dot2(__builtin_amdgcn_perm(e1.y, e1.x, sl.y), x, 2 * l + 1, sm);
        }
        // (0.5 + s) * 0.5 = s / 2 + 1/4, exact either way (s < 16)
        const float db = half_f(g.d) * fmaf(static_cast<float>(g.aux >> 28), 0.5f, 0.25f);
        return db * (combine(sm) * x.u[0]);
    }
};

template <>
struct KqDg<MI355X_TYPE_IQ2_S> {
    __device__ static float compute(const Kq<MI355X_TYPE_IQ2_S>::Regs &g, int, const XDig &x,
                                    const uint32_t *grid) {
        int s0[2] = {0, 0}, s1[2] = {0, 0};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = byte_u(g.qs, l) | (((g.qh >> (2 * l)) & 3u) << 8);
            const uint2 e = reinterpret_cast<const uint2 *>(grid)[idx];
            const uint2 sl = reinterpret_cast<const uint2 *>(grid + 2048)[byte_u(g.sg, l)];
            const uint32_t g0 = __builtin_amdgcn_perm(0x01010100u - e.x, e.x, sl.x);
            const uint32_t g1 = __builtin_amdgcn_perm(0x01010100u - e.y, e.y, sl.y);
            if (l < 2) {
                dot2(g0, x, 2 * l, s0, l == 0);
                dot2(g1, x, 2 * l + 1, s0);
            } else {
                dot2(g0, x, 2 * l, s1, l == 2);
                dot2(g1, x, 2 * l + 1, s1);
            }
        }
        // db_h = d * (0.5 + ls_h) / 4 = d * (2 ls_h + 1) / 8: the odd factors
        // a_h = 2 ls_h + 1 <= 31 mix the halves' plane sums exactly in 24-bit
        // products (|s_p| <= 16 * 127 * 128, so |t_p| < 2^24), then one f32
        // combine, d / 8 and the unit
        const int a0 = static_cast<int>(((g.scb << 1) & 0x1Eu) | 1u);
        const int a1 = static_cast<int>((g.scb >> 3) | 1u);  // scb < 256
        int t[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) t[p] = __mul24(a0, s0[p]) + __mul24(a1, s1[p]);
        return (half_f(g.d) * 0.125f) * (combine_f(t) * x.u[0]);
    }
};

// Byte J of each of four words, gathered into one word (byte t from w_t):
// two v_perm (selector 0x0C gives a zero byte) and an or.
template <int J>
__device__ __forceinline__ uint32_t gather_byte(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    constexpr uint32_t lo = 0x0C0C0000u | ((4u + J) << 8) | J;
    constexpr uint32_t hi = ((4u + J) << 24) | (static_cast<uint32_t>(J) << 16) | 0x0C0Cu;
    return __builtin_amdgcn_perm(w1, w0, lo) | __builtin_amdgcn_perm(w3, w2, hi);
}

// One DPP move of a float: row_ror:8 (the lane 8 apart within its row of 16)
__device__ __forceinline__ float ror8_f(float v) {
    return __builtin_bit_cast(float, dpp_i<0x128>(__builtin_bit_cast(int, v)));
}
// lane ^ 16 within each half wavefront (ds_swizzle, bit mode: xor 0x10)
__device__ __forceinline__ float swz16_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// Digit record of the values v (load_record).  Each run takes the scale of
// its 32-value block, whose largest |x| is the maximum over the runs of that
// block: all in this record (S32); two here and two in the record of slice
// s ^ 1, lane ^ 8 (K4); one here and one in each record of slices 4hh + k',
// lanes ^ 8, ^ 16, ^ 24 (K6).  Every lane of the wavefront must take part
// (the exchanges read other lanes); `store` masks the stores.  The digits,
// units and Z sums equal those of staging each 32-value block at once: the
// maximum is exact in any order and each Z and dword sum is formed from the
// same values.
template <int SH>
__device__ __forceinline__ void put_record_dg(uint8_t *rec, const float4 (&v)[8], bool store) {
    float m[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const float4 a = v[2 * p], b = v[2 * p + 1];
        m[p] = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                     fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    }
    if constexpr (SH == kS32) {
        const float M = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
        m[0] = m[1] = m[2] = m[3] = M;
    } else if constexpr (SH == kK4) {
        float A = fmaxf(m[0], m[1]), B = fmaxf(m[2], m[3]);
        A = fmaxf(A, ror8_f(A));
        B = fmaxf(B, ror8_f(B));
        m[0] = m[1] = A;
        m[2] = m[3] = B;
    } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            m[p] = fmaxf(m[p], ror8_f(m[p]));
            m[p] = fmaxf(m[p], swz16_f(m[p]));
        }
    }
    uint32_t pl[2][8];
    float uf[4];
    float zs[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        float c;
        dg_scale(m[p], c, uf[p]);
        // F = bits of 1.5 * 2^23 + v * c: |v * c| < 2^22, so the sum lies in
        // [2^23, 2^24) where f32 spacing is 1 and F = 0x4B400000 + Z, Z the
        // rounded integer.  The signed digits z0 + 2^8 z1 = Z (z0 in
        // [-128, 127]) have z0 = sext(byte 0 of Z) and z1 = (Z + 128) >> 8,
        // whose byte is byte 1 of Z + 128; 0x4B400000 adds nothing below bit
        // 16, so the two digit bytes are bytes 0 and 1 of F and F + 128.
        uint32_t F[8], G1[8];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const float4 f = v[2 * p + w];
            const float q[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                F[4 * w + t] = __builtin_bit_cast(uint32_t, fmaf(q[t], c, 12582912.0f));
                G1[4 * w + t] = F[4 * w + t] + 128u;
            }
        }
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            pl[0][2 * p + w] = gather_byte<0>(F[4 * w], F[4 * w + 1], F[4 * w + 2], F[4 * w + 3]);
            pl[1][2 * p + w] = gather_byte<1>(G1[4 * w], G1[4 * w + 1], G1[4 * w + 2], G1[4 * w + 3]);
        }
        // sum of the eight Z: the F sum less 8 * 0x4B400000 (mod 2^32; the
        // true sum is below 2^18 in magnitude)
        const uint32_t fs = (F[0] + F[1] + F[2]) + (F[3] + F[4] + F[5]) + (F[6] + F[7]);
        zs[p] = static_cast<float>(static_cast<int>(fs - 8u * 0x4B400000u));
    }
    if (store) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            *reinterpret_cast<uint4 *>(rec + kLmSlot * (2 * p)) = make_uint4(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
            *reinterpret_cast<uint4 *>(rec + kLmSlot * (2 * p + 1)) =
                make_uint4(pl[p][4], pl[p][5], pl[p][6], pl[p][7]);
        }
        if constexpr (SH == kK4) {
            // the reader needs each 16-value half's unit and Z sum: one slot
            *reinterpret_cast<float4 *>(rec + kLmSlot * 4) = make_float4(uf[0], uf[2], zs[0] + zs[1], zs[2] + zs[3]);
        } else {
            *reinterpret_cast<float4 *>(rec + kLmSlot * 4) = make_float4(uf[0], uf[1], uf[2], uf[3]);
            *reinterpret_cast<float4 *>(rec + kLmSlot * 5) = make_float4(zs[0], zs[1], zs[2], zs[3]);
        }
    }
}

// ---- staging one run per thread -------------------------------------------------
// The row kernels split the chunk's staging evenly over their threads: thread
// r converts run r (8 values) of the chunk, i.e. run j = r % 32 of chunk
// superblock r / 32, and writes that run's part of its record -- the same
// bytes put_record_dg / put_record_f32 write for it.  Slice s and position p
// of run j (the inverse of run_of):
template <int SH>
__device__ __forceinline__ void run_slot(int j, int &s, int &p) {
    if constexpr (SH == kS32) {
        s = j >> 2;
        p = j & 3;
    } else if constexpr (SH == kK4) {
        const int m = j & 7;  // j = 8c + 2h + (p & 1) + 4 (p >> 1)
        s = 2 * (j >> 3) + ((m >> 1) & 1);
        p = 2 * (m >> 2) + (m & 1);
    } else {
        const int m = j & 15;  // j = 16hh + 4p + k
        s = 4 * (j >> 4) + (m & 3);
        p = m >> 2;
    }
}

// quad_perm DPP moves: the lane ^ 1 and lane ^ 2 of each quad (all four
// lanes active)
__device__ __forceinline__ float quad_x1_f(float v) {
    return __builtin_bit_cast(float, dpp_i<0xB1>(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float quad_x2_f(float v) {
    return __builtin_bit_cast(float, dpp_i<0x4E>(__builtin_bit_cast(int, v)));
}

// Digit fields of run j of chunk superblock bc, values va, vb.  The four runs
// of a 32-value block (j = 4q .. 4q + 3) sit in the four lanes of one quad,
// all active: the block's largest |x| is their maximum, and a K4 half's Z
// sum adds the quad's run pair in position order (p even + p odd), as
// put_record_dg does.
template <int SH>
__device__ __forceinline__ void stage_run_dg(uint8_t *lds, const float4 &va, const float4 &vb, int bc, int j) {
    const float q[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
    float m = fmaxf(fmaxf(fmaxf(fabsf(q[0]), fabsf(q[1])), fmaxf(fabsf(q[2]), fabsf(q[3]))),
                    fmaxf(fmaxf(fabsf(q[4]), fabsf(q[5])), fmaxf(fabsf(q[6]), fabsf(q[7]))));
    m = fmaxf(m, quad_x1_f(m));
    m = fmaxf(m, quad_x2_f(m));
    // scale, F words, digit bytes and Z sum exactly as put_record_dg
    float c, uf;
    dg_scale(m, c, uf);
    uint32_t F[8], G1[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        F[t] = __builtin_bit_cast(uint32_t, fmaf(q[t], c, 12582912.0f));
        G1[t] = F[t] + 128u;
    }
    const uint32_t fs = (F[0] + F[1] + F[2]) + (F[3] + F[4] + F[5]) + (F[6] + F[7]);
    const float zs = static_cast<float>(static_cast<int>(fs - 8u * 0x4B400000u));
    int s, p;
    run_slot<SH>(j, s, p);
    uint8_t *rec = lds + lm_record(kDgGroupBytes, bc, s);
    // plane P of run p: bytes 8 (p & 1) .. +8 of slot 2P + (p >> 1)
    const int off = 8 * (p & 1);
    *reinterpret_cast<uint2 *>(rec + kLmSlot * (0 + (p >> 1)) + off) =
        make_uint2(gather_byte<0>(F[0], F[1], F[2], F[3]), gather_byte<0>(F[4], F[5], F[6], F[7]));
    *reinterpret_cast<uint2 *>(rec + kLmSlot * (2 + (p >> 1)) + off) =
        make_uint2(gather_byte<1>(G1[0], G1[1], G1[2], G1[3]), gather_byte<1>(G1[4], G1[5], G1[6], G1[7]));
    if constexpr (SH == kK4) {
        const float zo = quad_x1_f(zs);  // the half's other run (p ^ 1)
        if ((p & 1) == 0) {
            *reinterpret_cast<float *>(rec + kLmSlot * 4 + 4 * (p >> 1)) = uf;
            *reinterpret_cast<float *>(rec + kLmSlot * 4 + 8 + 4 * (p >> 1)) = zs + zo;
        }
    } else if constexpr (SH == kS32) {
        if (p == 0) *reinterpret_cast<float *>(rec + kLmSlot * 4) = uf;
    } else {
        *reinterpret_cast<float *>(rec + kLmSlot * 4 + 4 * p) = uf;
        *reinterpret_cast<float *>(rec + kLmSlot * 5 + 4 * p) = zs;
    }
}

// f32 fields of run j of chunk superblock bc: its values (slots 2p, 2p + 1)
// and their sum (slot 8, word p), as put_record_f32.
template <int SH>
__device__ __forceinline__ void stage_run_f32(uint8_t *lds, const float4 &va, const float4 &vb, int bc, int j) {
    int s, p;
    run_slot<SH>(j, s, p);
    uint8_t *rec = lds + lm_record(kXGroupBytes, bc, s);
    *reinterpret_cast<float4 *>(rec + kLmSlot * (2 * p)) = va;
    *reinterpret_cast<float4 *>(rec + kLmSlot * (2 * p + 1)) = vb;
    *reinterpret_cast<float *>(rec + kLmSlot * 8 + 4 * p) = ((va.x + va.y) + (va.z + va.w)) + ((vb.x + vb.y) + (vb.z + vb.w));
}

// LDS words of the digit kernels' codebook tables (GridRegs::put_dg).
constexpr int dg_table_words(int type) {
    return type == MI355X_TYPE_IQ3_S     ? 2 * kIq3sGridSize + 2 * 256
           : type == MI355X_TYPE_IQ3_XXS ? 2 * 256 + 2 * 128
           : type == MI355X_TYPE_IQ2_S   ? 2048 + 2 * 256
                                         : 0;
}

// ---- codebook staging ----------------------------------------------------------
// A thread's share of the codebook (words tid + nthr * k) is read into
// registers before the weight loads and written to LDS after them: vector
// loads retire in order, so a copy issued after the weight loads would wait
// for all of them before the workgroup's first barrier.  NMIN is the
// smallest thread count the kernel runs with.
template <int TYPE, int NMIN>
struct GridRegs {
    static constexpr int kN = Kq<TYPE>::kGrid > 0 ? (Kq<TYPE>::kGrid + NMIN - 1) / NMIN : 1;
    uint32_t w[kN];
    __device__ void fetch(const KqArgs &a, int tid, int nthr) {
        if constexpr (Kq<TYPE>::kGrid > 0) {
            const uint32_t *src = TYPE == MI355X_TYPE_IQ3_S ? kIq3sGrid : a.grid;
#pragma unroll
            for (int k = 0; k < kN; ++k) {
                const int i = tid + nthr * k;
                w[k] = src[i < Kq<TYPE>::kGrid ? i : Kq<TYPE>::kGrid - 1];
            }
        }
    }
    __device__ void put(uint32_t *grid, int tid, int nthr) const {
        if constexpr (Kq<TYPE>::kGrid > 0) {
#pragma unroll
            for (int k = 0; k < kN; ++k) {
                const int i = tid + nthr * k;
                if (i < Kq<TYPE>::kGrid) grid[i] = w[k];
            }
        }
    }
    // The digit kernels' tables (dg_table_words): each codebook word beside
    // its bytewise negation (IQ2_S: the words alone, its decode negates the
    // two words of an entry itself -- half the LDS bytes per lookup, 0.2 us
    // at 8192x8192), then the v_perm selector pairs of every sign byte
    // (IQ3_XXS: of every 7-bit sign index, through ksigns).
    __device__ void put_dg(uint32_t *tab, int tid, int nthr) const {
        if constexpr (Kq<TYPE>::kGrid > 0) {
            constexpr int G = Kq<TYPE>::kGrid;
            // IQ2_S keeps its words plain (the decode negates them)
            constexpr int kW = TYPE == MI355X_TYPE_IQ2_S ? 1 : 2;
#pragma unroll
            for (int k = 0; k < kN; ++k) {
                const int i = tid + nthr * k;
                if (i < G) {
                    tab[kW * i] = w[k];
                    if constexpr (kW == 2) tab[2 * i + 1] = 0x01010100u - w[k];
                }
            }
            constexpr int nsel = TYPE == MI355X_TYPE_IQ3_XXS ? 128 : 256;
            for (int b = tid; b < nsel; b += nthr) {
                const uint32_t bits = TYPE == MI355X_TYPE_IQ3_XXS ? ksigns(static_cast<uint32_t>(b)) : b;
                tab[kW * G + 2 * b] = sign_sel(bits & 15u);
                tab[kW * G + 2 * b + 1] = sign_sel(bits >> 4);
            }
        }
    }
};

}  // namespace
}  // namespace mi355x
