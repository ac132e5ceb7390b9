// K-quant and IQ decode GEMVs for gfx950: Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS,
// IQ3_S, IQ3_XXS, IQ2_S on the field-plane resident layout (kq_layout.h).
//
// Replaces the reference's dispatch_quant_gemv (src/xdna-gemv-engine.cpp:
// 1404-1500), which ran ggml-cpu's q8_K vec_dot or the AVX2 fallbacks on the
// host.  Numerics follow the scalar refs (include/xdna/kquants.h:290-577) in
// f32: every weight is (scale) * (code), each product with x is exact up to
// f32 rounding, and the sum order differs from the sequential reference only
// by re-association.
//
// Work split: a 512-thread workgroup stages the activations of one K chunk in
// LDS once, together with their sums over every 8 values, and (IQ types) the
// codebook.  Each wavefront then owns R rows at a time; its 64 lanes cover
// 8 superblocks per step, 8 lanes per superblock, one 32-value slice per
// lane.  A lane reads its slice's codes and its block's scales from the
// field planes with buffer loads (out-of-range reads return 0), decodes codes
// to f32 with byte converts, and forms
//     sum_i scale_g * (code_i - offset_g) * x_i
//       = sum_g scale_g * (sum_i code_i * x_i - offset_g * sum_i x_i)
// so the per-value work is one convert and one FMA; the offsets (Q6_K 32,
// Q3_K 4, IQ4_XS codebook bias 128, Q4_K/Q5_K mins) use the staged sums.
#include "device_common.h"
#include "internal.h"
#include "iq3s_grid.h"
#include "kq_layout.h"

#include <algorithm>
#include <cstdint>

namespace mi355x {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kSlices = 8;                 // lanes per superblock
constexpr int kBlocksPerStep = 64 / kSlices;
// Superblocks of x staged per pass: 60 (15360 values) keeps the LDS of a
// workgroup under 80 KB with the largest codebook, so two fit on a CU.
constexpr int kChunkBlocks = 60;

struct KqArgs {
    const uint8_t *W;
    int64_t N;
    int64_t row_bytes;
    int B;       // superblocks per row
    int b0;      // first superblock of this chunk
    int nb;      // superblocks in this chunk
    const void *x;
    float *y;
    int accumulate;
    const uint32_t *grid;  // device codebook (IQ3_XXS, IQ2_S), else null
};

__device__ __forceinline__ float byte_f(uint32_t w, int t) { return static_cast<float>((w >> (8 * t)) & 0xFFu); }

__device__ __forceinline__ uint32_t byte_u(uint32_t w, int t) { return (w >> (8 * t)) & 0xFFu; }

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
    uint32_t P[5];  // plane starts inside the row
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

__device__ __forceinline__ float half_f(uint32_t bits) { return half_bits_to_float(static_cast<uint16_t>(bits)); }

// The activation slice of lane slice s of one superblock: 32 values in
// xv[0..31] and the sums of its runs in xs[].
struct XSlice {
    float v[32];
    float s[4];
};

template <int TYPE>
struct Kq;

// ---- Q4_K / Q5_K -------------------------------------------------------------
// Slice s = (chunk c = s/2, half h = s%2): code bytes [32c+16h, +16) of the
// chunk's 32; low nibbles are values 64c+16h+l (sub-block 2c), high nibbles
// 64c+32+16h+l (sub-block 2c+1) (include/xdna/kquants.h:290-348).
__device__ __forceinline__ void x_slice_k4(int s, const float *xb, const float *sb, XSlice &x) {
    const int c = s >> 1, h = s & 1;
    const float4 *p0 = reinterpret_cast<const float4 *>(xb + 64 * c + 16 * h);
    const float4 *p1 = reinterpret_cast<const float4 *>(xb + 64 * c + 32 + 16 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 a = p0[i], b = p1[i];
        x.v[4 * i + 0] = a.x;
        x.v[4 * i + 1] = a.y;
        x.v[4 * i + 2] = a.z;
        x.v[4 * i + 3] = a.w;
        x.v[16 + 4 * i + 0] = b.x;
        x.v[16 + 4 * i + 1] = b.y;
        x.v[16 + 4 * i + 2] = b.z;
        x.v[16 + 4 * i + 3] = b.w;
    }
    const int g0 = (64 * c + 16 * h) >> 3;
    x.s[0] = sb[g0] + sb[g0 + 1];
    x.s[1] = sb[g0 + 4] + sb[g0 + 5];
}

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

template <>
struct Kq<MI355X_TYPE_Q4_K> {
    static constexpr int kGrid = 0;
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_k4(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *) {
        const int c = s >> 1, h = s & 1;
        const u32x4 q = ld128(r, r.P[0] + 128 * b + 32 * c + 16 * h);
        const u32x4 hd = ld128(r, r.P[1] + 16 * b);
        float sc0, m0, sc1, m1;
        scale_min_k4(2 * c, hd[1], hd[2], hd[3], sc0, m0);
        scale_min_k4(2 * c + 1, hd[1], hd[2], hd[3], sc1, m1);
        const float d = half_f(hd[0] & 0xFFFF), dmin = half_f(hd[0] >> 16);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            slo = dot4(q[i] & 0x0F0F0F0Fu, &x.v[4 * i], slo);
            shi = dot4((q[i] >> 4) & 0x0F0F0F0Fu, &x.v[16 + 4 * i], shi);
        }
        return (d * sc0) * slo - (dmin * m0) * x.s[0] + (d * sc1) * shi - (dmin * m1) * x.s[1];
    }
};

template <>
struct Kq<MI355X_TYPE_Q5_K> {
    static constexpr int kGrid = 0;
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_k4(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *) {
        const int c = s >> 1, h = s & 1;
        const u32x4 q = ld128(r, r.P[0] + 128 * b + 32 * c + 16 * h);
        const u32x4 qh = ld128(r, r.P[1] + 32 * b + 16 * h);
        const u32x4 hd = ld128(r, r.P[2] + 16 * b);
        float sc0, m0, sc1, m1;
        scale_min_k4(2 * c, hd[1], hd[2], hd[3], sc0, m0);
        scale_min_k4(2 * c + 1, hd[1], hd[2], hd[3], sc1, m1);
        const float d = half_f(hd[0] & 0xFFFF), dmin = half_f(hd[0] >> 16);
        float slo = 0.f, shi = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            slo = dot4(lo, &x.v[4 * i], slo);
            shi = dot4(hi, &x.v[16 + 4 * i], shi);
        }
        return (d * sc0) * slo - (dmin * m0) * x.s[0] + (d * sc1) * shi - (dmin * m1) * x.s[1];
    }
};

// ---- Q3_K / Q6_K -------------------------------------------------------------
// Slice s = (half hh = s/4, k = s%4): positions l in [8k, 8k+8) of each of the
// four 32-value groups j of the half, values 128hh + 32j + l; every 8-value
// run lies inside one 16-value scale group (8hh + 2j + k/2).
__device__ __forceinline__ void x_slice_k6(int s, const float *xb, const float *sb, XSlice &x) {
    const int hh = s >> 2, k = s & 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float4 *p = reinterpret_cast<const float4 *>(xb + 128 * hh + 32 * j + 8 * k);
        const float4 a = p[0], b = p[1];
        x.v[8 * j + 0] = a.x;
        x.v[8 * j + 1] = a.y;
        x.v[8 * j + 2] = a.z;
        x.v[8 * j + 3] = a.w;
        x.v[8 * j + 4] = b.x;
        x.v[8 * j + 5] = b.y;
        x.v[8 * j + 6] = b.z;
        x.v[8 * j + 7] = b.w;
        x.s[j] = sb[16 * hh + 4 * j + k];
    }
}

// Q6_K: ql[128] (low nibbles), qh[64] (2 high bits), int8 scales[16], fp16 d;
// value = d * sc * (code6 - 32) (include/xdna/kquants.h:391-419).
template <>
struct Kq<MI355X_TYPE_Q6_K> {
    static constexpr int kGrid = 0;
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_k6(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *) {
        const int hh = s >> 2, k = s & 3;
        const u32x2 qa = ld64(r, r.P[0] + 128 * b + 64 * hh + 8 * k);
        const u32x2 qb = ld64(r, r.P[0] + 128 * b + 64 * hh + 32 + 8 * k);
        const u32x2 qh = ld64(r, r.P[1] + 64 * b + 32 * hh + 8 * k);
        const u32x2 sw = ld64(r, r.P[2] + 16 * b + 8 * hh);
        const float d = half_f(ld16(r, r.P[3] + 2 * b));
        float sg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t A = qa[w], Bq = qb[w], H = qh[w];
            sg[0] = dot4((A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u), &x.v[0 + 4 * w], sg[0]);
            sg[1] = dot4((Bq & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u), &x.v[8 + 4 * w], sg[1]);
            sg[2] = dot4(((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u), &x.v[16 + 4 * w], sg[2]);
            sg[3] = dot4(((Bq >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u), &x.v[24 + 4 * w], sg[3]);
        }
        const int kk = k >> 1;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t word = j < 2 ? sw[0] : sw[1];
            const int idx = 2 * (j & 1) + kk;
            const float sc = static_cast<float>(static_cast<int32_t>(word << (24 - 8 * idx)) >> 24);
            acc = fmaf(sc, sg[j] - 32.0f * x.s[j], acc);
        }
        return d * acc;
    }
};

// Q3_K: hmask[32], qs[64] (2-bit codes), 12 bytes of sixteen 6-bit scales,
// fp16 d; value = d * (scale - 32) * (code2 + 4*hbit - 4)
// (include/xdna/kquants.h:350-389).
template <>
struct Kq<MI355X_TYPE_Q3_K> {
    static constexpr int kGrid = 0;
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_k6(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *) {
        const int hh = s >> 2, k = s & 3;
        const u32x2 q = ld64(r, r.P[0] + 64 * b + 32 * hh + 8 * k);
        const u32x2 hm = ld64(r, r.P[1] + 32 * b + 8 * k);
        const u32x2 sw01 = ld64(r, r.P[2] + 12 * b);
        const uint32_t sw2 = ld32(r, r.P[2] + 12 * b + 8);
        const float d = half_f(ld16(r, r.P[3] + 2 * b));
        float sg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t code = ((q[w] >> (2 * j)) & 0x03030303u) | (((hm[w] >> (4 * hh + j)) & 0x01010101u) << 2);
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
            const uint32_t lo_w = lo_byte < 4 ? sw01[0] : sw01[1];
            const uint32_t lo = (byte_u(lo_w, lo_byte & 3) >> (4 * hh)) & 15u;
            const uint32_t hi = (byte_u(sw2, lo_byte & 3) >> (2 * (2 * hh + (j >> 1)))) & 3u;
            const float sc = static_cast<float>(static_cast<int>(lo | (hi << 4)) - 32);
            acc = fmaf(sc, sg[j] - 4.0f * x.s[j], acc);
        }
        return d * acc;
    }
};

// ---- 32-value slices: IQ4_XS, IQ3_S, IQ3_XXS, IQ2_S ---------------------------
__device__ __forceinline__ void x_slice_32(int s, const float *xb, const float *sb, XSlice &x) {
    const float4 *p = reinterpret_cast<const float4 *>(xb + 32 * s);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 a = p[i];
        x.v[4 * i + 0] = a.x;
        x.v[4 * i + 1] = a.y;
        x.v[4 * i + 2] = a.z;
        x.v[4 * i + 3] = a.w;
    }
    x.s[0] = (sb[4 * s] + sb[4 * s + 1]) + (sb[4 * s + 2] + sb[4 * s + 3]);
}

// IQ4_XS: d, scales_h, scales_l[4], qs[128]; sub-block ib has the 6-bit
// scale ls and 32 codebook indices (low nibbles first); value =
// d * (ls - 32) * kvalues_iq4nl[idx] (include/xdna/kquants.h:421-441).
// The codebook (biased by +128 into unsigned bytes) is looked up four
// indices at a time with byte permutes.
template <>
struct Kq<MI355X_TYPE_IQ4_XS> {
    static constexpr int kGrid = 0;
    // kvalues_iq4nl + 128: {1, 24, 45, 63, 79, 93, 106, 118, 129, 141, 153, 166, 181, 197, 217, 241}
    static constexpr uint32_t kT0 = 0x3F2D1801u, kT1 = 0x766A5D4Fu, kT2 = 0xA6998D81u, kT3 = 0xF1D9C5B5u;
    __device__ static uint32_t lookup(uint32_t n) {
        const uint32_t sel = n & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(kT1, kT0, sel);
        const uint32_t hi = __builtin_amdgcn_perm(kT3, kT2, sel);
        const uint32_t m1 = (n >> 3) & 0x01010101u;
        const uint32_t mask = (m1 << 8) - m1;
        return (hi & mask) | (lo & ~mask);
    }
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_32(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *) {
        const u32x4 q = ld128(r, r.P[0] + 128 * b + 16 * s);
        const u32x2 hd = ld64(r, r.P[1] + 8 * b);
        const float d = half_f(hd[0] & 0xFFFF);
        const uint32_t sh = hd[0] >> 16;
        const uint32_t ls = ((hd[1] >> (4 * s)) & 15u) | (((sh >> (2 * s)) & 3u) << 4);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc = dot4(lookup(q[i] & 0x0F0F0F0Fu), &x.v[4 * i], acc);
            acc = dot4(lookup((q[i] >> 4) & 0x0F0F0F0Fu), &x.v[16 + 4 * i], acc);
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
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_32(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *grid) {
        const u32x2 qs = ld64(r, r.P[0] + 64 * b + 8 * s);
        const uint32_t sg = ld32(r, r.P[1] + 32 * b + 4 * s);
        const uint32_t qh = ld8(r, r.P[2] + 8 * b + s);
        const uint32_t scb = ld8(r, r.P[3] + 4 * b + (s >> 1));
        const float d = half_f(ld16(r, r.P[4] + 2 * b));
        const float db = d * (1.0f + 2.0f * static_cast<float>((scb >> (4 * (s & 1))) & 15u));
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t idx = byte_u(qs[k >> 2], k & 3) | (((qh >> k) & 1u) << 8);
            const uint32_t gv = grid[idx];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = fmaf(byte_f(gv, j), signed_x(x.v[4 * k + j], sg, 4 * k + j), acc);
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
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_32(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *grid) {
        const u32x2 qs = ld64(r, r.P[0] + 64 * b + 8 * s);
        const uint32_t aux = ld32(r, r.P[1] + 32 * b + 4 * s);
        const float d = half_f(ld16(r, r.P[2] + 2 * b));
        const float db = d * (0.5f + static_cast<float>(aux >> 28)) * 0.5f;
        float acc = 0.f;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t sg = ksigns((aux >> (7 * l)) & 127u);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t gv = grid[byte_u(qs[l >> 1], 2 * (l & 1) + h)];
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
    __device__ static void x_slice(int s, const float *xb, const float *sb, XSlice &x) { x_slice_32(s, xb, sb, x); }
    __device__ static float dot(const Row &r, uint32_t b, int s, const XSlice &x, const uint32_t *grid) {
        const uint32_t qs = ld32(r, r.P[0] + 32 * b + 4 * s);
        const uint32_t sg = ld32(r, r.P[1] + 32 * b + 4 * s);
        const uint32_t qh = ld8(r, r.P[2] + 8 * b + s);
        const uint32_t scb = ld8(r, r.P[3] + 8 * b + s);
        const float d = half_f(ld16(r, r.P[4] + 2 * b));
        float part[2] = {0.f, 0.f};
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const uint32_t idx = byte_u(qs, l) | (((qh >> (2 * l)) & 3u) << 8);
            const uint32_t g0 = grid[2 * idx], g1 = grid[2 * idx + 1];
            const uint32_t sb8 = byte_u(sg, l);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                part[l >> 1] = fmaf(byte_f(j < 4 ? g0 : g1, j & 3), signed_x(x.v[8 * l + j], sb8, j), part[l >> 1]);
        }
        const float db0 = d * (0.5f + static_cast<float>(scb & 15u)) * 0.25f;
        const float db1 = d * (0.5f + static_cast<float>(scb >> 4)) * 0.25f;
        return db0 * part[0] + db1 * part[1];
    }
};

// ---- kernel ------------------------------------------------------------------
template <int TYPE, int R, bool XBF16>
__global__ __launch_bounds__(kThreads) void gemv_kq_kernel(KqArgs a) {
    extern __shared__ float4 lds_kq[];
    float *xs = reinterpret_cast<float *>(lds_kq);       // nb * 256 values
    float *sums = xs + a.nb * 256;                        // nb * 32 sums of 8
    uint32_t *grid = reinterpret_cast<uint32_t *>(sums + a.nb * 32);

    // stage x[b0*256 .. (b0+nb)*256) and its 8-value sums
    const int n8 = a.nb * 32;
    for (int i = threadIdx.x; i < n8; i += kThreads) {
        float v[8];
        const int64_t base = static_cast<int64_t>(a.b0) * 256 + 8 * i;
        if constexpr (XBF16) {
            const uint16_t *xb = static_cast<const uint16_t *>(a.x) + base;
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = bf16_bits_to_float(xb[t]);
        } else {
            const float *xf = static_cast<const float *>(a.x) + base;
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = xf[t];
        }
        float4 *dst = reinterpret_cast<float4 *>(xs + 8 * i);
        dst[0] = make_float4(v[0], v[1], v[2], v[3]);
        dst[1] = make_float4(v[4], v[5], v[6], v[7]);
        sums[i] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    }
    if constexpr (Kq<TYPE>::kGrid > 0) {
        const uint32_t *src = TYPE == MI355X_TYPE_IQ3_S ? kIq3sGrid : a.grid;
        for (int i = threadIdx.x; i < Kq<TYPE>::kGrid; i += kThreads) grid[i] = src[i];
    }
    __syncthreads();

    constexpr KqLayout L = kq_layout(TYPE);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int s = lane & (kSlices - 1);
    const int bl = lane / kSlices;
    const int64_t n_groups = (a.N + R - 1) / R;
    const uint32_t records = static_cast<uint32_t>(a.row_bytes);

    for (int64_t g = static_cast<int64_t>(blockIdx.x) * kWaves + wave; g < n_groups;
         g += static_cast<int64_t>(gridDim.x) * kWaves) {
        Row rows[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = g * R + r < a.N ? g * R + r : a.N - 1;
            const uint8_t *base = a.W + row * a.row_bytes;
            rows[r].rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, records, kBufferWord3);
            const bool flipped = kq_row_flipped(reinterpret_cast<uintptr_t>(base));
#pragma unroll
            for (int i = 0; i < 5; ++i)
                rows[r].P[i] = i < L.nfields ? static_cast<uint32_t>(kq_plane_start(L, i, a.B, flipped)) : 0u;
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.f;
        for (int it = 0; it < a.nb; it += kBlocksPerStep) {
            const int bloc = it + bl;
            const bool valid = bloc < a.nb;
            const int bc = valid ? bloc : a.nb - 1;
            XSlice x;
            Kq<TYPE>::x_slice(s, xs + 256 * bc, sums + 32 * bc, x);
            const uint32_t babs = static_cast<uint32_t>(a.b0 + bc);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float p = Kq<TYPE>::dot(rows[r], babs, s, x, grid);
                acc[r] += valid ? p : 0.f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float t = wave_sum(acc[r]);
            const int64_t row = g * R + r;
            if (lane == 0 && row < a.N) a.y[row] = a.accumulate ? a.y[row] + t : t;
        }
    }
}

template <int TYPE>
const void *pick(int R, bool bf16) {
    if (R == 2) return bf16 ? (const void *)gemv_kq_kernel<TYPE, 2, true> : (const void *)gemv_kq_kernel<TYPE, 2, false>;
    return bf16 ? (const void *)gemv_kq_kernel<TYPE, 1, true> : (const void *)gemv_kq_kernel<TYPE, 1, false>;
}

const void *pick_kernel(int type, int R, bool bf16) {
    switch (type) {
    case MI355X_TYPE_Q4_K: return pick<MI355X_TYPE_Q4_K>(R, bf16);
    case MI355X_TYPE_Q5_K: return pick<MI355X_TYPE_Q5_K>(R, bf16);
    case MI355X_TYPE_Q3_K: return pick<MI355X_TYPE_Q3_K>(R, bf16);
    case MI355X_TYPE_Q6_K: return pick<MI355X_TYPE_Q6_K>(R, bf16);
    case MI355X_TYPE_IQ4_XS: return pick<MI355X_TYPE_IQ4_XS>(R, bf16);
    case MI355X_TYPE_IQ3_S: return pick<MI355X_TYPE_IQ3_S>(R, bf16);
    case MI355X_TYPE_IQ3_XXS: return pick<MI355X_TYPE_IQ3_XXS>(R, bf16);
    case MI355X_TYPE_IQ2_S: return pick<MI355X_TYPE_IQ2_S>(R, bf16);
    default: return nullptr;
    }
}

int grid_words(int type) {
    switch (type) {
    case MI355X_TYPE_IQ3_S: return kIq3sGridSize;
    case MI355X_TYPE_IQ3_XXS: return 256;
    case MI355X_TYPE_IQ2_S: return 2048;
    default: return 0;
    }
}

}  // namespace

int launch_gemv_kquant(mi355x_ctx *ctx, const GemvArgs &a) {
    const KqLayout L = kq_layout(a.type);
    if (L.block_bytes == 0) return set_error(MI355X_EUNSUPPORTED, "unsupported weight type for the K/IQ kernels");
    const int64_t B = a.K / 256;
    const int64_t row_bytes = B * L.block_bytes;
    if (row_bytes >= (int64_t(1) << 31))
        return set_error(MI355X_EUNSUPPORTED, "row too long for 32-bit buffer offsets");
    if (a.N == 0) return MI355X_OK;
    if (a.K == 0) return launch_fill(ctx, a.y, 0, static_cast<size_t>(a.N) * sizeof(float));
    const uint32_t *grid = nullptr;
    if (a.type == MI355X_TYPE_IQ3_XXS) grid = static_cast<const uint32_t *>(ctx->iq3xxs_grid);
    if (a.type == MI355X_TYPE_IQ2_S) grid = static_cast<const uint32_t *>(ctx->iq2s_grid);
    if (grid_words(a.type) > 0 && a.type != MI355X_TYPE_IQ3_S && !grid)
        return set_error(MI355X_EUNSUPPORTED, "grid table not installed for this IQ type");
    int R = a.N >= 8192 ? 2 : 1;
    if (ctx->rows_override == 1 || ctx->rows_override == 2) R = ctx->rows_override;
    const void *k = pick_kernel(a.type, R, a.x_bf16);
    const int64_t n_groups = (a.N + R - 1) / R;
    // equal chunks of at most kChunkBlocks superblocks
    const int64_t n_chunks = (B + kChunkBlocks - 1) / kChunkBlocks;
    const int64_t per_chunk = (B + n_chunks - 1) / n_chunks;
    for (int64_t b0 = 0; b0 < B; b0 += per_chunk) {
        const int nb = static_cast<int>(std::min<int64_t>(per_chunk, B - b0));
        const size_t lds = static_cast<size_t>(nb) * (256 + 32) * sizeof(float) + grid_words(a.type) * 4u;
        if (lds > ctx->max_lds_per_block) return set_error(MI355X_EUNSUPPORTED, "activation chunk exceeds LDS");
        const int occ = occupancy(k, kThreads, lds);
        int64_t wgs = std::min<int64_t>((n_groups + kWaves - 1) / kWaves, static_cast<int64_t>(ctx->num_cus) * occ);
        if (ctx->grid_override > 0) wgs = std::min<int64_t>(wgs, ctx->grid_override);
        KqArgs args{a.W, a.N, row_bytes, static_cast<int>(B), static_cast<int>(b0), nb, a.x, a.y, b0 > 0 ? 1 : 0,
                    grid};
        void *params[] = {&args};
        MI355X_HIP(hipLaunchKernel(k, dim3(static_cast<unsigned>(std::max<int64_t>(wgs, 1))), dim3(kThreads), params,
                                   lds, ctx->stream));
    }
    return MI355X_OK;
}

}  // namespace mi355x
