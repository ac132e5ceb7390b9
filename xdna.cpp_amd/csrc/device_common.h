// Device-side building blocks shared by the gfx950 GEMV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi355x {

typedef float float2_v __attribute__((ext_vector_type(2)));

// One DPP move of a float across lanes; lanes outside row_mask read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum of v over the 64 lanes of a wavefront, returned uniformly.  Must be
// called with every lane of the wave active: quad exchanges, half-row and
// row mirrors give each 16-lane row its total, then row_bcast15/row_bcast31
// fold rows 0..3 into lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);        // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);        // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);       // row_half_mirror
    v += dpp_mov<0x140>(v);       // row_mirror
    v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// IEEE half bits -> float (exact, including subnormals).
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Four nibble codes q in [0,15], one per byte of `bytes` (high nibbles
// clear), to floats.  A byte 0000qqqq read as OCP FP8 E4M3 (bias 7) is q/512
// exactly: q < 8 are the subnormals m*2^-9 and q >= 8 the normals with
// exponent field 1, (8+m)*2^-9.  The caller folds the 512 into its scale.
constexpr float kNibbleFp8Scale = 512.0f;

__device__ __forceinline__ void nibbles_to_float(uint32_t bytes, float out[4]) {
    float2_v a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(bytes), false);
    float2_v b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(bytes), true);
    out[0] = a[0];
    out[1] = a[1];
    out[2] = b[0];
    out[3] = b[1];
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw (untyped, stride 0) buffer descriptor on gfx9-family GPUs.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of buffer loads: non-temporal (read-once data).
constexpr int kNonTemporal = 2;

// 16-byte load of streamed (read-once) weight bytes; 16-byte aligned.
__device__ __forceinline__ u32x4 load_stream16(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// 16 weight bytes from a 2-byte aligned address.
__device__ __forceinline__ u32x4 load_16_a2(const uint8_t *p) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    u32x4 v;
    v[0] = h[0] | (static_cast<uint32_t>(h[1]) << 16);
    v[1] = h[2] | (static_cast<uint32_t>(h[3]) << 16);
    v[2] = h[4] | (static_cast<uint32_t>(h[5]) << 16);
    v[3] = h[6] | (static_cast<uint32_t>(h[7]) << 16);
    return v;
}

// s = 0, then s = s + c[i] for i = 0 .. n-1 in index order (ggml's
// sequential sum): exactly the rounding of the plain loop.  With c 16-byte
// aligned and n a multiple of 8, the reads of 8-value chunk k + 2 are issued
// before the additions of chunk k, so the chain waits on the additions
// rather than on each chunk's LDS latency; otherwise the plain loop.
__device__ __forceinline__ float ordered_sum(const float *c, int n) {
#pragma clang fp contract(off)
    float s = 0.0f;
    if ((reinterpret_cast<uintptr_t>(c) & 15u) != 0 || (n & 7) != 0) {
        for (int i = 0; i < n; ++i) s = s + c[i];
        return s;
    }
    // every read is in bounds (indices clamped to the last chunk) and
    // unconditional, so the reads stay LDS reads and their waits counted
    const float4 *p = reinterpret_cast<const float4 *>(c);
    const int nc = n >> 3, last = 2 * nc - 2;
    float4 a0 = p[0], a1 = p[1];
    float4 b0 = p[min(2, last)], b1 = p[min(2, last) + 1];
    for (int k = 0; k < nc; ++k) {
        const int q = min(2 * k + 4, last);
        const float4 n0 = p[q], n1 = p[q + 1];
        __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the additions
        s = s + a0.x;
        s = s + a0.y;
        s = s + a0.z;
        s = s + a0.w;
        s = s + a1.x;
        s = s + a1.y;
        s = s + a1.z;
        s = s + a1.w;
        a0 = b0;
        a1 = b1;
        b0 = n0;
        b1 = n1;
    }
    return s;
}

}  // namespace mi355x
