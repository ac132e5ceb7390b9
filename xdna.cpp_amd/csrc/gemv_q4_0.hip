// Q4_0 decode GEMV for gfx950 (the path of XdnaGemvEngine::run,
// src/xdna-gemv-engine.cpp:1817-1892, whose host loop is
// dot_q4_0_f32_4rows, src/xdna-gemv-engine.cpp:149-203).
//
// Resident row layout (made by the prepack stage, same bytes as ggml):
//   [qs of block 0 .. qs of block B-1 : 16*B bytes][fp16 d of every block : 2*B]
//   (code bytes XOR 0x88, d plane lane-major: see q4_0_layout.h)
// Work split:
//   * a workgroup of WAVES wavefronts stages the f32 activation row in LDS,
//     transposed so that lane b reads float4 k of block b at xs[k*KC + b]
//     (consecutive lanes -> consecutive 16-byte LDS words, no bank conflict),
//     plus bias[b] = (sum of block b's 32 activations) / 64;
//   * each wavefront owns R rows at a time; lane l owns blocks l, l+64, ...,
//     so every 16-byte weight load of a wave is one contiguous 1 KiB span;
//   * nibbles become floats through the FP8 E4M3 converter (q -> q/512), the
//     "-8" offset of Q4_0 is applied once per block through the bias:
//       sum_j (q_j - 8) x_j = 512 * (sum_j (q_j/512) x_j - bias_b);
//   * the 64 lane partials of a row are folded with DPP (wave_sum).
// Workgroups walk row groups grid-stride, so the activation row is staged
// once per workgroup when the whole row fits in one LDS chunk.
#include "device_common.h"
#include "internal.h"
#include "q4_0_layout.h"

#include <algorithm>
#include <mutex>

namespace mi355x {
namespace {

constexpr int kWaves = 8;

template <bool XBF16>
__device__ __forceinline__ void stage_x_chunk(const void *__restrict__ xv, int c0, int cn, int KC,
                                              float4 *xs, float *bias, bool x_al16) {
    for (int b = threadIdx.x; b < cn; b += blockDim.x) {
        float4 v[8];
        if constexpr (XBF16) {
            const uint16_t *xb = static_cast<const uint16_t *>(xv) + 32 * static_cast<int64_t>(c0 + b);
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = make_float4(bf16_bits_to_float(xb[4 * k]), bf16_bits_to_float(xb[4 * k + 1]),
                                   bf16_bits_to_float(xb[4 * k + 2]), bf16_bits_to_float(xb[4 * k + 3]));
        } else {
            const float *xf = static_cast<const float *>(xv) + 32 * static_cast<int64_t>(c0 + b);
            if (x_al16) {
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = reinterpret_cast<const float4 *>(xf)[k];
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    v[k] = make_float4(xf[4 * k], xf[4 * k + 1], xf[4 * k + 2], xf[4 * k + 3]);
            }
        }
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            xs[k * KC + b] = v[k];
            s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
        }
        bias[b] = s * (1.0f / 64.0f);
    }
}

// (1/512) * sum_j q_j x_j over one block, x from registers.  The resident
// code bytes hold q XOR 8 per nibble; the XOR is undone here.
__device__ __forceinline__ float q4_block_dot(u32x4 q, const float4 xv[8]) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w = q[k] ^ 0x88888888u;
        float lo[4], hi[4];
        nibbles_to_float(w & 0x0F0F0F0Fu, lo);
        nibbles_to_float((w >> 4) & 0x0F0F0F0Fu, hi);
        a0 = fmaf(lo[0], xv[k].x, a0);
        a0 = fmaf(lo[1], xv[k].y, a0);
        a0 = fmaf(lo[2], xv[k].z, a0);
        a0 = fmaf(lo[3], xv[k].w, a0);
        a1 = fmaf(hi[0], xv[k + 4].x, a1);
        a1 = fmaf(hi[1], xv[k + 4].y, a1);
        a1 = fmaf(hi[2], xv[k + 4].z, a1);
        a1 = fmaf(hi[3], xv[k + 4].w, a1);
    }
    return a0 + a1;
}

template <int NBL, int R, bool A16, bool XBF16>
__global__ __launch_bounds__(64 * kWaves) void gemv_q4_0_kernel(
    const uint8_t *__restrict__ W, const void *__restrict__ x, float *__restrict__ y, int N, int B,
    int KC, int64_t row_bytes, int x_al16) {
    extern __shared__ float4 lds[];
    float4 *xs = lds;
    float *bias = reinterpret_cast<float *>(lds + 8 * KC);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n_chunks = (B + KC - 1) / KC;
    constexpr int ROWS = kWaves * R;
    const int n_groups = (N + ROWS - 1) / ROWS;
    const int64_t scale_off = 16 * static_cast<int64_t>(B);

    if (n_chunks == 1) {
        stage_x_chunk<XBF16>(x, 0, B, KC, xs, bias, x_al16 != 0);
        __syncthreads();
    }

    for (int g = blockIdx.x; g < n_groups; g += gridDim.x) {
        const int row0 = g * ROWS + wave * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;

        for (int c = 0; c < n_chunks; ++c) {
            const int c0 = c * KC;
            const int cn = min(KC, B - c0);
            if (n_chunks > 1) {
                __syncthreads();
                stage_x_chunk<XBF16>(x, c0, cn, KC, xs, bias, x_al16 != 0);
                __syncthreads();
            }
            for (int s0 = 0; s0 < cn; s0 += 64 * NBL) {
                u32x4 q[R][NBL];
                float d[R][NBL];
                // unconditional loads from clamped addresses keep every
                // request in flight; blocks past the chunk get scale 0
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint8_t *rp = W + static_cast<int64_t>(min(row0 + r, N - 1)) * row_bytes;
#pragma unroll
                    for (int j = 0; j < NBL; ++j) {
                        const int b = s0 + lane + 64 * j;
                        const int64_t blk = c0 + min(b, cn - 1);
                        const uint8_t *qp = rp + 16 * blk;
                        q[r][j] = A16 ? load_stream16(qp) : load_16_a2(qp);
                        const uint16_t dh = *reinterpret_cast<const uint16_t *>(
                            rp + scale_off + 2 * static_cast<int64_t>(q4_0_d_slot(blk, B)));
                        d[r][j] = b < cn ? half_bits_to_float(dh) * kNibbleFp8Scale : 0.0f;
                    }
                }
#pragma unroll
                for (int j = 0; j < NBL; ++j) {
                    const int bc = min(s0 + lane + 64 * j, cn - 1);
                    float4 xv[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) xv[k] = xs[k * KC + bc];
                    const float sb = bias[bc];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float t = q4_block_dot(q[r][j], xv) - sb;
                        acc[r] = fmaf(d[r][j], t, acc[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == 0 && row0 + r < N) y[row0 + r] = s;
        }
    }
}

typedef void (*q4_kernel_t)(const uint8_t *, const void *, float *, int, int, int, int64_t, int);

template <int NBL, int R>
q4_kernel_t pick_ax(bool a16, bool xbf16) {
    if (a16) return xbf16 ? gemv_q4_0_kernel<NBL, R, true, true> : gemv_q4_0_kernel<NBL, R, true, false>;
    return xbf16 ? gemv_q4_0_kernel<NBL, R, false, true> : gemv_q4_0_kernel<NBL, R, false, false>;
}

template <int NBL>
q4_kernel_t pick_r(int r, bool a16, bool xbf16) {
    switch (r) {
    case 1: return pick_ax<NBL, 1>(a16, xbf16);
    case 2: return pick_ax<NBL, 2>(a16, xbf16);
    default: return pick_ax<NBL, 4>(a16, xbf16);
    }
}

q4_kernel_t pick(int nbl, int r, bool a16, bool xbf16) {
    switch (nbl) {
    case 1: return pick_r<1>(r, a16, xbf16);
    case 2: return pick_r<2>(r, a16, xbf16);
    default: return pick_r<4>(r, a16, xbf16);
    }
}

}  // namespace

int launch_gemv_q4_0(mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const int64_t row_bytes = 18 * B;
    if (a.N == 0) return MI355X_OK;
    if (B == 0) return launch_fill(ctx, a.y, 0, sizeof(float) * static_cast<size_t>(a.N));
    if (a.N > INT32_MAX || B > INT32_MAX / 64)
        return set_error(MI355X_EUNSUPPORTED, "Q4_0 GEMV: N or K beyond 32-bit kernel indexing");
    if (reinterpret_cast<uintptr_t>(a.W) % 2 != 0)
        return set_error(MI355X_EINVAL, "Q4_0 GEMV: weight pointer must be 2-byte aligned");
    if (ctx->kernel_variant == MI355X_VARIANT_GGML_Q8) {
        if (!q4_0_q8_supports(ctx, a))
            return set_error(MI355X_EUNSUPPORTED,
                             "Q4_0 GEMV: the ggml-cpu numerics variant takes f32 activations and K <= 16384");
        return launch_gemv_q4_0_q8(ctx, a);
    }
    if (ctx->kernel_variant != MI355X_VARIANT_EXACT_F32 && ctx->form_override == MI355X_FORM_STREAM &&
        q4_0_st_supports(ctx, a))
        return launch_gemv_q4_0_st(ctx, a);
    if (ctx->kernel_variant != MI355X_VARIANT_EXACT_F32 && q4_0_dp_supports(ctx, a))
        return launch_gemv_q4_0_dp(ctx, a);
    if (ctx->kernel_variant == MI355X_VARIANT_DIGITS)
        return set_error(MI355X_EUNSUPPORTED, "Q4_0 GEMV: digit-plane kernel does not take this shape/activation type");
    const bool a16 = (row_bytes % 16 == 0) && (reinterpret_cast<uintptr_t>(a.W) % 16 == 0);
    const bool x_al16 = !a.x_bf16 && (reinterpret_cast<uintptr_t>(a.x) % 16 == 0);

    // LDS: 8 float4 + 1 float per staged block.
    const size_t per_block = 8 * sizeof(float4) + sizeof(float);
    int64_t kc_cap = static_cast<int64_t>(ctx->max_lds_per_block / per_block);
    kc_cap = std::max<int64_t>(64, (kc_cap / 64) * 64);
    const int KC = static_cast<int>(std::min<int64_t>(B, kc_cap));
    const int nbl = B <= 64 ? 1 : (B <= 128 ? 2 : 4);
    int R = nbl == 4 ? 2 : 4;
    if (ctx->rows_override) R = ctx->rows_override;
    const size_t lds = per_block * static_cast<size_t>(KC);

    q4_kernel_t k = pick(nbl, R, a16, a.x_bf16);
    const int occ = occupancy(reinterpret_cast<const void *>(k), 64 * kWaves, lds);
    const int64_t rows_per_group = static_cast<int64_t>(kWaves) * R;
    const int64_t n_groups = (a.N + rows_per_group - 1) / rows_per_group;
    const int64_t grid = std::min<int64_t>(n_groups, static_cast<int64_t>(ctx->num_cus) * occ);

    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), lds, ctx->stream,
                       a.W, a.x, a.y, static_cast<int>(a.N), static_cast<int>(B), KC, row_bytes,
                       x_al16 ? 1 : 0);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

}  // namespace mi355x
