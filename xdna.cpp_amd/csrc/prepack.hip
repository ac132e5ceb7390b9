// Prepack stage: ggml block encoding <-> HBM-resident layout.
//
// Successor of Q4Prepacker (src/xdna-q4-prepack.cpp:262-340), which split
// Q4_0 into a nibble plane and a BF16 scale plane per AIE column.  Here the
// planes are per row and keep the exact fp16 scale bits, so the resident
// tensor is a row-local byte permutation of the ggml bytes:
//   ggml row  : B blocks of [d lo, d hi, qs[0..15]]          (18*B bytes)
//   resident  : [qs of block 0..B-1 (16*B)][d plane (2*B)]
// every qs byte is stored XOR 0x88, i.e. as the two signed 4-bit codes
// q - 8 that the integer kernels consume directly, and the d plane is
// lane-major over full 64-block columns (q4_0_layout.h).
// K-quant and IQ rows are regrouped into field planes (kq_layout.h).
// A byte of the ggml encoding at tensor offset o maps to exactly one resident
// byte, so set_tensor/get_tensor with any (offset, size) can be served
// without touching other bytes.
#include "device_common.h"
#include "internal.h"
#include "kq_layout.h"
#include "q4_0_layout.h"

#include <algorithm>

namespace mi355x {
namespace {

// Resident offset of ggml byte `o` in a Q4_0 tensor with `B` blocks per row;
// *xor_mask receives the byte transform (0x88 for code bytes, 0 for scales).
__device__ __forceinline__ uint64_t q4_0_to_resident(uint64_t o, uint64_t row_bytes, uint64_t B,
                                                     uint8_t *xor_mask) {
    const uint64_t row = o / row_bytes;
    const uint64_t p = o - row * row_bytes;
    const uint64_t blk = p / 18;
    const uint64_t e = p - blk * 18;
    *xor_mask = e < 2 ? 0 : 0x88;
    const uint64_t in_row = e < 2 ? 16 * B + 2 * q4_0_d_slot(blk, B) + e : 16 * blk + (e - 2);
    return row * row_bytes + in_row;
}

__global__ void q4_0_scatter_kernel(uint8_t *__restrict__ packed, const uint8_t *__restrict__ raw,
                                    uint64_t offset, uint64_t size, uint64_t row_bytes, uint64_t B) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < size; i += stride) {
        uint8_t m;
        const uint64_t dst = q4_0_to_resident(offset + i, row_bytes, B, &m);
        packed[dst] = raw[i] ^ m;
    }
}

__global__ void q4_0_gather_kernel(uint8_t *__restrict__ raw, const uint8_t *__restrict__ packed,
                                   uint64_t offset, uint64_t size, uint64_t row_bytes, uint64_t B) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < size; i += stride) {
        uint8_t m;
        const uint64_t src = q4_0_to_resident(offset + i, row_bytes, B, &m);
        raw[i] = packed[src] ^ m;
    }
}

// Resident offset of ggml byte `o` of a K/IQ tensor whose resident copy
// starts at `base` (row flips depend on the row's address).
__device__ __forceinline__ uint64_t kq_to_resident(const KqLayout &L, uint64_t o, uint64_t row_bytes, uint64_t B,
                                                   uintptr_t base) {
    const uint64_t row = o / row_bytes;
    const uint64_t p = o - row * row_bytes;
    const uint64_t blk = p / L.block_bytes;
    const int e = static_cast<int>(p - blk * L.block_bytes);
    const bool flipped = kq_row_flipped(base + row * row_bytes);
    return row * row_bytes + kq_row_offset(L, blk, e, B, flipped);
}

template <int TYPE>
__global__ void kq_scatter_kernel(uint8_t *__restrict__ packed, const uint8_t *__restrict__ raw, uint64_t offset,
                                  uint64_t size, uint64_t row_bytes, uint64_t B) {
    constexpr KqLayout L = kq_layout(TYPE);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < size; i += stride)
        packed[kq_to_resident(L, offset + i, row_bytes, B, reinterpret_cast<uintptr_t>(packed))] = raw[i];
}

template <int TYPE>
__global__ void kq_gather_kernel(uint8_t *__restrict__ raw, const uint8_t *__restrict__ packed, uint64_t offset,
                                 uint64_t size, uint64_t row_bytes, uint64_t B) {
    constexpr KqLayout L = kq_layout(TYPE);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < size; i += stride)
        raw[i] = packed[kq_to_resident(L, offset + i, row_bytes, B, reinterpret_cast<uintptr_t>(packed))];
}

typedef void (*kq_copy_fn)(uint8_t *, const uint8_t *, uint64_t, uint64_t, uint64_t, uint64_t);

template <bool SCATTER>
kq_copy_fn kq_copy_kernel(int type) {
    switch (type) {
#define MI355X_KQ_CASE(T) \
    case T: return SCATTER ? kq_scatter_kernel<T> : kq_gather_kernel<T>;
        MI355X_KQ_CASE(MI355X_TYPE_Q3_K)
        MI355X_KQ_CASE(MI355X_TYPE_Q4_K)
        MI355X_KQ_CASE(MI355X_TYPE_Q5_K)
        MI355X_KQ_CASE(MI355X_TYPE_Q6_K)
        MI355X_KQ_CASE(MI355X_TYPE_IQ4_XS)
        MI355X_KQ_CASE(MI355X_TYPE_IQ3_S)
        MI355X_KQ_CASE(MI355X_TYPE_IQ3_XXS)
        MI355X_KQ_CASE(MI355X_TYPE_IQ2_S)
#undef MI355X_KQ_CASE
    default: return nullptr;
    }
}

__global__ void fill_kernel(uint8_t *__restrict__ dst, uint8_t value, uint64_t bytes) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride)
        dst[i] = value;
}

unsigned grid_for(uint64_t work, int num_cus) {
    const uint64_t want = (work + 255) / 256;
    const uint64_t cap = static_cast<uint64_t>(std::max(num_cus, 1)) * 16;
    return static_cast<unsigned>(std::max<uint64_t>(1, std::min(want, cap)));
}

}  // namespace

int launch_prepack_scatter(mi355x_ctx *ctx, int type, int64_t N, int64_t K, uint8_t *packed,
                           const uint8_t *raw, size_t offset, size_t size) {
    (void)N;
    if (size == 0) return MI355X_OK;
    if (type == MI355X_TYPE_Q4_0) {
        const uint64_t B = static_cast<uint64_t>(K / 32);
        hipLaunchKernelGGL(q4_0_scatter_kernel, dim3(grid_for(size, ctx->num_cus)), dim3(256), 0,
                           ctx->stream, packed, raw, static_cast<uint64_t>(offset),
                           static_cast<uint64_t>(size), 18 * B, B);
        MI355X_HIP(hipGetLastError());
        return MI355X_OK;
    }
    const kq_copy_fn k = kq_copy_kernel<true>(type);
    if (!k) return set_error(MI355X_EINVAL, "prepack: unknown weight type");
    const uint64_t B = static_cast<uint64_t>(K / 256);
    hipLaunchKernelGGL(k, dim3(grid_for(size, ctx->num_cus)), dim3(256), 0, ctx->stream, packed, raw,
                       static_cast<uint64_t>(offset), static_cast<uint64_t>(size), B * kq_layout(type).block_bytes, B);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

int launch_prepack_gather(mi355x_ctx *ctx, int type, int64_t N, int64_t K, uint8_t *raw,
                          const uint8_t *packed, size_t offset, size_t size) {
    (void)N;
    if (size == 0) return MI355X_OK;
    if (type == MI355X_TYPE_Q4_0) {
        const uint64_t B = static_cast<uint64_t>(K / 32);
        hipLaunchKernelGGL(q4_0_gather_kernel, dim3(grid_for(size, ctx->num_cus)), dim3(256), 0,
                           ctx->stream, raw, packed, static_cast<uint64_t>(offset),
                           static_cast<uint64_t>(size), 18 * B, B);
        MI355X_HIP(hipGetLastError());
        return MI355X_OK;
    }
    const kq_copy_fn k = kq_copy_kernel<false>(type);
    if (!k) return set_error(MI355X_EINVAL, "unpack: unknown weight type");
    const uint64_t B = static_cast<uint64_t>(K / 256);
    hipLaunchKernelGGL(k, dim3(grid_for(size, ctx->num_cus)), dim3(256), 0, ctx->stream, raw, packed,
                       static_cast<uint64_t>(offset), static_cast<uint64_t>(size), B * kq_layout(type).block_bytes, B);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

int launch_fill(mi355x_ctx *ctx, void *dst, uint8_t value, size_t bytes) {
    if (bytes == 0) return MI355X_OK;
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(bytes, ctx->num_cus)), dim3(256), 0, ctx->stream,
                       static_cast<uint8_t *>(dst), value, static_cast<uint64_t>(bytes));
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

}  // namespace mi355x
