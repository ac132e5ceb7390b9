// Q4_0 decode GEMV, "digit-plane" form, for gfx950.
//
// Same resident row layout as gemv_q4_0.hip ([qs planes][fp16 d plane]).
// The activation row is re-expressed once per workgroup, per 32-value block
// b, as a fixed-point integer vector: Z_j = rint(x_j / u_b) with u_b the
// power of two that puts max_j |x_j| / u_b in (244667, 489335], so
// |Z_j| <= 489335 < 2^19 and the scaling itself is exact.  Each Z_j is split into
// five signed base-16 digits z_p in [-8, 7] (balanced: Z + 0x88888 has
// nibbles z_p + 8), stored as five 32-nibble "digit planes" in the nibble
// order of the Q4_0 bytes.  The block dot product is then exact integer
// arithmetic on the dot8 unit (v_dot8c_i32_i4, 8 signed 4-bit products per
// instruction):
//   A_p = sum_j (q_j - 8) * z_p(j)           (4 dot8 per plane)
//   T   = sum_p 16^p A_p = sum_j (q_j - 8) Z_j,  |T| < 1.5e8
//   y_r += d_rb * u_b * float(T)
// Compared with converting nibbles to f32 (2 VALU ops per weight) this costs
// about 1.1 VALU ops per weight.  The only approximation beyond f32 rounding
// is the activation quantization: |x_j - Z_j u_b| <= u_b/2 <= 2^-18.9 max|x_b|.
//
// Work split: workgroups of 8 or 16 wavefronts; each wavefront owns R rows
// per step and walks its row groups grid-stride.  The first group's weight
// loads are issued right after the activation loads and before the digit
// planes are built, so HBM traffic starts with the kernel.  Lane l owns
// blocks l, l+64, ... of a row (contiguous 1 KiB per 16-byte load
// instruction); row partials are folded with DPP.
#include "device_common.h"
#include "internal.h"
#include "q4_0_layout.h"
#include "wave_rows.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

namespace mi355x {
namespace {

constexpr int kPlanes = 5;
constexpr float kZmax = 489335.0f;  // 0x77777: largest balanced 5-digit value
constexpr uint32_t kBalance = 0x88888u;
// 1.5 * 2^23 + 0x88888: adding it to a value of magnitude < 2^21 rounds the
// value to an integer and leaves integer + 0x88888 in the low mantissa bits
constexpr float kMagic = 13142152.0f;

// Digit planes of the activation row: planes[p * B + b] holds, as four
// dwords k = 0..3, the digit p of values 4k+e (nibble 2e) and 16+4k+e
// (nibble 2e+1), e = 0..3 -- the nibble positions of Q4_0 byte 4k+e.
//
// Staging is split in two so that the activation loads can be issued before
// the weight loads: the vector-memory counter retires loads in order, so
// data loaded *after* the weights could only be used once every weight
// byte had arrived.  Thread t handles value group i = t + it*blockDim.x
// (block b = i/4, dword k = i%4), XI groups per thread.
template <int XI>
struct XTile {
    float v[XI][8];

    __device__ __forceinline__ void load(const float *__restrict__ x, int B, bool x_al16) {
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int i = min(static_cast<int>(threadIdx.x + it * blockDim.x), 4 * B - 1);
            const float *xb = x + 32 * static_cast<int64_t>(i >> 2) + 4 * (i & 3);
            if (x_al16) {
                const float4 lo = *reinterpret_cast<const float4 *>(xb);
                const float4 hi = *reinterpret_cast<const float4 *>(xb + 16);
                v[it][0] = lo.x; v[it][1] = hi.x; v[it][2] = lo.y; v[it][3] = hi.y;
                v[it][4] = lo.z; v[it][5] = hi.z; v[it][6] = lo.w; v[it][7] = hi.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[it][2 * e] = xb[e];
                    v[it][2 * e + 1] = xb[16 + e];
                }
            }
        }
    }

    // The math runs for every thread (groups past the row repeat the last
    // group); only the LDS stores are predicated.  A branch around the math
    // would let the compiler sink the activation loads behind the weights.
    __device__ __forceinline__ void store(int B, uint32_t *planes, float *ub) const {
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int i = threadIdx.x + it * blockDim.x;
            const int ic = min(i, 4 * B - 1);
            stage_group(v[it], ic >> 2, ic & 3, B, i < 4 * B, planes, ub);
        }
    }

    // one group of 8 values -> five plane dwords (+ the block scale)
    __device__ __forceinline__ static void stage_group(const float *v, int b, int k, int B, bool write,
                                                       uint32_t *planes, float *ub) {
        float m = 0.0f;
        float poison = 0.0f;  // NaN iff some value of the block is inf or NaN
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m = fmaxf(m, fabsf(v[e]));
            poison += v[e] * 0.0f;
        }
        // the four threads of block b are one DPP quad (i = 4b + k)
        m = fmaxf(m, dpp_mov<0xB1>(m));
        m = fmaxf(m, dpp_mov<0x4E>(m));
        poison += dpp_mov<0xB1>(poison);
        poison += dpp_mov<0x4E>(poison);
        // power-of-two block scale 2^e0 with max|x|/2^e0 in (kZmax/2, kZmax]:
        // scaling is exact, so activations with <= 19 significant bits are
        // represented exactly
        // m in [2^(ex-1), 2^ex) (hardware frexp: exact for every finite m)
        const int ex = __builtin_amdgcn_frexp_expf(m);
        int e0 = ex - 19;
        if (__builtin_amdgcn_ldexpf(m, -e0) > kZmax) e0 += 1;
        // blocks below 2^-108 keep the largest finite scale 2^127 (their
        // digits then resolve 2^-128 absolute instead of 19 bits relative)
        e0 = max(e0, -127);
        const bool live = m > 0.0f && poison == 0.0f;
        // One FMA per value gives rint(v * 2^-e0) + 0x88888 in the low 20 bits
        // of a float in [2^23, 2^24) (ulp 1, round-to-nearest-even); XOR 0x88888
        // turns its five nibbles into the balanced signed digits.  |v| <= m
        // and m * 2^-e0 <= kZmax keep the value inside the 20-bit field.
        const float s = live ? __builtin_amdgcn_ldexpf(1.0f, -e0) : 0.0f;
        uint32_t L[4], H[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            L[e] = __builtin_bit_cast(uint32_t, fmaf(v[2 * e], s, kMagic)) ^ kBalance;
            H[e] = __builtin_bit_cast(uint32_t, fmaf(v[2 * e + 1], s, kMagic)) ^ kBalance;
        }
        // Nibble transpose: byte e of plane p = digit p of L[e] (low nibble)
        // and of H[e] (high nibble).  M[e] holds planes 0/2/4 in bytes 0/1/2,
        // N[e] planes 1/3 in bytes 0/1; byte permutes gather them.
        uint32_t M[4], Nn[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            M[e] = (L[e] & 0x0F0F0F0Fu) | ((H[e] << 4) & 0xF0F0F0F0u);
            Nn[e] = ((L[e] >> 4) & 0x0F0F0F0Fu) | (H[e] & 0xF0F0F0F0u);
        }
        const uint32_t m01 = __builtin_amdgcn_perm(M[1], M[0], 0x05010400u);
        const uint32_t m23 = __builtin_amdgcn_perm(M[3], M[2], 0x05010400u);
        const uint32_t c01 = __builtin_amdgcn_perm(M[1], M[0], 0x0C0C0602u);
        const uint32_t c23 = __builtin_amdgcn_perm(M[3], M[2], 0x0C0C0602u);
        const uint32_t n01 = __builtin_amdgcn_perm(Nn[1], Nn[0], 0x05010400u);
        const uint32_t n23 = __builtin_amdgcn_perm(Nn[3], Nn[2], 0x05010400u);
        uint32_t w[kPlanes];
        w[0] = __builtin_amdgcn_perm(m23, m01, 0x05040100u);
        w[2] = __builtin_amdgcn_perm(m23, m01, 0x07060302u);
        w[4] = __builtin_amdgcn_perm(c23, c01, 0x05040100u);
        w[1] = __builtin_amdgcn_perm(n23, n01, 0x05040100u);
        w[3] = __builtin_amdgcn_perm(n23, n01, 0x07060302u);
        // non-finite activations poison the block the way f32 arithmetic would
        const float scale = live ? __builtin_amdgcn_ldexpf(1.0f, e0) : poison;
        if (write) {
#pragma unroll
            for (int p = 0; p < kPlanes; ++p) planes[(p * B + b) * 4 + k] = w[p];
            if (k == 0) ub[b] = scale;
        }
    }
};

// sum_j (q_j - 8) * Z_j for one block.  The resident bytes already hold the
// signed nibbles q - 8 (prepack XORs every nibble with 8).  Horner over the
// planes runs inside the dot8 accumulator: T <- dot8 chain seeded with 16*T.
__device__ __forceinline__ int block_dot_digits(u32x4 qs, const uint4 P[kPlanes]) {
    int T = 0;
#pragma unroll
    for (int p = kPlanes - 1; p >= 0; --p) {
        int a = __builtin_amdgcn_sdot8(static_cast<int>(qs[0]), static_cast<int>(P[p].x), T * 16, false);
        a = __builtin_amdgcn_sdot8(static_cast<int>(qs[1]), static_cast<int>(P[p].y), a, false);
        a = __builtin_amdgcn_sdot8(static_cast<int>(qs[2]), static_cast<int>(P[p].z), a, false);
        T = __builtin_amdgcn_sdot8(static_cast<int>(qs[3]), static_cast<int>(P[p].w), a, false);
    }
    return T;
}

// Weight bytes of R rows x NBL blocks per lane, read through a buffer
// descriptor based at the wave's first row: every load is unconditional with
// a 32-bit offset, reads past the tensor end return 0 (buffer range check),
// and blocks past the row end are neutralised by a zero scale, so
// the compiler keeps all requests in flight.
//
// Scales: the F = NBL - TAIL full 64-block columns have lane-major scale
// slots (q4_0_layout.h), so for F in {1, 2, 4, 8} one 2F-byte load fetches a
// lane's scales; other F use one 2-byte load per column.  The tail column
// (TAIL: B % 64 != 0) keeps natural slots; lanes past the row end get 0.
template <int NBL, int R, bool A16, bool TAIL>
struct RowGroup {
    static constexpr int F = NBL - (TAIL ? 1 : 0);
    static constexpr bool WIDE = F == 1 || F == 2 || F == 4 || F == 8;
    static constexpr int DW = WIDE ? (F + 1) / 2 : (F > 0 ? F : 1);
    u32x4 q[R][NBL];
    uint32_t dw[R][DW];  // fp16 bits of the full-column scales
    uint32_t dt[R];      // fp16 bits of the tail-column scale

    // fp16 bits of the scale of block column j of row r
    __device__ __forceinline__ uint32_t d_bits(int r, int j, uint32_t tail_mask) const {
        if (TAIL && j == F) return dt[r] & tail_mask;
        if constexpr (WIDE) return (dw[r][j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
        return dw[r][j] & 0xFFFFu;
    }

    // Lane-dependent parts of the offsets stay in VGPRs (16*lane, 2*F*lane);
    // row and block-column parts go in the scalar soffset operand.
    __device__ __forceinline__ void load(const uint8_t *__restrict__ W, int row0, int N, int B,
                                         int64_t row_bytes, int lane) {
        load_at(row_rsrc(W, row0, N, row_bytes), 0, B, row_bytes, lane);
    }

    // Descriptor based at row row0 whose range ends with row N; a group past
    // the last row gets an empty range: every access is out of range and
    // returns 0 without touching memory.
    __device__ __forceinline__ static __amdgpu_buffer_rsrc_t row_rsrc(const uint8_t *__restrict__ W, int row0, int N,
                                                                      int64_t row_bytes) {
        const uint8_t *base = W + static_cast<int64_t>(row0) * row_bytes;
        const int64_t left = static_cast<int64_t>(N - row0) * row_bytes;
        const uint32_t records =
            left <= 0 ? 0u : static_cast<uint32_t>(left < 0xFFFFFFFFll ? left : 0xFFFFFFFFll);
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, records, kBufferWord3);
    }

    // The R rows starting at byte offset roff0 of the descriptor's range.
    __device__ __forceinline__ void load_at(__amdgpu_buffer_rsrc_t rsrc, int roff0, int B, int64_t row_bytes,
                                            int lane) {
        const int scale_off = 16 * B;
        const int qv = 16 * lane;
        const int dv = 2 * F * lane;
        const int tv = 2 * lane;
        // scales first (one or few loads), then code bytes in the order
        // accumulate() consumes them (block column major)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int roff = roff0 + r * static_cast<int>(row_bytes);
            if constexpr (F == 1) {
                dw[r][0] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, dv, roff + scale_off, 0);
            } else if constexpr (F == 2) {
                dw[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, dv, roff + scale_off, 0);
            } else if constexpr (F == 4) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, dv, roff + scale_off, 0);
                dw[r][0] = v[0];
                dw[r][1] = v[1];
            } else if constexpr (F == 8) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, dv, roff + scale_off, 0);
#pragma unroll
                for (int h = 0; h < 4; ++h) dw[r][h] = v[h];
            } else {
#pragma unroll
                for (int j = 0; j < F; ++j)
                    dw[r][j] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, dv, roff + scale_off + 2 * j, 0);
            }
            if constexpr (TAIL)
                dt[r] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, tv, roff + scale_off + 128 * F, 0);
        }
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int roff = roff0 + r * static_cast<int>(row_bytes);
                if constexpr (A16) {
                    q[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, qv, roff + 1024 * j, kNonTemporal);
                } else {
                    u32x4 v;
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rsrc, qv + 4 * h, roff + 1024 * j, kNonTemporal);
                        const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rsrc, qv + 4 * h + 2, roff + 1024 * j, kNonTemporal);
                        v[h] = lo | (hi << 16);
                    }
                    q[r][j] = v;
                }
            }
        }
    }

    __device__ __forceinline__ void accumulate(float acc[R], const uint4 *planes, const float *ub, int B,
                                               const int bc[NBL], uint32_t tail_mask) const {
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
            // one block column at a time: keeps the scheduler from hoisting
            // every column's digit planes into registers at once
            if (j > 0) __builtin_amdgcn_sched_barrier(0);
            uint4 P[kPlanes];
#pragma unroll
            for (int p = 0; p < kPlanes; ++p) P[p] = planes[p * B + bc[j]];
            const float u = ub[bc[j]];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int T = block_dot_digits(q[r][j], P);
                const float dr = half_bits_to_float(static_cast<uint16_t>(d_bits(r, j, tail_mask)));
                acc[r] = fmaf(dr * u, static_cast<float>(T), acc[r]);
            }
        }
    }
};

// One kernel covers rows whose blocks fit NBL per lane (B <= 64*NBL);
// TAIL <=> B % 64 != 0.  WAVES wavefronts per workgroup: 16 caps a wave at
// 128 VGPRs, 8 at 256.
template <int NBL, int R, int WAVES, bool A16, bool TAIL, bool PF>
__global__ __launch_bounds__(64 * WAVES) void gemv_q4_0_dp_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y, int N, int B,
    int64_t row_bytes, int x_al16) {
    extern __shared__ uint4 lds_dp[];
    uint4 *planes = lds_dp;
    float *ub = reinterpret_cast<float *>(lds_dp + kPlanes * B);
    const int lane = threadIdx.x & 63;
    // wave index made explicitly uniform so row bases and buffer descriptors
    // live in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    constexpr int ROWS = WAVES * R;
    const int n_groups = (N + ROWS - 1) / ROWS;

    int bc[NBL];
#pragma unroll
    for (int j = 0; j < NBL; ++j) bc[j] = min(lane + 64 * j, B - 1);
    const uint32_t tail_mask = lane + 64 * (NBL - 1) < B ? 0xFFFFu : 0u;

    // Order of the prologue: activation loads, then the first group's weight
    // loads (HBM traffic starts with the kernel), then the staging math,
    // which waits only for the activation loads.  Later groups rely on the
    // other wavefronts of the SIMD to cover their latency.
    constexpr int XI = (4 * NBL + WAVES - 1) / WAVES;
    XTile<XI> xt;
    xt.load(x, B, x_al16 != 0);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads first
    int g = blockIdx.x;
    RowGroup<NBL, R, A16, TAIL> grp;
    // unconditional (a missing group reads nothing): a branch here would make
    // the wait before the staging math cover the weight loads as well
    grp.load(W, g * ROWS + wave * R, N, B, row_bytes, lane);
    xt.store(B, reinterpret_cast<uint32_t *>(planes), ub);
    __syncthreads();

    while (g < n_groups) {
        const int row0 = g * ROWS + wave * R;
        const int gn = g + gridDim.x;
        // PF: the next group's bytes are requested before this group is
        // reduced (two register sets in flight per wave)
        RowGroup<NBL, R, A16, TAIL> nxt;
        if constexpr (PF) nxt.load(W, gn * ROWS + wave * R, N, B, row_bytes, lane);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        grp.accumulate(acc, planes, ub, B, bc, tail_mask);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == 0 && row0 + r < N) y[row0 + r] = s;
        }
        g = gn;
        if constexpr (PF) grp = nxt;
        else grp.load(W, g * ROWS + wave * R, N, B, row_bytes, lane);
    }
}

// ---- K-split form -------------------------------------------------------------
// For long matrices the digit-plane reads, not the weight stream, limit the
// per-wave form above: every row re-reads the planes of all its blocks from
// LDS.  Here a wavefront owns one 64-block column (lane = block) of R rows,
// so one plane read serves R rows, and only R code vectors are live, which
// keeps 32 wavefronts per CU resident.  A workgroup holds G row groups x
// NBL columns (G * NBL <= 16 wavefronts); the NBL column partials of a row
// meet in LDS and are added in column order.  Every load of a workgroup's
// rows is issued in the prologue, before the activation staging.
template <int R>
struct ColumnGroup {
    u32x4 q[R];
    uint32_t d[R];  // fp16 bits of this lane's block scale, per row

    __device__ __forceinline__ void load(const uint8_t *__restrict__ W, int row0, int N, int B, int64_t row_bytes,
                                         int b, int slot) {
        const uint8_t *base = W + static_cast<int64_t>(row0) * row_bytes;
        const int64_t left = static_cast<int64_t>(N - row0) * row_bytes;
        const uint32_t records =
            left <= 0 ? 0u : static_cast<uint32_t>(left < 0xFFFFFFFFll ? left : 0xFFFFFFFFll);
        const __amdgpu_buffer_rsrc_t rsrc =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, records, kBufferWord3);
        const int scale_off = 16 * B;
#pragma unroll
        for (int r = 0; r < R; ++r)
            d[r] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, 2 * slot, r * static_cast<int>(row_bytes) + scale_off, 0);
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * b, r * static_cast<int>(row_bytes), kNonTemporal);
    }
};

template <int R, int G, int NBL>
__global__ __launch_bounds__(64 * G * NBL) void gemv_q4_0_ks_kernel(const uint8_t *__restrict__ W,
                                                                    const float *__restrict__ x,
                                                                    float *__restrict__ y, int N, int B,
                                                                    int64_t row_bytes, int x_al16) {
    constexpr int WAVES = G * NBL;
    constexpr int ROWS = G * R;  // rows per workgroup step
    extern __shared__ uint4 lds_dp[];
    uint4 *planes = lds_dp;
    float *ub = reinterpret_cast<float *>(lds_dp + kPlanes * B);
    float *red = ub + B;  // [G][R][NBL] column partials
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int gi = wave / NBL;  // row group of this wavefront
    const int c = wave % NBL;   // block column of this wavefront
    const int n_groups = (N + ROWS - 1) / ROWS;

    // lane's block; past the row end a lane reads the last block and its
    // scale is masked to 0
    const int braw = 64 * c + lane;
    const bool live = braw < B;
    const int b = live ? braw : B - 1;
    const int F = B >> 6;  // full 64-block columns (lane-major scale slots)
    const int slot = b < 64 * F ? (b & 63) * F + (b >> 6) : b;
    const uint32_t dmask = live ? 0xFFFFu : 0u;

    constexpr int XI = (4 * NBL + WAVES - 1) / WAVES;
    XTile<XI> xt;
    xt.load(x, B, x_al16 != 0);
    __builtin_amdgcn_sched_barrier(0);
    int g = blockIdx.x;
    ColumnGroup<R> grp;
    grp.load(W, g * ROWS + gi * R, N, B, row_bytes, b, slot);
    xt.store(B, reinterpret_cast<uint32_t *>(planes), ub);
    __syncthreads();

    uint4 P[kPlanes];
#pragma unroll
    for (int p = 0; p < kPlanes; ++p) P[p] = planes[p * B + b];
    const float u = ub[b];

    while (g < n_groups) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int T = block_dot_digits(grp.q[r], P);
            const float dr = half_bits_to_float(static_cast<uint16_t>(grp.d[r] & dmask));
            const float s = wave_sum(dr * u * static_cast<float>(T));
            if (lane == 0) red[(gi * R + r) * NBL + c] = s;
        }
        const int gn = g + gridDim.x;
        if (gn < n_groups) grp.load(W, gn * ROWS + gi * R, N, B, row_bytes, b, slot);
        __syncthreads();
        if (threadIdx.x < ROWS) {
            const int row = g * ROWS + threadIdx.x;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < NBL; ++j) s += red[threadIdx.x * NBL + j];
            if (row < N) y[row] = s;
        }
        __syncthreads();
        g = gn;
    }
}

// ---- batched form: M activation rows, weights read once ---------------------
// y_m = W x_m for m < M <= MB, reading the weights once.  A staging kernel
// turns every activation into its digit-plane tile (the row form's staging
// math, once per call) in a context buffer.  The batched kernel follows the
// K-split schedule: a wavefront owns one 64-block column (lane = block) of
// R = 2 rows per step and holds its block's planes of every activation in
// registers (20 VGPRs each), so each code vector meets all MB plane sets and
// the main loop touches no LDS but the partial sums.  Code vectors are
// requested kMbDepth steps ahead.  The R x MB partials of a lane go through
// one batched cross-lane reduction; the column partials of a (row,
// activation) are added in column order through LDS.
constexpr int kMbMax = 8;
constexpr int kMbRows = 2;   // rows per wavefront step
constexpr int kMbDepth = 3;  // steps whose code vectors are in flight

// uint4 units of one activation tile: kPlanes planes of B blocks, then B scales
__host__ __device__ constexpr int mb_tile(int B) { return kPlanes * B + (B + 3) / 4; }
// row groups per workgroup: 8 wavefronts at most (register budget of MB = 8)
__host__ __device__ constexpr int mb_groups(int nbl) { return nbl >= 8 ? 1 : 8 / nbl; }

// One thread per 8-value group f = m * 4B + i of activations 0 .. M-1; 4B
// and the workgroup size are multiples of 4, so the DPP quad of a block never
// straddles two activations.
__global__ __launch_bounds__(256) void q4_0_mb_stage_kernel(const float *__restrict__ x, int64_t x_stride, int M,
                                                            int B, int x_al16, uint4 *__restrict__ tiles) {
    const int gpa = 4 * B;
    const int total = M * gpa;
    const int fr = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int f = min(fr, total - 1);
    const int m = f / gpa, i = f - m * gpa;
    const float *xb = x + m * x_stride + 32 * (i >> 2) + 4 * (i & 3);
    float v[8];
    if (x_al16) {
        const float4 lo = *reinterpret_cast<const float4 *>(xb);
        const float4 hi = *reinterpret_cast<const float4 *>(xb + 16);
        v[0] = lo.x; v[1] = hi.x; v[2] = lo.y; v[3] = hi.y;
        v[4] = lo.z; v[5] = hi.z; v[6] = lo.w; v[7] = hi.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = xb[e];
            v[2 * e + 1] = xb[16 + e];
        }
    }
    uint4 *t = tiles + static_cast<int64_t>(m) * mb_tile(B);
    XTile<1>::stage_group(v, i >> 2, i & 3, B, fr < total, reinterpret_cast<uint32_t *>(t),
                          reinterpret_cast<float *>(t + kPlanes * B));
}

template <int NBL, int MB>
__global__ __launch_bounds__(64 * 8) void gemv_q4_0_mb_kernel(const uint8_t *__restrict__ W,
                                                              const uint4 *__restrict__ tiles,
                                                              float *__restrict__ y, int64_t y_stride, int N,
                                                              int B, int64_t row_bytes, int M) {
    constexpr int R = kMbRows;
    constexpr int G = mb_groups(NBL);
    constexpr int ROWS = G * R;  // rows per workgroup step
    constexpr int S = R * MB;    // partials per lane per step
    static_assert(S == 4 || S == 8 || S == 16, "batched reduction size");
    __shared__ float red[G * S * NBL];  // [G][R][MB][NBL]
    const int tile = mb_tile(B);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int gi = wave / NBL;  // row group of this wavefront
    const int c = wave % NBL;   // block column of this wavefront
    const int n_groups = (N + ROWS - 1) / ROWS;

    // lane's block (as the K-split form): past the row end a lane reads the
    // last block and its weight scale is masked to 0
    const int braw = 64 * c + lane;
    const bool live = braw < B;
    const int b = live ? braw : B - 1;
    const int F = B >> 6;
    const int slot = b < 64 * F ? (b & 63) * F + (b >> 6) : b;
    const uint32_t dmask = live ? 0xFFFFu : 0u;

    // the first kMbDepth steps' code vectors (an empty range past the end)
    int g = blockIdx.x;
    ColumnGroup<R> ring[kMbDepth];
#pragma unroll
    for (int d = 0; d < kMbDepth; ++d)
        ring[d].load(W, (g + d * static_cast<int>(gridDim.x)) * ROWS + gi * R, N, B, row_bytes, b, slot);

    // this lane's block of every activation; slots m >= M repeat the last
    // activation (their partials are never stored)
    uint4 P[MB][kPlanes];
    float u[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const uint4 *t = tiles + min(m, M - 1) * tile;
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) P[m][p] = t[p * B + b];
        u[m] = reinterpret_cast<const float *>(t + kPlanes * B)[b];
    }

    // steps g, g + grid, ... in turns of kMbDepth; a step's slot of the ring
    // is refilled with the step kMbDepth ahead once its dot products are done
    for (; g < n_groups; g += kMbDepth * static_cast<int>(gridDim.x)) {
#pragma unroll
        for (int d = 0; d < kMbDepth; ++d) {
            const int gd = g + d * static_cast<int>(gridDim.x);
            if (gd >= n_groups) break;  // uniform across the workgroup
            float part[S];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float dr = half_bits_to_float(static_cast<uint16_t>(ring[d].d[r] & dmask));
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    const int T = block_dot_digits(ring[d].q[r], P[m]);
                    part[r * MB + m] = dr * u[m] * static_cast<float>(T);
                }
            }
            ring[d].load(W, (gd + kMbDepth * static_cast<int>(gridDim.x)) * ROWS + gi * R, N, B, row_bytes, b,
                         slot);
            // lane l ends with the column total of partial l >> (6 - log2 S)
            const float tot = st_reduce<S>(part, lane);
            constexpr int SPAN = 64 / S;
            if ((lane & (SPAN - 1)) == 0) red[((gi * S) + lane / SPAN) * NBL + c] = tot;
            __syncthreads();
            // one thread per (row, activation) of the step adds the columns in order
            if (threadIdx.x < ROWS * MB) {
                const int k = threadIdx.x;  // = (g_i * R + r) * MB + m
                const int m = k % MB;
                const int row = gd * ROWS + k / MB;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < NBL; ++j) s += red[k * NBL + j];
                if (m < M && row < N) y[m * y_stride + row] = s;
            }
            __syncthreads();
        }
    }
}

// ---- ggml-cpu numerics ------------------------------------------------------
// ggml's CPU backend does not multiply Q4_0 weights by f32 activations: it
// quantizes the activation row to Q8_0 and takes integer block dot
// products (quantize_row_q8_0 and ggml_vec_dot_q4_0_q8_0 of ggml, llama.cpp
// 0ec4027a2; ggml is not part of the reference).  gemv_q4_0_q8_kernel and
// the server's Q8_0 job form reproduce that arithmetic so that decode can
// pick ggml-cpu's tokens:
//   staging, per 32-value block (a DPP quad of 4 threads, as the digit
//   staging): amax = max|x_j|, d = amax / 127, id = d ? 1/d : 0,
//   q_j = roundf(x_j * id), d_x = f32(fp16(d)) (round to even), S = sum q_j;
//   LDS holds the codes as two planes Q[h][b] (uint4; byte e of dword k is
//   value 16h + 4k + e, the nibble order of the Q4_0 code dwords), d_x and S;
//   per block: sumi = sum_j (q4_j - 8) q8_j  (exact: v_dot4_i32_i8 on the
//   unsigned nibbles, minus 8 S), contribution (float(sumi) * d_w) * d_x,
//   ggml's expression order.  Blocks are summed per lane, then across the
//   wavefront: the same products as ggml's generic path, re-associated.
template <int XI>
__device__ __forceinline__ void q8_stage(const XTile<XI> &xt, int B, uint32_t *Q, float *dx, int *sx) {
#pragma clang fp contract(off)
#pragma unroll
    for (int it = 0; it < XI; ++it) {
        const int i = threadIdx.x + it * blockDim.x;
        const int ic = min(i, 4 * B - 1);
        const int b = ic >> 2, k = ic & 3;
        // XTile order: v[2e] = value 4k+e, v[2e+1] = value 16+4k+e
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xt.v[it][e]));
        amax = fmaxf(amax, dpp_mov<0xB1>(amax));
        amax = fmaxf(amax, dpp_mov<0x4E>(amax));
        // correctly rounded division, reciprocal and products, as ggml's C
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        uint32_t lo = 0, hi = 0;
        int sum = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int ql = static_cast<int>(roundf((xt.v[it][2 * e] * id)));
            const int qh = static_cast<int>(roundf((xt.v[it][2 * e + 1] * id)));
            lo |= (static_cast<uint32_t>(ql) & 0xFFu) << (8 * e);
            hi |= (static_cast<uint32_t>(qh) & 0xFFu) << (8 * e);
            sum += ql + qh;
        }
        sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, false);
        sum += __builtin_amdgcn_update_dpp(0, sum, 0x4E, 0xF, 0xF, false);
        if (i < 4 * B) {
            Q[b * 4 + k] = lo;
            Q[(B + b) * 4 + k] = hi;
            if (k == 0) {
                dx[b] = static_cast<float>(static_cast<_Float16>(d));
                sx[b] = sum;
            }
        }
    }
}

// Block contributions (float(sumi) * d_w) * d_x of R rows into
// cs[r * cs_stride + b] (blocks past the row end are not written).
template <int NBL, int R, bool A16, bool TAIL>
__device__ __forceinline__ void q8_blocks(const RowGroup<NBL, R, A16, TAIL> &g, float *cs, int cs_stride,
                                          const uint4 *Q, const float *dx, const int *sx, int B, int lane,
                                          const int bc[NBL], uint32_t tail_mask) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < NBL; ++j) {
        if (j > 0) __builtin_amdgcn_sched_barrier(0);
        const uint4 q0 = Q[bc[j]], q1 = Q[B + bc[j]];
        const float d_x = dx[bc[j]];
        const int s8 = sx[bc[j]];
        const uint32_t a[4] = {q0.x, q0.y, q0.z, q0.w};
        const uint32_t c[4] = {q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int dot = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // resident code bytes hold q - 8 per nibble; XOR 8 gives q
                const uint32_t u = g.q[r][j][k] ^ 0x88888888u;
                dot = __builtin_amdgcn_sdot4(static_cast<int>(u & 0x0F0F0F0Fu), static_cast<int>(a[k]), dot, false);
                dot = __builtin_amdgcn_sdot4(static_cast<int>((u >> 4) & 0x0F0F0F0Fu), static_cast<int>(c[k]), dot,
                                             false);
            }
            const int sumi = dot - 8 * s8;
            const float dw = half_bits_to_float(static_cast<uint16_t>(g.d_bits(r, j, tail_mask)));
            if (lane + 64 * j < B)
                cs[r * cs_stride + lane + 64 * j] = (static_cast<float>(sumi) * dw) * d_x;
        }
    }
}

// ---- persistent server form (decode loops) ------------------------------------
// A decode loop issues one GEMV group at a time and waits for it; launch and
// completion then cost more than the kernel.  The server form keeps one
// workgroup per CU resident (cooperative launch) and takes commands from
// pinned host memory:
//   host: x -> pinned buffer, jobs -> command record, then the command number
//         (seq, with K) last; waits for the completion word to reach seq;
//   workgroup 0: polls seq over PCIe and republishes it in device memory,
//         where the other workgroups poll it;
//   every workgroup: reads the command and x through system-coherent
//         accesses (never a stale cached line; polls carry no fences, as a
//         fence at agent or system scope invalidates the whole L2), stages
//         x's digit planes in LDS, computes its contiguous share of
//         each job's rows with the row form's arithmetic (bit-identical to
//         MI355X_FORM_ROWS), writes outputs through to memory and waits for
//         them, then one arrival on a
//         per-XCD counter in device memory; the last arrival of a group
//         arrives on the top counter, and the last of those stores seq into
//         the completion word.
// Every wait is bounded: the kernel exits on an exit command or after
// kSrvIdleTicks without one (workgroup 0 then tells the others), so the grid
// always drains.
constexpr int kSrvMaxJobs = 4;
constexpr int kSrvWaves = 8;
constexpr uint64_t kSrvClockHz = 100000000ull;  // s_memrealtime

struct SrvJob {
    const uint8_t *W;
    float *y;
    int64_t N;
};

struct SrvCmd {
    uint64_t seqk;  // command number | K << 32, written last by the host
    uint32_t exit;
    int32_t K;
    int32_t njobs;
    int32_t mode;  // kSrvDigits or kSrvGgmlQ8
    SrvJob jobs[kSrvMaxJobs];
    // how the store pass writes job 0's rows (kSrvStore*) and, for the
    // residual kinds, the vector added to them
    int32_t kind;
    int32_t stage;  // the stage's number within its command (phase stamps)
    const float *add;
    // SwiGLU command (K2 > 0): jobs 0 and 1 are the gate and up matrices,
    // both of K2 rows and both with y = h; the first stage writes
    // h = silu(gate x) * (up x) instead of their outputs (kind
    // kSrvStoreGlu), every workgroup waits at a grid barrier, and the second
    // stage computes down h (K2 columns).  K2 == 0: one stage.
    int32_t K2;
    int32_t H;  // block command: rows of pre and columns of gate / up
    float *h;
    SrvJob down;
    // block command (pre.N > 0): before the SwiGLU stages, r = resid +
    // pre x (pre: H rows, K columns; resid: the H floats after x in the
    // payload) into r_dev, a grid barrier, then xn = rmsnorm(r) * norm_w
    // (eps) as the gate / up activation; the down stage writes y = r + down h.
    SrvJob pre;
    float *r_dev;
    const float *norm_w;
    float eps;
    int32_t pad2_;
    // block command with a next stage (post.N > 0): the down stage also
    // writes y into r_dev; after a grid barrier, post (H columns) runs over
    // rmsnorm(y) * post_norm_w (eps) into post.y
    SrvJob post;
    const float *post_norm_w;
    // residual store kinds: also write the result here (device memory)
    float *mirror;
    // rows per share unit of this stage's jobs: 16 (one 64-byte line of y,
    // for outputs in pinned host memory) or, with unit8, 8 (device outputs)
    int32_t unit8;
    // block command: the residual is resid_dev (device) instead of the H
    // floats after x in the payload; the down stage writes y + into
    // resid_dev (and into down.y unless it is null)
    int32_t resid_on_dev;
    float *resid_dev;
};
// store-pass kinds
constexpr int32_t kSrvStoreY = 0;     // y[row] = out
constexpr int32_t kSrvStoreGlu = 1;   // h[row] = silu(out of job 0) * out of job 1
constexpr int32_t kSrvStoreAddL = 2;  // y[row] = out + add[row], add in this workgroup's LDS
// job arithmetic: the row form's digit planes, or ggml-cpu's Q8_0 numerics
constexpr int32_t kSrvDigits = 0;
constexpr int32_t kSrvGgmlQ8 = 1;

// device-memory state, one 128-byte line per word that is polled or counted
struct SrvDev {
    uint32_t seq[32];
    uint32_t quit[32];
    uint64_t group[8][16];
    uint64_t top[16];
    // grid barrier of multi-stage commands, one slot per workgroup (the
    // host refuses grids of more than kSrvBarSlots workgroups): each
    // workgroup stores its barrier count, one wavefront reads them all
    uint32_t bar_slot[1024];
    SrvCmd cmd;  // copy of the current command record
};

__device__ __forceinline__ uint64_t srv_clock() { return __builtin_amdgcn_s_memrealtime(); }

// Phase timestamps of server commands, in builds with MI355X_SRV_STAMPS only
// (the stamps library, xdna.cpp_amd/server_phases.py): thread 0 of each of
// the first 256 workgroups records s_memrealtime at fixed points of the last
// 64 commands; mi355x_server_stamps copies the table out.  Slots: 0 command
// seen, 1 record and x read, 2 + 2s / 3 + 2s stage s staged / rows done,
// 10 last stores done, 11 arrived, 12 completion stored (the last arrival),
// 12 + s stage s's barrier passed (s >= 1), 16 / 17 / 18 RMSNorm: r read,
// sums done, done (the last RMSNorm of the command).
#ifdef MI355X_SRV_STAMPS
constexpr int kSrvStampSlots = 20;
__device__ uint64_t g_srv_stamps[64][256][kSrvStampSlots];
__shared__ uint32_t s_srv_cmd;
#define SRV_STAMP(cmd, k)                                                                                         \
    do {                                                                                                          \
        if (threadIdx.x == 0 && blockIdx.x < 256)                                                                 \
            g_srv_stamps[(cmd) & 63][blockIdx.x][k] = __builtin_amdgcn_s_memrealtime();                           \
    } while (0)
#define SRV_CMD() s_srv_cmd
#else
#define SRV_STAMP(cmd, k) \
    do {                  \
    } while (0)
#define SRV_CMD() 0u
#endif

// Cache policy sc0 sc1 (system coherent): the load reads host memory itself,
// never a line a GPU cache kept from an earlier command.
constexpr int kSysCoherent = 1 | 16;
constexpr int kSrvCopyDepth = 8;  // 16-byte pieces of x in flight per thread (K <= 16384)

// XTile::load for the device copy of the activation, through the system-
// coherent path, so no L2 line kept from an earlier command is read (group i
// of this thread: block i / 4, dword i % 4, clamped).
template <int XI>
__device__ __forceinline__ void srv_load_x(XTile<XI> &xt, const float *x, int B) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(x), 0, static_cast<uint32_t>(128 * B), kBufferWord3);
#pragma unroll
    for (int it = 0; it < XI; ++it) {
        const int i = min(static_cast<int>(threadIdx.x + it * blockDim.x), 4 * B - 1);
        const int off = 4 * (32 * (i >> 2) + 4 * (i & 3));
        const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kSysCoherent);
        const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 64, 0, kSysCoherent);
        // copy the elements out before bit-casting: clang lowers a bit cast
        // of a vector element lvalue as a load from the vector's base
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t l = lo[e], h = hi[e];
            xt.v[it][2 * e] = __builtin_bit_cast(float, l);
            xt.v[it][2 * e + 1] = __builtin_bit_cast(float, h);
        }
    }
}

// Outputs of one job are gathered in LDS and written out together: one
// workgroup's rows are contiguous, so the stores of a wavefront cover 256
// contiguous bytes (written through to memory one 4-byte row at a time they
// would cost a PCIe transaction each when y is host memory).
constexpr int kSrvOutMax = 4096;  // rows of a command's jobs per workgroup (padded)

// A workgroup's rows of a command's jobs as one local row space: job j's
// share [lo_j, hi_j) of its N_j rows takes local rows [start_j, start_j +
// hi_j - lo_j), each job's segment padded to a multiple of ROWS so that a
// wavefront's group of R rows never spans two jobs.  A wavefront walks its
// groups wave * R + k * ROWS through every job in one sequence, so the next
// group's loads are in flight across job boundaries too, and the outputs of
// all jobs are stored once at the end.  Indices are uniform; the per-job
// values sit in registers behind constant-index selects.
// A workgroup's share [lo, hi) of a job's N rows: a run of whole units of
// `unit` outputs, the first ending at y's first unit boundary.  16 outputs
// are one 64-byte line: workgroups that stored parts of one line of pinned
// host memory would serialise on it (~6 us per job of small shares); for
// outputs in device memory 8 spreads short jobs over twice the workgroups.
// (32-bit arithmetic: N < 2^27 and G <= 1024, which the host checks through
// the rows a workgroup holds, keep U * G below 2^32.)
__device__ __forceinline__ void srv_share(int64_t N64, const float *y, int g, int G, int &lo, int &hi,
                                          uint32_t unit = 16) {
    const uint32_t N = static_cast<uint32_t>(N64);
    const uint32_t b0 = (unit - (static_cast<uint32_t>(reinterpret_cast<uintptr_t>(y)) >> 2)) & (unit - 1);
    const uint32_t U = 1 + (N > b0 ? N - b0 + unit - 1 : 0) / unit;
    auto at = [&](uint32_t u) { return u == 0 ? 0u : min(N, b0 + unit * (u - 1)); };
    lo = static_cast<int>(at(U * static_cast<uint32_t>(g) / static_cast<uint32_t>(G)));
    hi = static_cast<int>(at(U * static_cast<uint32_t>(g + 1) / static_cast<uint32_t>(G)));
}

template <int ROWS>
struct SrvSpan {
    static_assert(kSrvMaxJobs == 4, "four jobs per command");
    // separate scalars, not arrays: a select over an array becomes an
    // indexed load from scratch memory
    int lo0, lo1, lo2, lo3, hi0, hi1, hi2, hi3, st1, st2, st3, tot;
    __device__ __forceinline__ SrvSpan(const SrvCmd &c, int g, int G) {
        const int n = c.njobs;
        auto share = [&](int j, int &lo, int &hi) {
            lo = hi = 0;
            if (j < n) srv_share(c.jobs[j].N, c.jobs[j].y, g, G, lo, hi, c.unit8 ? 8u : 16u);
        };
        share(0, lo0, hi0);
        share(1, lo1, hi1);
        share(2, lo2, hi2);
        share(3, lo3, hi3);
        auto pad = [](int a) { return (a + ROWS - 1) / ROWS * ROWS; };
        st1 = pad(hi0 - lo0);
        st2 = st1 + pad(hi1 - lo1);
        st3 = st2 + pad(hi2 - lo2);
        tot = st3 + pad(hi3 - lo3);
    }
    __device__ __forceinline__ int total() const { return tot; }
    // job of local row L < total()
    __device__ __forceinline__ int job_of(int L) const {
        return (L >= st1 ? 1 : 0) + (L >= st2 ? 1 : 0) + (L >= st3 ? 1 : 0);
    }
    __device__ __forceinline__ int lo_of(int j) const { return j == 0 ? lo0 : j == 1 ? lo1 : j == 2 ? lo2 : lo3; }
    __device__ __forceinline__ int hi_of(int j) const { return j == 0 ? hi0 : j == 1 ? hi1 : j == 2 ? hi2 : hi3; }
    __device__ __forceinline__ int start_of(int j) const { return j == 0 ? 0 : j == 1 ? st1 : j == 2 ? st2 : st3; }
    // loads of the group at local row L (past the end: an empty range)
    template <class Grp>
    __device__ __forceinline__ void load(Grp &grp, const SrvCmd &c, int L, int B, int64_t row_bytes,
                                         int lane) const {
        const bool live = L < tot;
        const int j = live ? job_of(L) : 0;
        const int row = live ? lo_of(j) + (L - start_of(j)) : 0;
        grp.load(c.jobs[j].W, row, live ? hi_of(j) : 0, B, row_bytes, lane);
    }
    // every job's outputs from out[start_j + i], system-scope stores
    // (written through to memory, so the command completes without an L2
    // write-back)
    __device__ __forceinline__ void store(const SrvCmd &c, const float *out) const {
        auto one = [&](int j, int lo, int hi, int st) {
            float *y = c.jobs[j].y;
            const int n = j < c.njobs ? hi - lo : 0;
            for (int i = threadIdx.x; i < n; i += blockDim.x)
                __hip_atomic_store(&y[lo + i], out[st + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        };
        one(0, lo0, hi0, 0);
        one(1, lo1, hi1, st1);
        one(2, lo2, hi2, st2);
        one(3, lo3, hi3, st3);
    }
};

// Grid barrier inside a command (`n` = barriers this launch has passed, this
// one included).  A workgroup's arrival is one store of its barrier count
// into its own word (256 arrivals on one atomic counter serialised at ~25 ns
// each, measured), and wavefront 0 of every workgroup waits until every
// word of the grid has reached the count, reading all of them (4 per lane,
// system-coherent loads) per poll.  The arrival is ordered after the
// workgroup's stores of the stage by s_waitcnt(0) + __syncthreads() (the
// stores are write-through at system scope: acknowledged once memory holds
// them), not by a release fence, which would write back the whole L2.
// Bounded like every wait: srv_wait_slot returns 1 (and raises quit) after
// `limit` ticks or when quit is raised.
constexpr int kSrvBarSlots = 1024;
__device__ __forceinline__ void srv_arrive_slot(SrvDev *dev, int g, uint64_t n) {
    __hip_atomic_store(&dev->bar_slot[g], static_cast<uint32_t>(n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// wavefront 0 of the workgroup (all its lanes); 0 once every slot reached n
__device__ __forceinline__ uint32_t srv_wait_slot(SrvDev *dev, int G, uint64_t n, uint64_t limit) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(dev->bar_slot, 0, static_cast<uint32_t>(4 * G), kBufferWord3);
    const uint32_t want = static_cast<uint32_t>(n);
    const uint64_t t0 = srv_clock();
    for (;;) {
        bool ok = true;
        for (int i = 4 * lane; i < G; i += 256) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * i, 0, kSysCoherent);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t u = v[e];
                ok = ok && (i + e >= G || static_cast<int32_t>(u - want) >= 0);
            }
        }
        if (__all(ok)) return 0;
        if (__hip_atomic_load(&dev->quit[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 || srv_clock() - t0 > limit) {
            if (lane == 0) __hip_atomic_store(&dev->quit[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return 1;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// RMSNorm of the block command, every workgroup for itself: r (H floats,
// written by other workgroups in this command; plus r2 when given, one f32
// add) into rb, then
// xn[i] = r[i] * s * w[i] into xnb with s = 1 / sqrt(float(ss / H) + eps), the
// f32 steps and the summation order of the decode host's rmsnorm: ss in
// double as 16 partial sums p_k = sum over i0 = 0, 16, ... of r[i0 + k]^2
// (sequential; a square of a float is exact in double), combined as
// ((p0+p4)+(p8+p12)) + ((p1+p5)+(p9+p13)) + ... lane-wise, then
// (l0 + l1) + (l2 + l3).  H: a multiple of 256.
__device__ __forceinline__ void srv_rmsnorm(const float *r, const float *r2, const float *w, float eps, int H,
                                            float *rb, float *xnb, double *pbuf, float *sbuf) {
#pragma clang fp contract(off)
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(r), 0, static_cast<uint32_t>(4 * H), kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(r2 ? r2 : r), 0,
                                                                        static_cast<uint32_t>(4 * H), kBufferWord3);
    // r into rb, and transposed into xnb (free until the end): partial sum k's
    // elements r[k], r[16 + k], ... side by side at xnb[k * H / 16 ..], so its
    // lane reads them 4 at a time (rows L + 4 floats apart: 16-byte aligned,
    // and the 16 rows start in different banks)
    const int L = H / 16, LS = L + 4;
    for (int i = 4 * static_cast<int>(threadIdx.x); i < H; i += 4 * static_cast<int>(blockDim.x)) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * i, 0, kSysCoherent);
        const u32x4 v2 = __builtin_amdgcn_raw_buffer_load_b128(rs2, 4 * i, 0, kSysCoherent);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t u = v[e], u2 = v2[e];
            const float f = r2 ? __builtin_bit_cast(float, u) + __builtin_bit_cast(float, u2) : __builtin_bit_cast(float, u);
            rb[i + e] = f;
            xnb[((i + e) & 15) * LS + ((i + e) >> 4)] = f;
        }
    }
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 16);
    if (threadIdx.x < 16) {
        const float4 *q = reinterpret_cast<const float4 *>(xnb + threadIdx.x * LS);  // L: a multiple of 16
        double p = 0.0;
#pragma unroll 4
        for (int j = 0; j < L / 4; ++j) {
            const float4 f = q[j];
            const double a = f.x, b = f.y, c = f.z, d = f.w;
            p = __builtin_fma(a, a, p);
            p = __builtin_fma(b, b, p);
            p = __builtin_fma(c, c, p);
            p = __builtin_fma(d, d, p);
        }
        pbuf[threadIdx.x] = p;
    }
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 17);
    if (threadIdx.x == 0) {
        double l[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) l[k] = (pbuf[k] + pbuf[4 + k]) + (pbuf[8 + k] + pbuf[12 + k]);
        const double ss = (l[0] + l[1]) + (l[2] + l[3]);
        *sbuf = 1.0f / sqrtf(static_cast<float>(ss / H) + eps);
    }
    __syncthreads();
    const float sc = *sbuf;
    for (int i = threadIdx.x; i < H; i += blockDim.x) xnb[i] = rb[i] * sc * w[i];
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 18);
}

// What a stage waits for between requesting its first weight rows and
// reading its activation: the grid barrier after the stage before (whose
// stores must be complete: they are waited for before the arrival, so the
// new row loads are issued after it and arrive during the wait), then the
// block command's RMSNorm.  One type for every stage (runtime fields), so
// the row functions are instantiated once.
struct SrvPre {
    bool barrier = false;
    SrvDev *dev = nullptr;
    int g = 0, G = 1;
    uint64_t n = 0, limit = 0;  // barrier number, wait bound in ticks
    uint32_t *verdict = nullptr;
    int stage = 0;
    const float *norm_r = nullptr;  // RMSNorm of norm_r (+ norm_r2) when set
    const float *norm_r2 = nullptr, *norm_w = nullptr;
    float eps = 0.0f;
    int H = 0;
    float *rb = nullptr, *xnb = nullptr, *sbuf = nullptr;
    double *pbuf = nullptr;
    __device__ __forceinline__ void arrive() const {
        if (!barrier) return;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) srv_arrive_slot(dev, g, n);
    }
    // true: leave (the barrier timed out or quit was raised)
    __device__ __forceinline__ bool wait() const {
        if (barrier) {
            if (threadIdx.x < 64) {
                const uint32_t v = srv_wait_slot(dev, G, n, limit);
                if (threadIdx.x == 0) *verdict = v;
            }
            __syncthreads();
            SRV_STAMP(SRV_CMD(), 12 + stage);
            if (*verdict) return true;
        }
        if (norm_r) srv_rmsnorm(norm_r, norm_r2, norm_w, eps, H, rb, xnb, pbuf, sbuf);
        return false;
    }
};

// silu(g) * u = g / (1 + e^-g) * u, each step one IEEE f32 operation as
// written (contraction off, fmas explicit), so a host that performs the same
// steps gets the same bits.  e^t: t clamped to [-87.3, 88]; n = t / ln2
// rounded to an integer (one fma against 1.5 * 2^23); r = t - n ln2 in two
// fmas (ln2 split into a part exact in f32 and a remainder); e^r by its
// degree-7 Taylor polynomial in Horner fmas (|r| <= ln2 / 2: relative error
// < 5e-9); times 2^n from the exponent bits; 0 for t < -87.3.
__device__ __forceinline__ float srv_silu_mul(float g, float u) {
#pragma clang fp contract(off)
    const float t = -g;
    const float tc = fminf(fmaxf(t, -87.3f), 88.0f);
    const float n = __builtin_fmaf(tc, 1.44269504088896341f, 12582912.0f) - 12582912.0f;
    float r = __builtin_fmaf(-n, 0.693145751953125f, tc);
    r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float e = p * __builtin_bit_cast(float, (static_cast<int32_t>(n) + 127) << 23);
    const float ex = t < -87.3f ? 0.0f : e;
    return g / (1.0f + ex) * u;
}

// The store pass of a SwiGLU command's first stage: jobs 0 and 1 (gate and
// up) have the same rows and the same y, so a workgroup holds the same share
// [lo0, hi0) of both, at out[0 ..] and out[st1 ..]; it writes
// h[i] = silu(gate_i) * up_i for its share (system-scope stores).
template <int ROWS>
__device__ __forceinline__ void srv_store_glu(const SrvSpan<ROWS> &sp, const SrvCmd &c, const float *out) {
    const int n = sp.hi0 - sp.lo0;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        __hip_atomic_store(&c.h[sp.lo0 + i], srv_silu_mul(out[i], out[sp.st1 + i]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// Residual store pass (one job): y[lo0 + i] = out[i] + add[lo0 + i], add
// in this workgroup's LDS; with c.mirror, the sums also go there.
template <int ROWS>
__device__ __forceinline__ void srv_store_add(const SrvSpan<ROWS> &sp, const SrvCmd &c, const float *out) {
#pragma clang fp contract(off)
    const int n = sp.hi0 - sp.lo0;
    float *y = c.jobs[0].y;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int r = sp.lo0 + i;
        const float v = out[i] + c.add[r];
        __hip_atomic_store(&y[r], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (c.mirror) __hip_atomic_store(&c.mirror[r], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

template <int ROWS>
__device__ __forceinline__ void srv_store(const SrvSpan<ROWS> &sp, const SrvCmd &c, const float *out) {
    if (c.kind == kSrvStoreGlu) srv_store_glu(sp, c, out);
    else if (c.kind == kSrvStoreY) sp.store(c, out);
    else srv_store_add(sp, c, out);
}

// The activation of a stage: from device memory written in this command
// (the system-coherent path), or (XL) from this workgroup's LDS.
template <bool XL, int XI>
__device__ __forceinline__ void srv_activation(XTile<XI> &xt, const float *x, int B) {
    if constexpr (XL) xt.load(x, B, true);
    else srv_load_x(xt, x, B);
}

// A wavefront requests its next row group before computing the current one,
// except for rows of more than 6 block columns (K > 12288): two groups of
// those would raise the server kernel's register count (one for all its
// forms) above what leaves room on each CU for other kernels, such as HIP's
// copy kernels, while the server is resident.
template <int NBL>
constexpr bool kSrvNextGroup = NBL <= 6;

template <int NBL, bool TAIL, bool XL>
__device__ __forceinline__ bool srv_rows(const SrvCmd &c, int B, uint4 *lds, const float *__restrict__ x,
                                         float *out, const SrvPre &pre) {
    constexpr int R = NBL <= 1 ? 4 : (NBL == 2 ? 2 : 1);
    constexpr int ROWS = kSrvWaves * R;
    constexpr int XI = (4 * NBL + kSrvWaves - 1) / kSrvWaves;
    uint4 *planes = lds;
    float *ub = reinterpret_cast<float *>(lds + kPlanes * B);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t row_bytes = 18 * static_cast<int64_t>(B);
    int bc[NBL];
#pragma unroll
    for (int j = 0; j < NBL; ++j) bc[j] = min(lane + 64 * j, B - 1);
    const uint32_t tail_mask = lane + 64 * (NBL - 1) < B ? 0xFFFFu : 0u;
    const SrvSpan<ROWS> sp(c, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int T = sp.total();

    // the first group's rows are requested before the wait and the
    // staging math
    pre.arrive();
    RowGroup<NBL, R, true, TAIL> grp;
    sp.load(grp, c, wave * R, B, row_bytes, lane);
    if (pre.wait()) return false;
    XTile<XI> xt;
    srv_activation<XL>(xt, x, B);
    xt.store(B, reinterpret_cast<uint32_t *>(planes), ub);
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 2 + 2 * c.stage);

    for (int L = wave * R; L < T; L += ROWS) {
        RowGroup<NBL, R, true, TAIL> nxt;
        if constexpr (kSrvNextGroup<NBL>) sp.load(nxt, c, L + ROWS, B, row_bytes, lane);
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        grp.accumulate(acc, planes, ub, B, bc, tail_mask);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == 0) out[L + r] = s;  // padding rows (zero loads) are never stored
        }
        if constexpr (kSrvNextGroup<NBL>) grp = nxt;
        else sp.load(grp, c, L + ROWS, B, row_bytes, lane);
    }
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 3 + 2 * c.stage);
    srv_store(sp, c, out);
    return true;
}

// ggml-cpu numerics job form (MI355X_VARIANT_GGML_Q8): the arithmetic of
// gemv_q4_0_q8_kernel, bit for bit.  The activation row is staged as Q8_0
// codes; a workgroup takes its rows of a job in chunks whose block
// contributions fit kSrvCsFloats of LDS; within a chunk wavefront v computes
// runs of R rows (the row form's R: 4 for one block column, 2 for two, 1
// beyond) v*R, v*R + 8R, ... (lane = block, the next run's loads in flight)
// and stores (float(sumi) * d_w) * d_x per block; then one thread per row adds
// its row's contributions in block order (ggml's sequential sum).  Rows of a
// chunk sit B + 4 floats apart: 16-byte aligned for the sum's vector reads,
// and (B a multiple of 8) an odd number of 16-byte slots, so 16 consecutive
// rows start on 16 different bank groups.
constexpr int kSrvCsFloats = 8192;

template <int NBL, bool TAIL, bool XL>
__device__ __forceinline__ bool srv_rows_q8(const SrvCmd &c, int B, uint4 *lds, const float *__restrict__ x,
                                            float *out, float *csb, const SrvPre &pre) {
#pragma clang fp contract(off)
    constexpr int R = NBL <= 1 ? 4 : (NBL == 2 ? 2 : 1);
    constexpr int ROWS = kSrvWaves * R;
    constexpr int XI = (4 * NBL + kSrvWaves - 1) / kSrvWaves;
    uint4 *Q = lds;
    float *dxs = reinterpret_cast<float *>(lds + 2 * B);
    int *sxs = reinterpret_cast<int *>(dxs + B);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t row_bytes = 18 * static_cast<int64_t>(B);
    const int stride = B + 4;
    // rows per chunk: a multiple of ROWS, so a wavefront's groups continue
    // from one chunk into the next, and at most one per thread (>= ROWS:
    // B <= 64 for R = 4, B <= 128 for R = 2, B <= 512 for R = 1)
    const int chunk = min((kSrvCsFloats / stride) / ROWS * ROWS, 64 * kSrvWaves);
    int bc[NBL];
#pragma unroll
    for (int j = 0; j < NBL; ++j) bc[j] = min(lane + 64 * j, B - 1);
    const uint32_t tail_mask = lane + 64 * (NBL - 1) < B ? 0xFFFFu : 0u;
    const SrvSpan<ROWS> sp(c, static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int T = sp.total();

    pre.arrive();
    using Grp = RowGroup<NBL, R, true, TAIL>;
    Grp grp;
    sp.load(grp, c, wave * R, B, row_bytes, lane);
    if (pre.wait()) return false;
    XTile<XI> xt;
    srv_activation<XL>(xt, x, B);
    q8_stage<XI>(xt, B, reinterpret_cast<uint32_t *>(Q), dxs, sxs);
    __syncthreads();
    SRV_STAMP(SRV_CMD(), 2 + 2 * c.stage);

    for (int c0 = 0; c0 < T; c0 += chunk) {
        const int c1 = min(T, c0 + chunk);
        for (int L = c0 + wave * R; L < c1; L += ROWS) {
            Grp nxt;
            if constexpr (kSrvNextGroup<NBL>) sp.load(nxt, c, L + ROWS, B, row_bytes, lane);
            q8_blocks<NBL, R, true, TAIL>(grp, csb + (L - c0) * stride, stride, Q, dxs, sxs, B, lane, bc,
                                          tail_mask);
            if constexpr (kSrvNextGroup<NBL>) grp = nxt;
            else sp.load(grp, c, L + ROWS, B, row_bytes, lane);
        }
        __syncthreads();
        const int t = static_cast<int>(threadIdx.x);
        if (t < c1 - c0) {
            const int Lt = c0 + t, j = sp.job_of(Lt);
            if (sp.lo_of(j) + (Lt - sp.start_of(j)) < sp.hi_of(j)) out[Lt] = ordered_sum(csb + t * stride, B);
        }
        __syncthreads();  // csb is rewritten by the next chunk
    }
    SRV_STAMP(SRV_CMD(), 3 + 2 * c.stage);
    srv_store(sp, c, out);
    return true;
}

template <int NBL, bool TAIL, bool XL = false>
__device__ __forceinline__ bool srv_job(const SrvCmd &c, int B, uint4 *lds, const float *__restrict__ x,
                                        float *out, float *csb, const SrvPre &pre) {
    if (c.mode == kSrvGgmlQ8) return srv_rows_q8<NBL, TAIL, XL>(c, B, lds, x, out, csb, pre);
    return srv_rows<NBL, TAIL, XL>(c, B, lds, x, out, pre);
}

// A stage whose activation (c.K <= kSrvLdsXMax columns) is in LDS.
constexpr int kSrvLdsXMax = 4096;
__device__ __forceinline__ bool srv_stage_lds(const SrvCmd &c, uint4 *lds, const float *x, float *outb, float *csb,
                                              const SrvPre &pre) {
    const int B = c.K / 32;
    switch ((B + 63) / 64 * 2 + (B % 64 != 0 ? 1 : 0)) {
    case 2: return srv_job<1, false, true>(c, B, lds, x, outb, csb, pre);
    case 3: return srv_job<1, true, true>(c, B, lds, x, outb, csb, pre);
    case 4: return srv_job<2, false, true>(c, B, lds, x, outb, csb, pre);
    default: return srv_job<2, true, true>(c, B, lds, x, outb, csb, pre);  // B < 128 (the host checks K)
    }
}

// One stage of a command: its jobs over the activation x of c.K columns.
__device__ __forceinline__ bool srv_stage(const SrvCmd &c, uint4 *lds, const float *x, float *outb, float *csb,
                                          const SrvPre &pre) {
    const int B = c.K / 32;
    switch ((B + 63) / 64 * 2 + (B % 64 != 0 ? 1 : 0)) {
    case 2: return srv_job<1, false>(c, B, lds, x, outb, csb, pre);
    case 3: return srv_job<1, true>(c, B, lds, x, outb, csb, pre);
    case 4: return srv_job<2, false>(c, B, lds, x, outb, csb, pre);
    case 5: return srv_job<2, true>(c, B, lds, x, outb, csb, pre);
    case 6: return srv_job<3, false>(c, B, lds, x, outb, csb, pre);
    case 7: return srv_job<3, true>(c, B, lds, x, outb, csb, pre);
    case 8: return srv_job<4, false>(c, B, lds, x, outb, csb, pre);
    case 9: return srv_job<4, true>(c, B, lds, x, outb, csb, pre);
    case 10: return srv_job<5, false>(c, B, lds, x, outb, csb, pre);
    case 11: return srv_job<5, true>(c, B, lds, x, outb, csb, pre);
    case 12: return srv_job<6, false>(c, B, lds, x, outb, csb, pre);
    case 13: return srv_job<6, true>(c, B, lds, x, outb, csb, pre);
    case 14: return srv_job<7, false>(c, B, lds, x, outb, csb, pre);
    case 15: return srv_job<7, true>(c, B, lds, x, outb, csb, pre);
    case 16: return srv_job<8, false>(c, B, lds, x, outb, csb, pre);
    default: return srv_job<8, true>(c, B, lds, x, outb, csb, pre);  // 448 < B < 512 (the host checks K <= 16384)
    }
}

// Command-record fields as 32-bit words (the record is copied word by word).
constexpr int kSrvCmdWords = static_cast<int>(sizeof(SrvCmd) / 4);
static_assert(sizeof(SrvCmd) % 4 == 0, "command record in words");
static_assert(kSrvCmdWords <= 64 * kSrvWaves, "one record word per thread");
static_assert(kSrvCopyDepth * 64 * kSrvWaves * 4 >= 16384, "x of K <= 16384 in one batch");

__global__ __launch_bounds__(64 * kSrvWaves) void gemv_q4_0_server_kernel(SrvCmd *cmd, const float *hx,
                                                                            SrvDev *dev, float *dx,
                                                                            uint32_t *done, uint32_t first,
                                                                            uint64_t idle_ticks) {
    extern __shared__ uint4 lds_dp[];
    __shared__ uint32_t verdict;  // 0 run, 1 leave
    __shared__ int32_t shk;       // K of this command (workgroup 0)
    __shared__ SrvCmd cs;         // this command
    __shared__ SrvCmd cs2;        // the later stages of SwiGLU and block commands
    __shared__ __align__(16) float rb[kSrvLdsXMax];   // block command: r
    __shared__ __align__(16) float xnb[kSrvLdsXMax + 64];  // block command: rmsnorm(r) * norm_w
    __shared__ double pbuf[16];
    __shared__ float sbuf;
    __shared__ float outb[kSrvOutMax];
    __shared__ __align__(16) float csb[kSrvCsFloats];  // block contributions (Q8_0 jobs)
    const int G = static_cast<int>(gridDim.x), g = static_cast<int>(blockIdx.x);
    uint32_t *csw = reinterpret_cast<uint32_t *>(&cs);
    uint64_t nbar = 0;  // grid barriers passed in this launch
    for (uint32_t expect = first;; ++expect) {
        if (g == 0) {
            // workgroup 0: wait for the host, then copy the command record
            // and x into device memory (read from and written through to
            // memory itself), and only then publish the command number
            if (threadIdx.x == 0) {
                const uint64_t t0 = srv_clock();
                uint32_t leave = 0;
                for (;;) {
                    const uint64_t s = __hip_atomic_load(&cmd->seqk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    if (static_cast<int32_t>(static_cast<uint32_t>(s) - expect) >= 0) {
                        shk = static_cast<int32_t>(s >> 32);
                        break;
                    }
                    if (srv_clock() - t0 > idle_ticks) {
                        leave = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                verdict = leave;
                SRV_STAMP(expect, 0);
            }
            __syncthreads();
            if (verdict) {
                if (threadIdx.x == 0) __hip_atomic_store(&dev->quit[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
            // the record and x in one round trip: K came with the command
            // number; x in 16-byte pieces, kSrvCopyDepth per thread (one batch,
            // K <= 16384), issued before the record's words so that one wait
            // covers both; stores past the K / 4 pieces fall outside the
            // descriptor's range and are dropped
            const int K4 = __builtin_amdgcn_readfirstlane(shk / 4);  // uniform: descriptors in SGPRs
            const __amdgpu_buffer_rsrc_t hs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(hx), 0, static_cast<uint32_t>(16 * K4), kBufferWord3);
            const __amdgpu_buffer_rsrc_t ds =
                __builtin_amdgcn_make_buffer_rsrc(dx, 0, static_cast<uint32_t>(16 * K4), kBufferWord3);
            u32x4 v[kSrvCopyDepth];
#pragma unroll
            for (int k = 0; k < kSrvCopyDepth; ++k)
                v[k] = __builtin_amdgcn_raw_buffer_load_b128(hs, 16 * (k * 64 * kSrvWaves + static_cast<int>(threadIdx.x)),
                                                             0, kSysCoherent);
            const bool rec = static_cast<int>(threadIdx.x) < kSrvCmdWords;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(cmd);
            const uint32_t w = __hip_atomic_load(&src[rec ? threadIdx.x : 0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (int k = 0; k < kSrvCopyDepth; ++k)
                __builtin_amdgcn_raw_buffer_store_b128(v[k], ds, 16 * (k * 64 * kSrvWaves + static_cast<int>(threadIdx.x)),
                                                       0, kSysCoherent);
            uint32_t *dcw = reinterpret_cast<uint32_t *>(&dev->cmd);
            if (rec) {
                csw[threadIdx.x] = w;
                __hip_atomic_store(&dcw[threadIdx.x], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            __builtin_amdgcn_s_waitcnt(0);  // every copy store has completed
            __syncthreads();  // and the record is in LDS
            if (threadIdx.x == 0) __hip_atomic_store(&dev->seq[0], expect, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            SRV_STAMP(expect, 1);
            if (cs.exit) return;
        } else {
            if (threadIdx.x == 0) {
                const uint64_t t0 = srv_clock();
                uint32_t leave = 0;
                for (;;) {
                    const uint32_t s = __hip_atomic_load(&dev->seq[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (static_cast<int32_t>(s - expect) >= 0) break;
                    if (__hip_atomic_load(&dev->quit[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                        srv_clock() - t0 > 2 * idle_ticks) {
                        leave = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                verdict = leave;
                SRV_STAMP(expect, 0);
            }
            __syncthreads();
            if (verdict) return;
            const uint32_t *dcw = reinterpret_cast<const uint32_t *>(&dev->cmd);
            for (int i = threadIdx.x; i < kSrvCmdWords; i += blockDim.x)
                csw[i] = __hip_atomic_load(&dcw[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __syncthreads();
            SRV_STAMP(expect, 1);
            if (cs.exit) return;
        }
        // cs2 = cs, one word per thread, once every thread is done with the
        // stage before (then thread 0 patches the stage)
        auto copy_cmd = [&]() {
            __syncthreads();
            uint32_t *d = reinterpret_cast<uint32_t *>(&cs2);
            for (int i = threadIdx.x; i < kSrvCmdWords; i += blockDim.x) d[i] = csw[i];
            __syncthreads();
        };
        // stages: plain 1; SwiGLU 2 (gate|up -> h, down); block 3 (pre -> r,
        // gate|up over rmsnorm(r) -> h, down + r), 4 with post (over
        // rmsnorm(down + r)).  Every stage after the first starts with a
        // grid barrier (all workgroups are resident: the launch is
        // cooperative), inside the row functions, after the stage's first
        // rows were requested.  One call site per stage form keeps the
        // kernel's register count at that of one stage.
#ifdef MI355X_SRV_STAMPS
        if (threadIdx.x == 0) s_srv_cmd = expect;
#endif
        const bool blk = cs.pre.N > 0;
        const int nst = blk ? (cs.post.N > 0 ? 4 : 3) : (cs.K2 ? 2 : 1);
        for (int st = 0; st < nst; ++st) {
            SrvPre pre;
            if (st > 0) {
                pre.barrier = true;
                pre.dev = dev;
                pre.g = g;
                pre.G = G;
                pre.n = ++nbar;
                pre.limit = 2 * idle_ticks;
                pre.verdict = &verdict;
                pre.stage = st;
            }
            // r = (pre x) + resid (resid after x in the payload, or in
            // resid_dev); the next stage's r = down h + r, added in the down
            // stage's store pass and kept in resid_dev
            if ((blk && st == 1) || st == 3) {
                pre.norm_r = st == 1 ? cs.r_dev : cs.resid_dev;
                pre.norm_r2 = st == 3 ? nullptr : cs.resid_on_dev ? cs.resid_dev : dx + cs.K;
                pre.norm_w = st == 1 ? cs.norm_w : cs.post_norm_w;
                pre.eps = cs.eps;
                pre.H = cs.H;
                pre.rb = rb;
                pre.xnb = xnb;
                pre.pbuf = pbuf;
                pre.sbuf = &sbuf;
            }
            if (st > 0 || blk || cs.K2) {
                copy_cmd();
                if (threadIdx.x == 0) {
                    cs2.stage = st;
                    if (blk && st == 0) {
                        // block: pre x into r_dev (the residual is added
                        // when every workgroup reads it back)
                        cs2.njobs = 1;
                        cs2.jobs[0] = {cs.pre.W, cs.r_dev, cs.pre.N};
                        cs2.kind = kSrvStoreY;
                        cs2.unit8 = 1;
                    } else if (st == (blk ? 1 : 0)) {
                        // gate|up -> h (device)
                        if (blk) cs2.K = cs.H;
                        cs2.kind = kSrvStoreGlu;
                        cs2.unit8 = 1;
                    } else if (st == 3) {
                        cs2.K = cs.H;
                        cs2.njobs = 1;
                        cs2.jobs[0] = cs.post;
                        cs2.kind = kSrvStoreY;
                    } else {
                        cs2.K = cs.K2;
                        cs2.njobs = 1;
                        cs2.jobs[0] = cs.down;
                        cs2.kind = blk ? kSrvStoreAddL : kSrvStoreY;
                        cs2.add = rb;
                        // a block's result goes to resid_dev (the next
                        // stage's or command's residual; its readers
                        // finished before this stage's barrier), and to
                        // down.y when given
                        if (blk && !cs.down.y) {
                            cs2.jobs[0].y = cs.resid_dev;
                            cs2.unit8 = 1;
                        }
                        cs2.mirror = blk && cs.down.y ? cs.resid_dev : nullptr;
                    }
                }
                __syncthreads();
            }
            const SrvCmd &c = st > 0 || blk || cs.K2 ? cs2 : cs;
            const bool ok = blk && (st & 1) ? srv_stage_lds(c, lds_dp, xnb, outb, csb, pre)
                                            : srv_stage(c, lds_dp, st == 0 ? dx : cs.h, outb, csb, pre);
            if (!ok) return;
        }
        // every wave's output stores have completed (they write through) before
        // the barrier, and so before thread 0 counts the arrival; no fence:
        // a release fence writes back the whole L2, once per workgroup
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // also: LDS planes are rewritten by the next command
        SRV_STAMP(expect, 10);
        if (threadIdx.x == 0) {
            const int gi = g & 7;
            const uint64_t members = static_cast<uint64_t>((G - gi + 7) / 8);
            const uint64_t n = expect - first + 1;  // commands this launch has completed
            const uint64_t a =
                __hip_atomic_fetch_add(&dev->group[gi][0], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
            if (a == n * members) {
                const uint64_t groups = static_cast<uint64_t>(G < 8 ? G : 8);
                const uint64_t t =
                    __hip_atomic_fetch_add(&dev->top[0], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
                if (t == n * groups) {
                    __hip_atomic_store(done, expect, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    SRV_STAMP(expect, 12);
                }
            }
            SRV_STAMP(expect, 11);
        }
    }
}

// ---- pipelined form ---------------------------------------------------------
// Measured on MI355X, a wavefront that issues every load of its rows before
// it stages the activation row stalls at the loads: the CU accepts vector
// memory requests only as earlier ones drain, so the staging math and the
// first dot products wait until most of the matrix has streamed in, and
// the dot products then run after the stream instead of under it.  Here:
//  * one workgroup of eight wavefronts per CU (the grid never exceeds the CU
//    count, so every workgroup is resident from the start); wavefront v owns
//    the consecutive rows [v*RW, v*RW + RW);
//  * the activation loads go first, then the weight loads of the first two
//    rows, then the staging math (which waits only for the activations);
//    a row's loads are issued two rows ahead of its dot products;
//  * after staging, each lane copies the digit planes of its NBL blocks
//    from LDS into registers once (20 * NBL VGPRs), so the dot products read
//    no LDS;
//  * the per-lane partials of all RW rows are folded across the wavefront in
//    one batched butterfly (wave_rows.h) at the end, a few instructions per
//    row instead of a DPP reduction per row;
//  * rows are full 64-block columns (B = 64 * NBL) of 16-byte aligned rows.
// Per row and lane the arithmetic is the row form's; only the order in which
// the 64 lane partials are added differs.
// RW > 0: RW rows per wavefront, fully unrolled.  RW == 0: the row count is
// the argument rw (loop unrolled by three rows, one DPP reduction per row;
// loads past the wavefront's rows are issued against an empty range and read
// nothing).
constexpr int kPlWaves = 8;

// The body of one workgroup: `blk` is the workgroup's index among those of
// its matrix (W, y, N).
template <int NBL, int RW>
__device__ __forceinline__ void pl_body(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                        float *__restrict__ y, int N, int rw, int blk) {
    // rows are NBL full 64-block columns: B and the row length are constants
    constexpr int B = 64 * NBL;
    constexpr int64_t row_bytes = 18 * B;
    constexpr int D = RW == 0 ? 3 : (RW < 2 ? RW : 2);
    constexpr int ND0 = D < 2 ? D : 2;  // rows requested before the staging math
    __shared__ uint4 planes[kPlanes * B];
    __shared__ float ub[B];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int rows = RW > 0 ? RW : rw;
    const int row0 = (blk * kPlWaves + wave) * rows;
    // rows of this wavefront that exist; loads past them read nothing
    const int lim = min(N, row0 + rows);
    const int nrows = max(0, lim - row0);

    constexpr int XI = (4 * NBL + kPlWaves - 1) / kPlWaves;
    XTile<XI> xt;
    xt.load(x, B, true);  // the activation row is 16-byte aligned
    __builtin_amdgcn_sched_barrier(0);
    // one descriptor over the wavefront's rows; row r at byte offset r * row_bytes
    using Grp = RowGroup<NBL, 1, true, false>;
    const __amdgpu_buffer_rsrc_t rs = Grp::row_rsrc(W, row0, lim, row_bytes);
    constexpr int rb = static_cast<int>(row_bytes);
    Grp g[D];
#pragma unroll
    for (int s = 0; s < ND0; ++s) g[s].load_at(rs, s * rb, B, row_bytes, lane);
    __builtin_amdgcn_sched_barrier(0);
    xt.store(B, reinterpret_cast<uint32_t *>(planes), ub);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = ND0; s < D; ++s) g[s].load_at(rs, s * rb, B, row_bytes, lane);
    __syncthreads();

    uint4 P[NBL][kPlanes];
    float u[NBL];
#pragma unroll
    for (int j = 0; j < NBL; ++j) {
#pragma unroll
        for (int p = 0; p < kPlanes; ++p) P[j][p] = planes[p * B + lane + 64 * j];
        u[j] = ub[lane + 64 * j];
    }

    auto row_dot = [&](const Grp &grp) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
            const int T = block_dot_digits(grp.q[0][j], P[j]);
            const float dr = half_bits_to_float(static_cast<uint16_t>(grp.d_bits(0, j, 0xFFFFu)));
            acc = fmaf(dr * u[j], static_cast<float>(T), acc);
        }
        return acc;
    };

    if constexpr (RW > 0) {
        // partials of all rows, reduced together (a batch of 4 or 8)
        constexpr int RP = RW <= 4 ? 4 : 8;
        float part[RP];
#pragma unroll
        for (int r = RW; r < RP; ++r) part[r] = 0.0f;
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            part[r] = row_dot(g[r % D]);
            __builtin_amdgcn_sched_barrier(0);
            if (r + D < RW) g[r % D].load_at(rs, (r + D) * rb, B, row_bytes, lane);
            __builtin_amdgcn_sched_barrier(0);
        }
        const float tot = st_reduce<RP>(part, lane);
        constexpr int lgS = RP == 4 ? 2 : 3;
        const int r = lane >> (6 - lgS);
        if ((lane & ((64 >> lgS) - 1)) == 0 && r < nrows) y[row0 + r] = tot;
    } else {
        for (int r0 = 0; r0 < nrows; r0 += D) {
#pragma unroll
            for (int s = 0; s < D; ++s) {
                const int r = r0 + s;
                const float acc = row_dot(g[s]);
                __builtin_amdgcn_sched_barrier(0);
                g[s].load_at(rs, (r + D) * rb, B, row_bytes, lane);
                __builtin_amdgcn_sched_barrier(0);
                const float sum = wave_sum(acc);
                if (lane == 0 && r < nrows) y[row0 + r] = sum;
            }
        }
    }
}

template <int NBL, int RW>
__global__ __launch_bounds__(64 * kPlWaves) void gemv_q4_0_pl_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y, int N, int, int64_t, int,
    int rw) {
    pl_body<NBL, RW>(W, x, y, N, rw, static_cast<int>(blockIdx.x));
}

// Several matrices that share the activation row in one launch: job j owns
// workgroups [first[j], first[j + 1]), each running the pipelined body on
// its matrix with the same rows per wavefront.
constexpr int kPlMaxJobs = 8;
struct PlJobs {
    const uint8_t *W[kPlMaxJobs];
    float *y[kPlMaxJobs];
    int N[kPlMaxJobs];
    int first[kPlMaxJobs + 1];
    int n;
};

template <int NBL, int RW>
__global__ __launch_bounds__(64 * kPlWaves) void gemv_q4_0_plj_kernel(PlJobs jobs, const float *__restrict__ x,
                                                                      int rw) {
    const int b = static_cast<int>(blockIdx.x);
    int j = 0;
    while (j + 1 < jobs.n && b >= jobs.first[j + 1]) ++j;
    pl_body<NBL, RW>(jobs.W[j], x, jobs.y[j], jobs.N[j], rw, b - jobs.first[j]);
}

// Pipelined batched variant for NBL x MB <= 8 (rows of full 64-block
// columns): the pipelined form's schedule -- a wavefront owns a run of
// consecutive rows whose loads are issued kPlmDepth rows ahead -- with the
// lane's planes of every activation in registers (20 * NBL * MB VGPRs),
// staged in the workgroup's LDS as the pipelined form stages one.  No
// barrier in the row loop: a row's MB partial sums go through one batched
// cross-lane reduction.
constexpr int kPlmDepth = 3;

template <int NBL, int MB>
__global__ __launch_bounds__(64 * kPlWaves) void gemv_q4_0_plm_kernel(const uint8_t *__restrict__ W,
                                                                      const float *__restrict__ x,
                                                                      int64_t x_stride, int x_al16,
                                                                      float *__restrict__ y, int64_t y_stride,
                                                                      int N, int M, int rows) {
    static_assert(NBL * MB <= 8, "planes of every activation in registers");
    constexpr int B = 64 * NBL;
    constexpr int64_t row_bytes = 18 * B;
    constexpr int rb = static_cast<int>(row_bytes);
    constexpr int D = kPlmDepth;
    constexpr int S = MB <= 4 ? 4 : 8;  // reduction batch (MB padded)
    constexpr int tile = mb_tile(B);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row0 = (blockIdx.x * kPlWaves + wave) * rows;
    const int lim = min(N, row0 + rows);
    const int nrows = max(0, lim - row0);

    // as the pipelined form: every activation's loads, then the weight
    // loads, then the staging math (into one LDS tile per activation)
    constexpr int XI = (4 * NBL + kPlWaves - 1) / kPlWaves;
    XTile<XI> xt[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m)
        if (m < M) xt[m].load(x + m * x_stride, B, x_al16 != 0);
    __builtin_amdgcn_sched_barrier(0);
    using Grp = RowGroup<NBL, 1, true, false>;
    const __amdgpu_buffer_rsrc_t rs = Grp::row_rsrc(W, row0, lim, row_bytes);
    Grp g[D];
#pragma unroll
    for (int s = 0; s < D; ++s) g[s].load_at(rs, s * rb, B, row_bytes, lane);
    __builtin_amdgcn_sched_barrier(0);
    __shared__ uint4 lt[MB * tile];
#pragma unroll
    for (int m = 0; m < MB; ++m)
        if (m < M)
            xt[m].store(B, reinterpret_cast<uint32_t *>(lt + m * tile), reinterpret_cast<float *>(lt + m * tile + kPlanes * B));
    __syncthreads();

    // slots m >= M repeat the last activation (never stored)
    uint4 P[MB][NBL][kPlanes];
    float u[MB][NBL];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const uint4 *t = lt + min(m, M - 1) * tile;
#pragma unroll
        for (int j = 0; j < NBL; ++j) {
#pragma unroll
            for (int p = 0; p < kPlanes; ++p) P[m][j][p] = t[p * B + lane + 64 * j];
            u[m][j] = reinterpret_cast<const float *>(t + kPlanes * B)[lane + 64 * j];
        }
    }

    for (int r0 = 0; r0 < nrows; r0 += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int r = r0 + s;
            float part[S];
#pragma unroll
            for (int m = 0; m < S; ++m) part[m] = 0.0f;
#pragma unroll
            for (int j = 0; j < NBL; ++j) {
                const float dr = half_bits_to_float(static_cast<uint16_t>(g[s].d_bits(0, j, 0xFFFFu)));
#pragma unroll
                for (int m = 0; m < MB; ++m) {
                    const int T = block_dot_digits(g[s].q[0][j], P[m][j]);
                    part[m] = fmaf(dr * u[m][j], static_cast<float>(T), part[m]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            g[s].load_at(rs, (r + D) * rb, B, row_bytes, lane);  // empty range past the run
            __builtin_amdgcn_sched_barrier(0);
            // lane l ends with the total of partial l >> (6 - log2 S)
            const float tot = st_reduce<S>(part, lane);
            constexpr int SPAN = 64 / S;
            const int m = lane / SPAN;
            if ((lane & (SPAN - 1)) == 0 && m < M && r < nrows) y[m * y_stride + row0 + r] = tot;
        }
    }
}

typedef void (*pl_kernel_t)(const uint8_t *, const float *, float *, int, int, int64_t, int, int);

// compiled rows-per-wavefront counts of the unrolled kernel
constexpr int kPlRows[] = {1, 2, 3, 4, 6, 8};

// Rows of 7 or 8 block columns keep 140-160 VGPRs of digit planes; with more
// than four rows per wavefront (or the run-time count) the kernel would
// spill, so those combinations are not compiled (null: other forms).
template <int NBL>
pl_kernel_t pick_pl_rw(int rw) {
    switch (rw) {
    case 1: return gemv_q4_0_pl_kernel<NBL, 1>;
    case 2: return gemv_q4_0_pl_kernel<NBL, 2>;
    case 3: return gemv_q4_0_pl_kernel<NBL, 3>;
    case 4: return gemv_q4_0_pl_kernel<NBL, 4>;
    default: break;
    }
    if constexpr (NBL <= 6) {
        switch (rw) {
        case 6: return gemv_q4_0_pl_kernel<NBL, 6>;
        case 8: return gemv_q4_0_pl_kernel<NBL, 8>;
        default: return gemv_q4_0_pl_kernel<NBL, 0>;
        }
    }
    return nullptr;
}

typedef void (*plj_kernel_t)(PlJobs, const float *, int);

template <int NBL>
plj_kernel_t pick_plj_rw(int rw) {
    switch (rw) {
    case 1: return gemv_q4_0_plj_kernel<NBL, 1>;
    case 2: return gemv_q4_0_plj_kernel<NBL, 2>;
    case 3: return gemv_q4_0_plj_kernel<NBL, 3>;
    case 4: return gemv_q4_0_plj_kernel<NBL, 4>;
    default: break;
    }
    if constexpr (NBL <= 6) {
        switch (rw) {
        case 6: return gemv_q4_0_plj_kernel<NBL, 6>;
        case 8: return gemv_q4_0_plj_kernel<NBL, 8>;
        default: return gemv_q4_0_plj_kernel<NBL, 0>;
        }
    }
    return nullptr;
}

plj_kernel_t pick_plj(int nbl, int rw) {
    switch (nbl) {
    case 1: return pick_plj_rw<1>(rw);
    case 2: return pick_plj_rw<2>(rw);
    case 3: return pick_plj_rw<3>(rw);
    case 4: return pick_plj_rw<4>(rw);
    case 5: return pick_plj_rw<5>(rw);
    case 6: return pick_plj_rw<6>(rw);
    case 7: return pick_plj_rw<7>(rw);
    default: return pick_plj_rw<8>(rw);
    }
}

pl_kernel_t pick_pl(int nbl, int rw) {
    switch (nbl) {
    case 1: return pick_pl_rw<1>(rw);
    case 2: return pick_pl_rw<2>(rw);
    case 3: return pick_pl_rw<3>(rw);
    case 4: return pick_pl_rw<4>(rw);
    case 5: return pick_pl_rw<5>(rw);
    case 6: return pick_pl_rw<6>(rw);
    case 7: return pick_pl_rw<7>(rw);
    default: return pick_pl_rw<8>(rw);
    }
}

typedef void (*ks_kernel_t)(const uint8_t *, const float *, float *, int, int, int64_t, int);

template <int R>
ks_kernel_t pick_ks_r(int nbl) {
    switch (nbl) {
    case 1: return gemv_q4_0_ks_kernel<R, 16, 1>;
    case 2: return gemv_q4_0_ks_kernel<R, 8, 2>;
    case 3: return gemv_q4_0_ks_kernel<R, 5, 3>;
    case 4: return gemv_q4_0_ks_kernel<R, 4, 4>;
    case 5: return gemv_q4_0_ks_kernel<R, 3, 5>;
    case 6: return gemv_q4_0_ks_kernel<R, 2, 6>;
    case 7: return gemv_q4_0_ks_kernel<R, 2, 7>;
    default: return gemv_q4_0_ks_kernel<R, 2, 8>;
    }
}

// row groups (of R rows) per workgroup for a given column count
constexpr int ks_groups(int nbl) { return nbl <= 1 ? 16 : (nbl == 3 ? 5 : (nbl >= 6 ? 2 : 16 / nbl)); }

typedef void (*dp_kernel_t)(const uint8_t *, const float *, float *, int, int, int64_t, int);

// A16 = false (rows not 16-byte aligned: K % 256 != 0) only in its plain form.
template <int NBL, int R, int WAVES>
dp_kernel_t pick_dp_at(bool a16, bool tail, bool pf) {
    if (!a16)
        return tail ? gemv_q4_0_dp_kernel<NBL, R, WAVES, false, true, false>
                    : gemv_q4_0_dp_kernel<NBL, R, WAVES, false, false, false>;
    if (pf)
        return tail ? gemv_q4_0_dp_kernel<NBL, R, WAVES, true, true, true>
                    : gemv_q4_0_dp_kernel<NBL, R, WAVES, true, false, true>;
    return tail ? gemv_q4_0_dp_kernel<NBL, R, WAVES, true, true, false>
                : gemv_q4_0_dp_kernel<NBL, R, WAVES, true, false, false>;
}

template <int NBL, int WAVES>
dp_kernel_t pick_dp_r(int r, bool a16, bool tail, bool pf) {
    switch (r) {
    case 1: return pick_dp_at<NBL, 1, WAVES>(a16, tail, pf);
    case 2: return pick_dp_at<NBL, 2, WAVES>(a16, tail, pf);
    default: return pick_dp_at<NBL, 4, WAVES>(a16, tail, pf);
    }
}

template <int WAVES>
dp_kernel_t pick_dp_n(int nbl, int r, bool a16, bool tail, bool pf) {
    switch (nbl) {
    case 1: return pick_dp_r<1, WAVES>(r, a16, tail, pf);
    case 2: return pick_dp_r<2, WAVES>(r, a16, tail, pf);
    case 3: return pick_dp_r<3, WAVES>(r, a16, tail, pf);
    case 4: return pick_dp_r<4, WAVES>(r, a16, tail, pf);
    case 5: return pick_dp_r<5, WAVES>(r, a16, tail, pf);
    case 6: return pick_dp_r<6, WAVES>(r, a16, tail, pf);
    case 7: return pick_dp_r<7, WAVES>(r, a16, tail, pf);
    default: return pick_dp_r<8, WAVES>(r, a16, tail, pf);
    }
}

// LDS: Q planes (2 * B uint4), d_x (B floats), S (B ints), then a chunk of
// block contributions, `cg` row groups of WAVES * R rows (q8_cs_stride(B)
// floats per row).  Each row is summed by one thread in block order, ggml's
// sequential f32 sum, so the result is bit-identical to ggml's generic path
// for the same activations.
// Job lookup of the single-matrix kernel: group g of W.
struct Q8OneJob {
    const uint8_t *W;
    float *y;
    int N;
    __device__ void at(int g, const uint8_t *&w, float *&yy, int &n, int &gl) const {
        w = W;
        yy = y;
        n = N;
        gl = g;
    }
};
// Job lookup of the multi-matrix kernel: job j owns the row groups
// [first[j], first[j + 1]); groups past the last read nothing.
struct Q8JobTable {
    PlJobs t;
    __device__ void at(int g, const uint8_t *&w, float *&yy, int &n, int &gl) const {
        int j = 0;
        while (j + 1 < t.n && g >= t.first[j + 1]) ++j;
        w = t.W[j];
        yy = t.y[j];
        n = t.N[j];
        gl = g - t.first[j];
    }
};

// Row stride (floats) of the block-contribution chunk: 16-byte rows whose
// dword stride is an odd multiple of 4, so the summing lanes' b128 reads of
// a row each (one row per lane) fall in distinct banks.
__host__ __device__ constexpr int q8_cs_stride(int B) { return 4 * (((B + 3) / 4) % 2 == 0 ? (B + 3) / 4 + 1 : (B + 3) / 4 + 2); }

// A workgroup computes the block contributions of `cg` row groups (its
// groups g, g + G, ...) into one chunk, then sums every row of the chunk at
// once, one row per thread, each in block order (ordered_sum): the sums of
// many rows share each instruction instead of one lane per row.
template <int NBL, int R, bool A16, bool TAIL, class J>
__device__ __forceinline__ void q8_body(const J &jobs, int n_groups, const float *__restrict__ x, int B,
                                        int64_t row_bytes, int x_al16, int cg) {
#pragma clang fp contract(off)
    constexpr int WAVES = 8;
    extern __shared__ uint4 lds_q8[];
    uint4 *Q = lds_q8;
    float *dx = reinterpret_cast<float *>(lds_q8 + 2 * B);
    int *sx = reinterpret_cast<int *>(dx + B);
    // 16-byte aligned start of the chunk
    float *cs_all = reinterpret_cast<float *>(lds_q8 + 2 * B + (2 * B + 3) / 4);
    const int stride = q8_cs_stride(B);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    constexpr int ROWS = WAVES * R;
    int bc[NBL];
#pragma unroll
    for (int j = 0; j < NBL; ++j) bc[j] = min(lane + 64 * j, B - 1);
    const uint32_t tail_mask = lane + 64 * (NBL - 1) < B ? 0xFFFFu : 0u;

    // activation loads, then the first group's weights, then the staging
    // math (loads retire in order)
    constexpr int XI = (4 * NBL + WAVES - 1) / WAVES;
    XTile<XI> xt;
    xt.load(x, B, x_al16 != 0);
    __builtin_amdgcn_sched_barrier(0);
    const int G = static_cast<int>(gridDim.x);
    int g = blockIdx.x;
    const uint8_t *W;
    float *y;
    int N, gl;
    jobs.at(g, W, y, N, gl);
    RowGroup<NBL, R, A16, TAIL> grp;
    grp.load(W, gl * ROWS + wave * R, N, B, row_bytes, lane);
    q8_stage<XI>(xt, B, reinterpret_cast<uint32_t *>(Q), dx, sx);
    __syncthreads();

    while (g < n_groups) {
        const int g0 = g;
        int used = 0;
        for (; used < cg && g < n_groups; ++used) {
            q8_blocks<NBL, R, A16, TAIL>(grp, cs_all + (used * ROWS + wave * R) * stride, stride, Q, dx, sx, B, lane,
                                         bc, tail_mask);
            g += G;
            jobs.at(g, W, y, N, gl);
            grp.load(W, gl * ROWS + wave * R, N, B, row_bytes, lane);
        }
        __syncthreads();
        const int t = static_cast<int>(threadIdx.x);
        if (t < used * ROWS) {
            const uint8_t *Wt;
            float *yt;
            int Nt, glt;
            jobs.at(g0 + (t / ROWS) * G, Wt, yt, Nt, glt);
            const int row = glt * ROWS + t % ROWS;
            if (row < Nt) yt[row] = ordered_sum(cs_all + t * stride, B);
        }
        __syncthreads();  // the chunk is rewritten next
    }
}

template <int NBL, int R, bool A16, bool TAIL>
__global__ __launch_bounds__(512) void gemv_q4_0_q8_kernel(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                           float *__restrict__ y, int N, int B, int64_t row_bytes,
                                                           int x_al16, int cg) {
    constexpr int ROWS = 8 * R;
    q8_body<NBL, R, A16, TAIL>(Q8OneJob{W, y, N}, (N + ROWS - 1) / ROWS, x, B, row_bytes, x_al16, cg);
}

template <int NBL, int R, bool A16, bool TAIL>
__global__ __launch_bounds__(512) void gemv_q4_0_q8j_kernel(PlJobs jobs, const float *__restrict__ x, int B,
                                                            int64_t row_bytes, int x_al16, int cg) {
    q8_body<NBL, R, A16, TAIL>(Q8JobTable{jobs}, jobs.first[jobs.n], x, B, row_bytes, x_al16, cg);
}

typedef void (*q8_kernel_t)(const uint8_t *, const float *, float *, int, int, int64_t, int, int);

template <int NBL, int R>
q8_kernel_t pick_q8_at(bool a16, bool tail) {
    if (a16) return tail ? gemv_q4_0_q8_kernel<NBL, R, true, true> : gemv_q4_0_q8_kernel<NBL, R, true, false>;
    return tail ? gemv_q4_0_q8_kernel<NBL, R, false, true> : gemv_q4_0_q8_kernel<NBL, R, false, false>;
}

typedef void (*q8j_kernel_t)(PlJobs, const float *, int, int64_t, int, int);

template <int NBL, int R>
q8j_kernel_t pick_q8j_at(bool a16, bool tail) {
    if (a16) return tail ? gemv_q4_0_q8j_kernel<NBL, R, true, true> : gemv_q4_0_q8j_kernel<NBL, R, true, false>;
    return tail ? gemv_q4_0_q8j_kernel<NBL, R, false, true> : gemv_q4_0_q8j_kernel<NBL, R, false, false>;
}

q8j_kernel_t pick_q8j(int nbl, int R, bool a16, bool tail) {
    switch (nbl) {
    case 1: return R == 4 ? pick_q8j_at<1, 4>(a16, tail) : R == 2 ? pick_q8j_at<1, 2>(a16, tail) : pick_q8j_at<1, 1>(a16, tail);
    case 2: return R == 2 ? pick_q8j_at<2, 2>(a16, tail) : pick_q8j_at<2, 1>(a16, tail);
    case 3: return pick_q8j_at<3, 1>(a16, tail);
    case 4: return pick_q8j_at<4, 1>(a16, tail);
    case 5: return pick_q8j_at<5, 1>(a16, tail);
    case 6: return pick_q8j_at<6, 1>(a16, tail);
    case 7: return pick_q8j_at<7, 1>(a16, tail);
    default: return pick_q8j_at<8, 1>(a16, tail);
    }
}

// rows per wavefront: R = 4 for one block column, 2 for two, 1 beyond (the
// digit kernel's defaults), or fewer where R would leave CUs without a group
// (q8_rows)
q8_kernel_t pick_q8(int nbl, int R, bool a16, bool tail) {
    switch (nbl) {
    case 1: return R == 4 ? pick_q8_at<1, 4>(a16, tail) : R == 2 ? pick_q8_at<1, 2>(a16, tail) : pick_q8_at<1, 1>(a16, tail);
    case 2: return R == 2 ? pick_q8_at<2, 2>(a16, tail) : pick_q8_at<2, 1>(a16, tail);
    case 3: return pick_q8_at<3, 1>(a16, tail);
    case 4: return pick_q8_at<4, 1>(a16, tail);
    case 5: return pick_q8_at<5, 1>(a16, tail);
    case 6: return pick_q8_at<6, 1>(a16, tail);
    case 7: return pick_q8_at<7, 1>(a16, tail);
    default: return pick_q8_at<8, 1>(a16, tail);
    }
}

}  // namespace

// Largest blocks-per-row the digit-plane kernel takes (8 blocks per lane).
constexpr int64_t kDpMaxBlocks = 64 * 8;

bool q4_0_dp_supports(const mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const size_t lds = static_cast<size_t>(B) * (kPlanes * sizeof(uint4) + sizeof(float));
    return !a.x_bf16 && B > 0 && B <= kDpMaxBlocks && lds <= ctx->max_lds_per_block && a.N <= INT32_MAX &&
           static_cast<int64_t>(a.N) * 18 * B < (int64_t(1) << 40);
}

int launch_gemv_q4_0_dp(mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const int64_t row_bytes = 18 * B;
    const bool a16 = (row_bytes % 16 == 0) && (reinterpret_cast<uintptr_t>(a.W) % 16 == 0);
    const bool x_al16 = reinterpret_cast<uintptr_t>(a.x) % 16 == 0;
    const int nbl = static_cast<int>((B + 63) / 64);
    // Pipelined form: full 64-block columns, 16-byte aligned rows and
    // activation row.  By default wherever each wavefront gets at most 8 rows
    // (one workgroup per CU; sweeps on MI355X: 8192x8192 7.5 vs 8.1 us).
    const bool pl_ok = a16 && x_al16 && B % 64 == 0 && nbl <= 8;
    const int64_t pl_need = (a.N + static_cast<int64_t>(ctx->num_cus) * kPlWaves - 1) /
                            (static_cast<int64_t>(ctx->num_cus) * kPlWaves);
    if (pl_ok && (ctx->form_override == MI355X_FORM_PIPE ||
                  (ctx->form_override == MI355X_FORM_AUTO && pl_need <= kPlRows[5]))) {
        int rw = 0;  // runtime row count unless a compiled count covers pl_need
        for (int c : kPlRows)
            if (c >= pl_need) {
                rw = c;
                break;
            }
        const int rows = rw > 0 ? rw : static_cast<int>(pl_need);
        const pl_kernel_t k = pick_pl(nbl, rw);
        if (k) {  // null: this row length and count are left to the other forms
            const int64_t grid =
                (a.N + static_cast<int64_t>(rows) * kPlWaves - 1) / (static_cast<int64_t>(rows) * kPlWaves);
            hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * kPlWaves), 0, ctx->stream, a.W,
                               static_cast<const float *>(a.x), a.y, static_cast<int>(a.N), static_cast<int>(B),
                               row_bytes, 1, rows);
            MI355X_HIP(hipGetLastError());
            return MI355X_OK;
        }
    }
    // K-split form: 16-byte aligned rows.  By default (sweeps on MI355X) for
    // tall matrices with 1 or 3 block columns (151936x2048: 26.9 vs 27.8 us,
    // 17408x5120: 9.8 vs 10.1 us), with 2 rows per wavefront; the row form
    // stays ahead at 2 and 4 columns (4096x4096, 8192x8192).
    const bool ks = a16 && (ctx->form_override == MI355X_FORM_KSPLIT ||
                            (ctx->form_override == MI355X_FORM_AUTO && (nbl == 1 || nbl == 3) && a.N >= 16384));
    if (ks) {
        const int R = ctx->rows_override == 4 ? 4 : 2;
        const ks_kernel_t k = R == 2 ? pick_ks_r<2>(nbl) : pick_ks_r<4>(nbl);
        const int G = ks_groups(nbl);
        const int waves = G * nbl;
        const size_t lds = static_cast<size_t>(B) * (kPlanes * sizeof(uint4) + sizeof(float)) +
                           static_cast<size_t>(G) * R * nbl * sizeof(float);
        const int occ = occupancy(reinterpret_cast<const void *>(k), 64 * waves, lds);
        const int64_t n_groups = (a.N + static_cast<int64_t>(G) * R - 1) / (static_cast<int64_t>(G) * R);
        int64_t grid = std::min<int64_t>(n_groups, static_cast<int64_t>(ctx->num_cus) * occ);
        if (ctx->grid_override > 0) grid = std::min<int64_t>(n_groups, ctx->grid_override);
        hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * waves), lds, ctx->stream, a.W,
                           static_cast<const float *>(a.x), a.y, static_cast<int>(a.N), static_cast<int>(B),
                           row_bytes, x_al16 ? 1 : 0);
        MI355X_HIP(hipGetLastError());
        return MI355X_OK;
    }
    // defaults from sweeps on MI355X (8192x8192, 17408x5120, 151936x2048,
    // 4096x4096, 2048x11008): 8-wave groups; long rows one row per wave with
    // two workgroups per CU, short rows several rows per wave
    int waves = 8;
    int R = nbl <= 1 ? 4 : (nbl == 2 ? 2 : 1);
    if (ctx->waves_override == 8 || ctx->waves_override == 16) waves = ctx->waves_override;
    if (ctx->rows_override == 1 || ctx->rows_override == 2 || ctx->rows_override == 4) R = ctx->rows_override;
    const size_t lds = static_cast<size_t>(B) * (kPlanes * sizeof(uint4) + sizeof(float));
    const bool tail = B % 64 != 0;
    const bool pf = ctx->prefetch_override == 1;
    dp_kernel_t k = waves == 16 ? pick_dp_n<16>(nbl, R, a16, tail, pf) : pick_dp_n<8>(nbl, R, a16, tail, pf);
    const int occ = occupancy(reinterpret_cast<const void *>(k), 64 * waves, lds);
    const int64_t rows_per_group = static_cast<int64_t>(waves) * R;
    const int64_t n_groups = (a.N + rows_per_group - 1) / rows_per_group;
    int64_t grid = std::min<int64_t>(n_groups, static_cast<int64_t>(ctx->num_cus) * (nbl >= 3 ? std::min(occ, 2) : occ));
    if (ctx->grid_override > 0) grid = std::min<int64_t>(n_groups, ctx->grid_override);
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * waves), lds, ctx->stream, a.W,
                       static_cast<const float *>(a.x), a.y, static_cast<int>(a.N), static_cast<int>(B),
                       row_bytes, x_al16 ? 1 : 0);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

size_t q8_lds_bytes(int64_t B, int cg);
int q8_chunk_groups(int64_t B, int64_t n_groups, int64_t grid);

// Rows per wavefront of the Q8_0 kernels for `rows` rows: the default for
// the row length (4 for one block column, 2 for two, 1 beyond), halved while
// the launch would have fewer row groups (8 R rows each) than CUs -- at the
// decode's 2048-2560-row matrices R = 4 left 176 of 256 CUs idle.
int q8_rows(int nbl, int64_t rows, int num_cus) {
    int R = nbl <= 1 ? 4 : (nbl == 2 ? 2 : 1);
    while (R > 1 && (rows + 8 * R - 1) / (8 * R) < num_cus) R /= 2;
    return R;
}

// ggml-cpu numerics: the Q8_0 kernel's row groups of every matrix in one
// launch (row sums in block order by one lane, so bit-identical to one
// launch per matrix)
static int launch_q8_multi(mi355x_ctx *ctx, int64_t K, const float *x, const MultiJob *jobs, int n, bool *launched) {
    const int64_t B = K / 32;
    const int64_t row_bytes = 18 * B;
    const int nbl = static_cast<int>((B + 63) / 64);
    if (n < 1 || n > kPlMaxJobs || B <= 0 || B > kDpMaxBlocks || q8_lds_bytes(B, 1) > ctx->max_lds_per_block)
        return MI355X_OK;
    int64_t total_rows = 0;
    for (int j = 0; j < n; ++j) total_rows += std::max<int64_t>(jobs[j].N, 0);
    const int R = q8_rows(nbl, total_rows, ctx->num_cus);
    bool a16 = row_bytes % 16 == 0;
    PlJobs pj{};
    pj.n = n;
    int64_t groups = 0;
    for (int j = 0; j < n; ++j) {
        if (jobs[j].N <= 0 || jobs[j].N > INT32_MAX) return MI355X_OK;
        a16 = a16 && reinterpret_cast<uintptr_t>(jobs[j].W) % 16 == 0;
        pj.W[j] = jobs[j].W;
        pj.y[j] = jobs[j].y;
        pj.N[j] = static_cast<int>(jobs[j].N);
        pj.first[j] = static_cast<int>(groups);
        groups += (jobs[j].N + 8 * R - 1) / (8 * R);
    }
    if (groups > INT32_MAX) return MI355X_OK;
    pj.first[n] = static_cast<int>(groups);
    const q8j_kernel_t k = pick_q8j(nbl, R, a16, B % 64 != 0);
    // occupancy with the largest chunk, then the chunk this grid needs
    const int occ = occupancy(reinterpret_cast<const void *>(k), 512, q8_lds_bytes(B, q8_chunk_groups(B, groups, 1)));
    int64_t grid = std::min<int64_t>(groups, static_cast<int64_t>(ctx->num_cus) * (nbl >= 3 ? std::min(occ, 2) : occ));
    if (ctx->grid_override > 0) grid = std::min<int64_t>(groups, ctx->grid_override);
    const int cg = q8_chunk_groups(B, groups, grid);
    const size_t lds = q8_lds_bytes(B, cg);
    if (lds > ctx->max_lds_per_block) return MI355X_OK;
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(std::max<int64_t>(grid, 1))), dim3(512), lds, ctx->stream, pj, x,
                       static_cast<int>(B), row_bytes, reinterpret_cast<uintptr_t>(x) % 16 == 0 ? 1 : 0, cg);
    MI355X_HIP(hipGetLastError());
    *launched = true;
    return MI355X_OK;
}

int launch_gemv_q4_0_multi(mi355x_ctx *ctx, int64_t K, const float *x, const MultiJob *jobs, int n, bool *launched) {
    *launched = false;
    if (ctx->kernel_variant == MI355X_VARIANT_GGML_Q8) return launch_q8_multi(ctx, K, x, jobs, n, launched);
    const int64_t B = K / 32;
    const int64_t row_bytes = 18 * B;
    const int nbl = static_cast<int>((B + 63) / 64);
    // the pipelined form's conditions, for every matrix
    if (n < 1 || n > kPlMaxJobs || ctx->kernel_variant == MI355X_VARIANT_EXACT_F32 ||
        ctx->kernel_variant == MI355X_VARIANT_GGML_Q8 ||
        (ctx->form_override != MI355X_FORM_AUTO && ctx->form_override != MI355X_FORM_PIPE) || B % 64 != 0 ||
        nbl > 8 || row_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
        return MI355X_OK;
    int64_t total = 0;
    for (int j = 0; j < n; ++j) {
        if (reinterpret_cast<uintptr_t>(jobs[j].W) % 16 != 0 || jobs[j].N <= 0 || jobs[j].N > INT32_MAX) return MI355X_OK;
        total += jobs[j].N;
    }
    const int64_t slots = static_cast<int64_t>(ctx->num_cus) * kPlWaves;
    const int64_t need = (total + slots - 1) / slots;
    if (ctx->form_override == MI355X_FORM_AUTO && need > kPlRows[5]) return MI355X_OK;
    int rw = 0;
    for (int c : kPlRows)
        if (c >= need) {
            rw = c;
            break;
        }
    const int rows = rw > 0 ? rw : static_cast<int>(need);
    const plj_kernel_t k = pick_plj(nbl, rw);
    if (!k) return MI355X_OK;
    PlJobs pj{};
    pj.n = n;
    int64_t grid = 0;
    for (int j = 0; j < n; ++j) {
        pj.W[j] = jobs[j].W;
        pj.y[j] = jobs[j].y;
        pj.N[j] = static_cast<int>(jobs[j].N);
        pj.first[j] = static_cast<int>(grid);
        grid += (jobs[j].N + static_cast<int64_t>(rows) * kPlWaves - 1) / (static_cast<int64_t>(rows) * kPlWaves);
    }
    pj.first[n] = static_cast<int>(grid);
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * kPlWaves), 0, ctx->stream, pj, x, rows);
    MI355X_HIP(hipGetLastError());
    *launched = true;
    return MI355X_OK;
}

}  // namespace mi355x

namespace mi355x {

// LDS of the Q8_0 kernels for B blocks per row and cg row groups per chunk.
size_t q8_lds_bytes(int64_t B, int cg) {
    const int nbl = static_cast<int>((B + 63) / 64);
    const int R = nbl <= 1 ? 4 : (nbl == 2 ? 2 : 1);
    const size_t base = sizeof(uint4) * static_cast<size_t>(2 * B + (2 * B + 3) / 4);
    return base + static_cast<size_t>(cg) * 8 * R * q8_cs_stride(static_cast<int>(B)) * sizeof(float);
}

// Row groups per chunk: what one workgroup gets of n_groups (as the grid
// spreads them), at most 512 rows (one per thread) and a chunk that keeps
// the workgroup within 64 KiB of LDS (two per CU).
int q8_chunk_groups(int64_t B, int64_t n_groups, int64_t grid) {
    const int nbl = static_cast<int>((B + 63) / 64);
    const int R = nbl <= 1 ? 4 : (nbl == 2 ? 2 : 1);
    const size_t per = static_cast<size_t>(8 * R) * q8_cs_stride(static_cast<int>(B)) * sizeof(float);
    const size_t base = q8_lds_bytes(B, 0);
    const int64_t by_lds = base + per < (64u << 10) ? static_cast<int64_t>(((64u << 10) - base) / per) : 1;
    const int64_t per_wg = (n_groups + std::max<int64_t>(grid, 1) - 1) / std::max<int64_t>(grid, 1);
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({by_lds, per_wg, 512 / (8 * R)})));
}

bool q4_0_q8_supports(const mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const size_t lds = q8_lds_bytes(B, 1);
    return !a.x_bf16 && B > 0 && B <= kDpMaxBlocks && lds <= ctx->max_lds_per_block && a.N <= INT32_MAX &&
           static_cast<int64_t>(a.N) * 18 * B < (int64_t(1) << 40);
}

int launch_gemv_q4_0_q8(mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const int64_t row_bytes = 18 * B;
    const bool a16 = (row_bytes % 16 == 0) && (reinterpret_cast<uintptr_t>(a.W) % 16 == 0);
    const bool x_al16 = reinterpret_cast<uintptr_t>(a.x) % 16 == 0;
    const int nbl = static_cast<int>((B + 63) / 64);
    const int R = q8_rows(nbl, a.N, ctx->num_cus);
    const q8_kernel_t k = pick_q8(nbl, R, a16, B % 64 != 0);
    const int64_t n_groups = (a.N + 8 * R - 1) / (8 * R);
    // occupancy with the largest chunk, then the chunk this grid needs
    const int occ = occupancy(reinterpret_cast<const void *>(k), 512, q8_lds_bytes(B, q8_chunk_groups(B, n_groups, 1)));
    int64_t grid = std::min<int64_t>(n_groups, static_cast<int64_t>(ctx->num_cus) * (nbl >= 3 ? std::min(occ, 2) : occ));
    if (ctx->grid_override > 0) grid = std::min<int64_t>(n_groups, ctx->grid_override);
    const int cg = q8_chunk_groups(B, n_groups, grid);
    const size_t lds = q8_lds_bytes(B, cg);
    if (lds > ctx->max_lds_per_block) return set_error(MI355X_EUNSUPPORTED, "Q8_0 chunk exceeds LDS");
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(std::max<int64_t>(grid, 1))), dim3(512), lds, ctx->stream, a.W,
                       static_cast<const float *>(a.x), a.y, static_cast<int>(a.N), static_cast<int>(B), row_bytes,
                       x_al16 ? 1 : 0, cg);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

}  // namespace mi355x

namespace mi355x {

typedef void (*mb_kernel_t)(const uint8_t *, const uint4 *, float *, int64_t, int, int, int64_t, int);
typedef void (*plm_kernel_t)(const uint8_t *, const float *, int64_t, int, float *, int64_t, int, int, int);

// the pipelined batched variant: NBL full columns with NBL x MB <= 8
plm_kernel_t pick_plm(int nbl, int mb) {
    switch (nbl * 16 + mb) {
    case 16 + 2: return gemv_q4_0_plm_kernel<1, 2>;
    case 16 + 4: return gemv_q4_0_plm_kernel<1, 4>;
    case 16 + 8: return gemv_q4_0_plm_kernel<1, 8>;
    case 32 + 2: return gemv_q4_0_plm_kernel<2, 2>;
    case 32 + 4: return gemv_q4_0_plm_kernel<2, 4>;
    case 48 + 2: return gemv_q4_0_plm_kernel<3, 2>;
    case 64 + 2: return gemv_q4_0_plm_kernel<4, 2>;
    default: return nullptr;
    }
}

template <int NBL>
mb_kernel_t pick_mb_m(int mb) {
    switch (mb) {
    case 2: return gemv_q4_0_mb_kernel<NBL, 2>;
    case 4: return gemv_q4_0_mb_kernel<NBL, 4>;
    default: return gemv_q4_0_mb_kernel<NBL, 8>;
    }
}

mb_kernel_t pick_mb(int nbl, int mb) {
    switch (nbl) {
    case 1: return pick_mb_m<1>(mb);
    case 2: return pick_mb_m<2>(mb);
    case 3: return pick_mb_m<3>(mb);
    case 4: return pick_mb_m<4>(mb);
    case 5: return pick_mb_m<5>(mb);
    case 6: return pick_mb_m<6>(mb);
    case 7: return pick_mb_m<7>(mb);
    default: return pick_mb_m<8>(mb);
    }
}

// Activations per batched launch (kMbMax), or 0 if the batched form does not
// apply: f32 activations, rows a multiple of 256 values up to the digit
// kernels' limit, 16-byte aligned weights.
int q4_0_mb_capacity(const mi355x_ctx *, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    if (a.x_bf16 || B <= 0 || B > kDpMaxBlocks || B % 8 != 0 || reinterpret_cast<uintptr_t>(a.W) % 16 != 0 ||
        a.N > INT32_MAX || static_cast<int64_t>(a.N) * 18 * B >= (int64_t(1) << 40))
        return 0;
    return kMbMax;
}

// ---- static scratch of the allocation-free batched entry point --------------
// The activation tiles of one K-split batched launch, for callers that cannot
// allocate (graph capture, serving loops): kMbMax activations of the longest
// row the batched form stages (kDpMaxBlocks blocks) -- 336 KiB, held by every
// device the library runs on until the process ends.  In host code `scratch`
// names a host-side stand-in: its device address, per device, comes from
// hipGetSymbolAddress (resolve_scratch) and only that address is used.
constexpr size_t kScratchBytes = static_cast<size_t>(kMbMax) * 16 * mb_tile(static_cast<int>(kDpMaxBlocks));
static_assert(kScratchBytes == MI355X_NOALLOC_SCRATCH_BYTES, "static scratch size as declared in the C-ABI");
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices] = {};
}  // namespace

int resolve_scratch(int device, void **out) {
    *out = nullptr;
    if (device < 0 || device >= kScratchDevices)
        return set_error(MI355X_EUNSUPPORTED, "static scratch: device index beyond the library's table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return MI355X_OK;
}

size_t scratch_bytes() { return kScratchBytes; }

int launch_gemv_q4_0_mb(mi355x_ctx *ctx, const GemvArgs &a, int64_t x_stride, int64_t y_stride, int M,
                        void *fixed_tiles) {
    const int64_t B = a.K / 32;
    const int64_t row_bytes = 18 * B;
    const int nbl = static_cast<int>((B + 63) / 64);
    const int mb = M <= 2 ? 2 : (M <= 4 ? 4 : 8);
    const bool x_al16 = reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && x_stride % 4 == 0;
    // rows of full columns whose planes of every activation fit in registers:
    // the pipelined variant, staging in its own LDS (sweeps on MI355X)
    const plm_kernel_t kp = B % 64 == 0 ? pick_plm(nbl, mb) : nullptr;
    if (kp) {
        const int64_t slots = static_cast<int64_t>(ctx->num_cus) * kPlWaves;
        const int64_t rows = (a.N + slots - 1) / slots;
        const int64_t grid = (a.N + rows * kPlWaves - 1) / (rows * kPlWaves);
        hipLaunchKernelGGL(kp, dim3(static_cast<unsigned>(grid)), dim3(64 * kPlWaves), 0, ctx->stream, a.W,
                           static_cast<const float *>(a.x), x_stride, x_al16 ? 1 : 0, a.y, y_stride,
                           static_cast<int>(a.N), M, static_cast<int>(rows));
        MI355X_HIP(hipGetLastError());
        return MI355X_OK;
    }
    // the tiles stay in place from the staging launch to the batched launch
    // that reads them (calls on one context share the buffer; with
    // fixed_tiles, the device's static scratch, calls on any context of the
    // device share it and overlapping calls race)
    std::unique_lock<std::mutex> lk(ctx->mu, std::defer_lock);
    const size_t need = static_cast<size_t>(M) * 16 * mb_tile(static_cast<int>(B));
    uint4 *tiles = static_cast<uint4 *>(fixed_tiles);
    if (tiles) {
        if (need > kScratchBytes)
            return set_error(MI355X_EINVAL, "batched GEMV needs " + std::to_string(need) +
                                                " bytes of activation tiles, the static scratch holds " +
                                                std::to_string(kScratchBytes));
    } else {
        lk.lock();
        if (ctx->mbtiles_bytes < need) {
            const int rc = free_device(ctx, ctx->mbtiles);
            if (rc) return rc;
            ctx->mbtiles = nullptr;
            ctx->mbtiles_bytes = 0;
            MI355X_HIP(hipMalloc(&ctx->mbtiles, need));
            ctx->mbtiles_bytes = need;
        }
        tiles = static_cast<uint4 *>(ctx->mbtiles);
    }
    const int64_t groups = static_cast<int64_t>(M) * 4 * B;
    hipLaunchKernelGGL(q4_0_mb_stage_kernel, dim3(static_cast<unsigned>((groups + 255) / 256)), dim3(256), 0,
                       ctx->stream, static_cast<const float *>(a.x), x_stride, M, static_cast<int>(B),
                       x_al16 ? 1 : 0, tiles);
    MI355X_HIP(hipGetLastError());
    const mb_kernel_t k = pick_mb(nbl, mb);
    const int waves = mb_groups(nbl) * nbl;
    const int occ = occupancy(reinterpret_cast<const void *>(k), 64 * waves, 0);
    const int64_t rows = static_cast<int64_t>(mb_groups(nbl)) * kMbRows;
    const int64_t n_groups = (a.N + rows - 1) / rows;
    int64_t grid = std::min<int64_t>(n_groups, static_cast<int64_t>(ctx->num_cus) * occ);
    if (ctx->grid_override > 0) grid = std::min<int64_t>(n_groups, ctx->grid_override);
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(64 * waves), 0, ctx->stream, a.W,
                       static_cast<const uint4 *>(tiles), a.y, y_stride, static_cast<int>(a.N), static_cast<int>(B),
                       row_bytes, M);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

}  // namespace mi355x

// ---- persistent server: host side ----------------------------------------------
namespace mi355x {
namespace {

struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        // a host-only context (device < 0) touches no device
        if (dev < 0 || hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (dev >= 0 && prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

struct ServerImpl {
    // held by every call that talks to the resident kernel; a stop from
    // another thread (a free on the same device) waits for the command in
    // flight
    std::mutex mu;
    mi355x_ctx *ctx = nullptr;
    hipStream_t stream = nullptr;
    int64_t max_k = 0;
    int grid = 0;
    size_t lds = 0;
    SrvCmd *cmd_h = nullptr, *cmd_d = nullptr;  // pinned, mapped
    float *hx_h = nullptr, *hx_d = nullptr;
    uint32_t *done_h = nullptr, *done_d = nullptr;
    SrvDev *dev = nullptr;
    float *dx = nullptr;   // device copy of x (written by workgroup 0)
    float *dh = nullptr;   // h of SwiGLU commands (max_k floats)
    float *dr = nullptr;   // pre x of block commands (kSrvLdsXMax floats)
    float *dres = nullptr; // the residual a block command leaves (kSrvLdsXMax floats)
    int64_t dres_h = 0;    // its length, 0 until a block command completed
    uint32_t seq = 0;      // last command number handed out
    bool running = false;
    std::chrono::steady_clock::time_point last{};
};

// The kernel leaves after kSrvIdleSeconds without a command; the host
// relaunches once it has been idle for half that, so a command never meets a
// kernel that is about to leave.
constexpr double kSrvIdleSeconds = 1.0;
constexpr double kSrvWaitSeconds = 5.0;  // host wait for one command

int server_launch(ServerImpl *s) {
    MI355X_HIP(hipMemsetAsync(s->dev, 0, sizeof(SrvDev), s->stream));
    const uint32_t first = s->seq + 1;
    __hip_atomic_store(s->done_h, s->seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    uint64_t idle = static_cast<uint64_t>(kSrvIdleSeconds * kSrvClockHz);
    const SrvCmd *cmd = s->cmd_d;
    const float *hx = s->hx_d;
    SrvDev *dev = s->dev;
    float *dx = s->dx;
    uint32_t *done = s->done_d;
    void *args[] = {&cmd, &hx, &dev, &dx, &done, const_cast<uint32_t *>(&first), &idle};
    MI355X_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(gemv_q4_0_server_kernel), dim3(s->grid),
                                          dim3(64 * kSrvWaves), args, s->lds, s->stream));
    s->running = true;
    s->last = std::chrono::steady_clock::now();
    return MI355X_OK;
}

int server_stop(ServerImpl *s) {
    if (!s->running) return MI355X_OK;
    s->cmd_h->exit = 1;
    s->cmd_h->K = 0;
    __hip_atomic_store(&s->cmd_h->seqk, static_cast<uint64_t>(++s->seq), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    s->running = false;
    MI355X_HIP(hipStreamSynchronize(s->stream));
    s->cmd_h->exit = 0;
    return MI355X_OK;
}

}  // namespace
}  // namespace mi355x

struct mi355x_server {
    mi355x::ServerImpl impl;
};

namespace mi355x {
namespace {
// Every server of the process.  A hipFree waits for every kernel running on
// its device, so a free stops the resident kernels of all servers on that
// device, whichever context created them.  Lock order: registry, then server.
std::mutex g_srv_mu;
std::vector<mi355x_server *> g_servers;
}  // namespace

int stop_servers(mi355x_ctx *ctx) {
    std::lock_guard<std::mutex> lk(g_srv_mu);
    for (mi355x_server *srv : g_servers) {
        ServerImpl &s = srv->impl;
        if (s.ctx->device != ctx->device) continue;
        std::lock_guard<std::mutex> sl(s.mu);
        DeviceScope dg(s.ctx->device);
        const int rc = server_stop(&s);
        if (rc) return rc;
    }
    return MI355X_OK;
}

}  // namespace mi355x

namespace mi355x {
namespace {
// A workgroup keeps its rows of every job of a stage in LDS: a share of
// whole 16-row units (one more, partial, at the start) padded to a multiple
// of its row group (at most 32 rows).
bool server_rows_fit(const ServerImpl &s, const mi355x_server_job *jobs, int njobs) {
    int64_t rows = 0;
    for (int j = 0; j < njobs; ++j) rows += 16 * ((jobs[j].N / 16 + 2 + s.grid - 1) / s.grid + 1) + 31;
    return rows <= kSrvOutMax;
}

// Hands command c (its jobs and stages filled in) with the payload x (nx
// floats, then x2's nx2) to the resident kernel, launching it first when
// needed, and waits for completion.
int server_submit(ServerImpl &s, const float *x, int64_t nx, const float *x2, int64_t nx2, const SrvCmd &c,
                  const char *who) {
    std::lock_guard<std::mutex> sl(s.mu);
    DeviceScope dg(s.ctx->device);
    const auto now = std::chrono::steady_clock::now();
    if (s.running && std::chrono::duration<double>(now - s.last).count() > kSrvIdleSeconds / 2) {
        int rc = server_stop(&s);
        if (rc) return rc;
    }
    if (!s.running) {
        int rc = server_launch(&s);
        if (rc) return rc;
    }
    std::memcpy(s.hx_h, x, static_cast<size_t>(nx) * sizeof(float));
    if (nx2) std::memcpy(s.hx_h + nx, x2, static_cast<size_t>(nx2) * sizeof(float));
    {
        // every field but the command number, which goes last
        SrvCmd r = c;
        r.seqk = s.cmd_h->seqk;
        r.exit = 0;
        *s.cmd_h = r;
    }
    const uint32_t v = ++s.seq;
    const uint64_t n = static_cast<uint64_t>(nx + nx2);  // payload floats for the relay
    __hip_atomic_store(&s.cmd_h->seqk, static_cast<uint64_t>(v) | (n << 32), __ATOMIC_RELEASE,
                       __HIP_MEMORY_SCOPE_SYSTEM);
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0;; ++i) {
        if (static_cast<int32_t>(__hip_atomic_load(s.done_h, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) - v) >= 0)
            break;
        if ((i & 1023) == 1023 &&
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kSrvWaitSeconds) {
            // the kernel leaves by its idle rule; collect it and report
            s.running = false;
            (void)hipStreamSynchronize(s.stream);
            return set_error(MI355X_EHIP, std::string(who) + ": no completion within 5 s");
        }
    }
    s.last = std::chrono::steady_clock::now();
    return MI355X_OK;
}
}  // namespace
}  // namespace mi355x

using mi355x::set_error;
using mi355x::hip_error;
using mi355x::clear_error;

extern "C" {

int mi355x_server_create(mi355x_ctx *ctx, int64_t max_k, mi355x_server **out) {
    clear_error();
    if (!ctx || !out) return set_error(MI355X_EINVAL, "mi355x_server_create: null pointer");
    *out = nullptr;
    if (max_k <= 0 || max_k % 256 != 0 || max_k > 64 * 8 * 32)
        return set_error(MI355X_EINVAL, "mi355x_server_create: max_k must be a multiple of 256 up to 16384");
    if (const int rc = mi355x::device_gate(ctx, "mi355x_server_create")) return rc;
    mi355x::DeviceScope dg(ctx->device);
    int coop = 0;
    MI355X_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, ctx->device));
    if (!coop) return set_error(MI355X_EUNSUPPORTED, "mi355x_server_create: no cooperative launch on this device");
    auto *srv = new (std::nothrow) mi355x_server();
    if (!srv) return set_error(MI355X_ENOMEM, "mi355x_server_create: out of memory");
    mi355x::ServerImpl &s = srv->impl;
    s.ctx = ctx;
    s.max_k = max_k;
    const int64_t B = max_k / 32;
    s.lds = static_cast<size_t>(B) * (mi355x::kPlanes * sizeof(uint4) + sizeof(float));
    hipError_t e = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking);
    void *p = nullptr;
    if (e == hipSuccess) e = hipHostMalloc(&p, sizeof(mi355x::SrvCmd), hipHostMallocMapped);
    if (e == hipSuccess) {
        s.cmd_h = static_cast<mi355x::SrvCmd *>(p);
        std::memset(p, 0, sizeof(mi355x::SrvCmd));
        e = hipHostGetDevicePointer(&p, s.cmd_h, 0);
        s.cmd_d = static_cast<mi355x::SrvCmd *>(p);
    }
    if (e == hipSuccess) e = hipHostMalloc(&p, static_cast<size_t>(max_k) * sizeof(float), hipHostMallocMapped);
    if (e == hipSuccess) {
        s.hx_h = static_cast<float *>(p);
        e = hipHostGetDevicePointer(&p, s.hx_h, 0);
        s.hx_d = static_cast<float *>(p);
    }
    if (e == hipSuccess) e = hipHostMalloc(&p, 64, hipHostMallocMapped);
    if (e == hipSuccess) {
        s.done_h = static_cast<uint32_t *>(p);
        std::memset(p, 0, 64);
        e = hipHostGetDevicePointer(&p, s.done_h, 0);
        s.done_d = static_cast<uint32_t *>(p);
    }
    if (e == hipSuccess) e = hipMalloc(&p, sizeof(mi355x::SrvDev));
    if (e == hipSuccess) s.dev = static_cast<mi355x::SrvDev *>(p);
    if (e == hipSuccess) e = hipMalloc(&p, static_cast<size_t>(max_k) * sizeof(float));
    if (e == hipSuccess) s.dx = static_cast<float *>(p);
    if (e == hipSuccess) e = hipMalloc(&p, static_cast<size_t>(max_k) * sizeof(float));
    if (e == hipSuccess) s.dh = static_cast<float *>(p);
    if (e == hipSuccess) e = hipMalloc(&p, mi355x::kSrvLdsXMax * sizeof(float));
    if (e == hipSuccess) s.dr = static_cast<float *>(p);
    if (e == hipSuccess) e = hipMalloc(&p, mi355x::kSrvLdsXMax * sizeof(float));
    if (e == hipSuccess) s.dres = static_cast<float *>(p);
    int per_cu = 0;
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(mi355x::gemv_q4_0_server_kernel), 64 * mi355x::kSrvWaves, s.lds);
    if (e != hipSuccess || per_cu < 1) {
        mi355x_server_destroy(srv);
        return e != hipSuccess ? hip_error(e, "mi355x_server_create")
                               : set_error(MI355X_EUNSUPPORTED, "mi355x_server_create: kernel does not fit a CU");
    }
    s.grid = ctx->num_cus;
    if (s.grid > mi355x::kSrvBarSlots) {
        mi355x_server_destroy(srv);
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_create: more CUs than the grid barrier has slots");
    }
    {
        std::lock_guard<std::mutex> lk(mi355x::g_srv_mu);
        mi355x::g_servers.push_back(srv);
    }
    *out = srv;
    return MI355X_OK;
}

int mi355x_server_gemv(mi355x_server *srv, const float *x, int64_t K, int njobs, const mi355x_server_job *jobs) {
    clear_error();
    if (!srv || !x || !jobs) return set_error(MI355X_EINVAL, "mi355x_server_gemv: null pointer");
    mi355x::ServerImpl &s = srv->impl;
    if (njobs < 1 || njobs > mi355x::kSrvMaxJobs)
        return set_error(MI355X_EINVAL, "mi355x_server_gemv: 1 to 4 jobs per call");
    if (K <= 0 || K % 256 != 0 || K > s.max_k)
        return set_error(MI355X_EINVAL, "mi355x_server_gemv: K must be a multiple of 256 up to the server's max_k");
    // the context's kernel variant picks the arithmetic of every job
    const int variant = s.ctx->kernel_variant;
    if (variant == MI355X_VARIANT_EXACT_F32)
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_gemv: no exact-f32 form in the server");
    const int32_t mode = variant == MI355X_VARIANT_GGML_Q8 ? mi355x::kSrvGgmlQ8 : mi355x::kSrvDigits;
    for (int j = 0; j < njobs; ++j) {
        if (!jobs[j].W || !jobs[j].y || jobs[j].N <= 0)
            return set_error(MI355X_EINVAL, "mi355x_server_gemv: bad job");

        if (reinterpret_cast<uintptr_t>(jobs[j].W) % 16 != 0)
            return set_error(MI355X_EINVAL, "mi355x_server_gemv: weights must be 16-byte aligned");
    }
    if (!mi355x::server_rows_fit(s, jobs, njobs))
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_gemv: jobs of more rows than the server holds");
    mi355x::SrvCmd c{};
    c.K = static_cast<int32_t>(K);
    c.njobs = njobs;
    c.mode = mode;
    for (int j = 0; j < njobs; ++j) c.jobs[j] = {static_cast<const uint8_t *>(jobs[j].W), jobs[j].y, jobs[j].N};
    if (const int grc = mi355x::device_gate(s.ctx, "mi355x_server_gemv")) return grc;
    return mi355x::server_submit(s, x, K, nullptr, 0, c, "mi355x_server_gemv");
}

int mi355x_server_swiglu(mi355x_server *srv, const float *x, int64_t K, const void *W_gate, const void *W_up,
                         int64_t F, const void *W_down, int64_t N, float *y) {
    clear_error();
    if (!srv || !x || !W_gate || !W_up || !W_down || !y)
        return set_error(MI355X_EINVAL, "mi355x_server_swiglu: null pointer");
    mi355x::ServerImpl &s = srv->impl;
    if (K <= 0 || K % 256 != 0 || K > s.max_k || F <= 0 || F % 256 != 0 || F > s.max_k)
        return set_error(MI355X_EINVAL, "mi355x_server_swiglu: K and F must be multiples of 256 up to max_k");
    if (N <= 0) return set_error(MI355X_EINVAL, "mi355x_server_swiglu: N must be positive");
    for (const void *w : {W_gate, W_up, W_down})
        if (reinterpret_cast<uintptr_t>(w) % 16 != 0)
            return set_error(MI355X_EINVAL, "mi355x_server_swiglu: weights must be 16-byte aligned");
    const int variant = s.ctx->kernel_variant;
    if (variant == MI355X_VARIANT_EXACT_F32)
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_swiglu: no exact-f32 form in the server");
    const mi355x_server_job up_stage[2] = {{W_gate, F, s.dh}, {W_up, F, s.dh}};
    const mi355x_server_job down_stage[1] = {{W_down, N, y}};
    if (!mi355x::server_rows_fit(s, up_stage, 2) || !mi355x::server_rows_fit(s, down_stage, 1))
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_swiglu: jobs of more rows than the server holds");
    mi355x::SrvCmd c{};
    c.K = static_cast<int32_t>(K);
    c.njobs = 2;
    c.mode = variant == MI355X_VARIANT_GGML_Q8 ? mi355x::kSrvGgmlQ8 : mi355x::kSrvDigits;
    c.jobs[0] = {static_cast<const uint8_t *>(W_gate), s.dh, F};
    c.jobs[1] = {static_cast<const uint8_t *>(W_up), s.dh, F};
    c.kind = mi355x::kSrvStoreGlu;
    c.K2 = static_cast<int32_t>(F);
    c.h = s.dh;
    c.down = {static_cast<const uint8_t *>(W_down), y, N};
    if (const int grc = mi355x::device_gate(s.ctx, "mi355x_server_swiglu")) return grc;
    return mi355x::server_submit(s, x, K, nullptr, 0, c, "mi355x_server_swiglu");
}

int mi355x_server_block(mi355x_server *srv, const float *x, int64_t K, const void *W_o, const float *resid,
                        int64_t H, const float *norm_w, float eps, const void *W_gate, const void *W_up, int64_t F,
                        const void *W_down, float *y, const float *next_norm_w, const void *W_next, int64_t N_next,
                        float *y_next) {
    clear_error();
    if (!srv || !x || !W_o || !norm_w || !W_gate || !W_up || !W_down)
        return set_error(MI355X_EINVAL, "mi355x_server_block: null pointer");
    const bool post = W_next != nullptr;
    if (post && (!next_norm_w || !y_next || N_next <= 0 || reinterpret_cast<uintptr_t>(W_next) % 16 != 0 ||
                 reinterpret_cast<uintptr_t>(next_norm_w) % 4 != 0))
        return set_error(MI355X_EINVAL, "mi355x_server_block: bad next stage");
    mi355x::ServerImpl &s = srv->impl;
    if (K <= 0 || K % 256 != 0 || F <= 0 || F % 256 != 0 || F > s.max_k || H <= 0 || H % 256 != 0 ||
        H > mi355x::kSrvLdsXMax || K + (resid ? H : 0) > s.max_k)
        return set_error(MI355X_EINVAL,
                         "mi355x_server_block: K, H and F must be multiples of 256, H <= 4096, F and K + H <= max_k");
    for (const void *w : {W_o, W_gate, W_up, W_down})
        if (reinterpret_cast<uintptr_t>(w) % 16 != 0)
            return set_error(MI355X_EINVAL, "mi355x_server_block: weights must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(norm_w) % 4 != 0)
        return set_error(MI355X_EINVAL, "mi355x_server_block: norm_w must be 4-byte aligned");
    if (!resid && s.dres_h != H)
        return set_error(MI355X_EINVAL, "mi355x_server_block: no residual of H values kept from an earlier block command");
    const int variant = s.ctx->kernel_variant;
    if (variant == MI355X_VARIANT_EXACT_F32)
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_block: no exact-f32 form in the server");
    const mi355x_server_job pre_stage[1] = {{W_o, H, s.dr}};
    const mi355x_server_job up_stage[2] = {{W_gate, F, s.dh}, {W_up, F, s.dh}};
    const mi355x_server_job down_stage[1] = {{W_down, H, y ? y : s.dres}};
    const mi355x_server_job next_stage[1] = {{W_next, N_next, y_next}};
    if (!mi355x::server_rows_fit(s, pre_stage, 1) || !mi355x::server_rows_fit(s, up_stage, 2) ||
        !mi355x::server_rows_fit(s, down_stage, 1) || (post && !mi355x::server_rows_fit(s, next_stage, 1)))
        return set_error(MI355X_EUNSUPPORTED, "mi355x_server_block: jobs of more rows than the server holds");
    mi355x::SrvCmd c{};
    c.K = static_cast<int32_t>(K);
    c.njobs = 2;
    c.mode = variant == MI355X_VARIANT_GGML_Q8 ? mi355x::kSrvGgmlQ8 : mi355x::kSrvDigits;
    c.jobs[0] = {static_cast<const uint8_t *>(W_gate), s.dh, F};
    c.jobs[1] = {static_cast<const uint8_t *>(W_up), s.dh, F};
    c.K2 = static_cast<int32_t>(F);
    c.H = static_cast<int32_t>(H);
    c.h = s.dh;
    c.down = {static_cast<const uint8_t *>(W_down), y, H};
    c.pre = {static_cast<const uint8_t *>(W_o), s.dr, H};
    c.r_dev = s.dr;
    c.norm_w = norm_w;
    c.eps = eps;
    c.resid_on_dev = resid ? 0 : 1;
    c.resid_dev = s.dres;
    if (post) {
        c.post = {static_cast<const uint8_t *>(W_next), y_next, N_next};
        c.post_norm_w = next_norm_w;
    }
    if (const int grc = mi355x::device_gate(s.ctx, "mi355x_server_block")) return grc;
    s.dres_h = 0;  // set again once the command completed
    const int rc = mi355x::server_submit(s, x, K, resid, resid ? H : 0, c, "mi355x_server_block");
    if (rc == MI355X_OK) s.dres_h = H;
    return rc;
}

#ifdef MI355X_SRV_STAMPS
// The phase-stamp table of the stamps build (64 commands x 256 workgroups x
// kSrvStampSlots), for xdna.cpp_amd/server_phases.py; stop the server first.
__attribute__((visibility("default"))) int mi355x_server_stamps(uint64_t *out) {
    const hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(mi355x::g_srv_stamps), sizeof(mi355x::g_srv_stamps));
    return e == hipSuccess ? MI355X_OK : hip_error(e, "mi355x_server_stamps");
}
#endif

int mi355x_server_stop(mi355x_server *srv) {
    clear_error();
    if (!srv) return set_error(MI355X_EINVAL, "mi355x_server_stop: null pointer");
    std::lock_guard<std::mutex> sl(srv->impl.mu);
    mi355x::DeviceScope dg(srv->impl.ctx->device);
    return mi355x::server_stop(&srv->impl);
}

int mi355x_server_running(mi355x_server *srv) {
    clear_error();
    if (!srv) return set_error(MI355X_EINVAL, "mi355x_server_running: null pointer");
    std::lock_guard<std::mutex> sl(srv->impl.mu);
    mi355x::DeviceScope dg(srv->impl.ctx->device);
    // the server's stream holds nothing but the resident kernel
    const hipError_t e = hipStreamQuery(srv->impl.stream);
    if (e == hipErrorNotReady) return 1;
    if (e == hipSuccess) return 0;
    return hip_error(e, "hipStreamQuery");
}

void mi355x_server_destroy(mi355x_server *srv) {
    if (!srv) return;
    mi355x::ServerImpl &s = srv->impl;
    if (s.ctx) {
        {
            std::lock_guard<std::mutex> lk(mi355x::g_srv_mu);
            auto &v = mi355x::g_servers;
            v.erase(std::remove(v.begin(), v.end(), srv), v.end());
        }
        std::lock_guard<std::mutex> sl(s.mu);
        mi355x::DeviceScope dg(s.ctx->device);
        (void)mi355x::server_stop(&s);
        if (s.stream) (void)hipStreamDestroy(s.stream);
        if (s.dev) (void)hipFree(s.dev);
        if (s.dx) (void)hipFree(s.dx);
        if (s.dh) (void)hipFree(s.dh);
        if (s.dr) (void)hipFree(s.dr);
        if (s.dres) (void)hipFree(s.dres);
    }
    if (s.cmd_h) (void)hipHostFree(s.cmd_h);
    if (s.hx_h) (void)hipHostFree(s.hx_h);
    if (s.done_h) (void)hipHostFree(s.done_h);
    delete srv;
}

}  // extern "C"
