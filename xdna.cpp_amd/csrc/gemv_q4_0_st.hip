// Q4_0 decode GEMV, "stream" form, for gfx950.
//
// Same resident row layout as the other Q4_0 kernels ([16-byte code groups
// of blocks 0..B-1][fp16 d plane], codes stored as signed nibbles q - 8) and
// the same fixed-point activation digits as gemv_q4_0_dp.hip, arranged for
// a machine whose time goes to HBM streaming:
//
//  * One workgroup per CU.  A workgroup is T "teams" of NBL wavefronts, one
//    wavefront per 64-block column of the row (NBL = ceil(B / 64)), and a
//    team owns a contiguous range of rows.  Every wavefront requests its
//    first S rows before doing anything else and the next S rows before
//    computing the current ones, so HBM traffic starts with the kernel and
//    never waits on arithmetic.
//  * Lane l of the column-c wavefront owns block b = 64c + l of every row
//    of its team.  It converts its own 32 activations into five digit
//    planes held in registers (no LDS staging, no barrier before the dot),
//    and each row then costs it one 16-byte code load, one 2-byte scale
//    load and 20 v_dot8_i32_i4.
//  * The S per-lane row partials are summed across the wavefront by a
//    batched butterfly (permlane32/permlane16 swaps, then row mirrors and
//    quad exchanges): about 2 instructions per row instead of a full wave
//    reduction per row.  Column partials meet in LDS and are added in
//    column order, so results are deterministic.
//
// Activation digits: per 32-value block b with m = max|x_j| = 2^(ex-1..ex),
// the scale u = 2^e0 with e0 = max(ex - 18, -126) gives |x_j / u| < 2^18,
// Z_j = rint(x_j / u) (exact power-of-two scaling, one rounding), and five
// balanced base-16 digits per Z_j.  |x_j - Z_j u| <= u/2 <= m 2^-18, so per
// row |err| <= sqrt(32) * 2^-18 * ||w_r|| * ||x|| ~= 2.2e-5 ||w_r|| ||x||.
#include "device_common.h"
#include "internal.h"
#include "q4_0_layout.h"
#include "wave_rows.h"

#include <algorithm>

namespace mi355x {
namespace {

constexpr int kStPlanes = 5;
// 1.5 * 2^23 + 0x88888: adding v*s (|v*s| < 2^18) leaves rint(v*s) + 0x88888
// in the low 20 mantissa bits of a float in [2^23, 2^24)
constexpr float kStMagic = 13142152.0f;
// largest bit pattern of such a float; anything above is inf or NaN input
constexpr uint32_t kStFiniteMax = 0x4B7FFFFFu;
constexpr int kStMaxWaves = 16;

// Digit planes of one group of 8 activations: L[e] = value 4k+e and
// H[e] = value 16+4k+e of the block (k = 0..3 picks the dword), already
// scaled.  w[p] gets digit p of the 8 values in the nibble order of Q4_0
// code dword k: nibble 2e <- L[e], nibble 2e+1 <- H[e].
__device__ __forceinline__ void st_group(const float L[4], const float H[4], float s, uint32_t w[kStPlanes],
                                         uint32_t &maxbits) {
    uint32_t Lb[4], Hb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        Lb[e] = __builtin_bit_cast(uint32_t, fmaf(L[e], s, kStMagic));
        Hb[e] = __builtin_bit_cast(uint32_t, fmaf(H[e], s, kStMagic));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) maxbits = max(maxbits, max(Lb[e], Hb[e]));
    // bytes 0/1/2 of M[e]: digits 0/2/4 of L[e] (low nibble) and H[e] (high)
    // bytes 0/1 of N[e]:   digits 1/3
    uint32_t M[4], Nn[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        M[e] = (Lb[e] & 0x0F0F0F0Fu) | ((Hb[e] << 4) & 0xF0F0F0F0u);
        Nn[e] = ((Lb[e] >> 4) & 0x0F0F0F0Fu) | (Hb[e] & 0xF0F0F0F0u);
    }
    const uint32_t m01 = __builtin_amdgcn_perm(M[1], M[0], 0x05010400u);
    const uint32_t m23 = __builtin_amdgcn_perm(M[3], M[2], 0x05010400u);
    const uint32_t c01 = __builtin_amdgcn_perm(M[1], M[0], 0x0C0C0602u);
    const uint32_t c23 = __builtin_amdgcn_perm(M[3], M[2], 0x0C0C0602u);
    const uint32_t n01 = __builtin_amdgcn_perm(Nn[1], Nn[0], 0x05010400u);
    const uint32_t n23 = __builtin_amdgcn_perm(Nn[3], Nn[2], 0x05010400u);
    // every nibble so far is digit + 8; XOR 8 makes it the signed digit
    w[0] = __builtin_amdgcn_perm(m23, m01, 0x05040100u) ^ 0x88888888u;
    w[2] = __builtin_amdgcn_perm(m23, m01, 0x07060302u) ^ 0x88888888u;
    w[4] = __builtin_amdgcn_perm(c23, c01, 0x05040100u) ^ 0x88888888u;
    w[1] = __builtin_amdgcn_perm(n23, n01, 0x05040100u) ^ 0x88888888u;
    w[3] = __builtin_amdgcn_perm(n23, n01, 0x07060302u) ^ 0x88888888u;
}

// Activation staging, shared by the workgroup: "group" i = 4b + k is the 8
// values of block b that meet code dword k (values 4k..4k+3 and
// 16+4k..16+4k+3).  Thread t handles groups t, t + blockDim, ... (XG of
// them): it loads the two float4s of each (the four groups of a block are
// one DPP quad, so a wavefront's loads cover 16 consecutive blocks), and
// after the first rows' weight loads are issued it computes the group's
// five plane dwords with the block's scale and stores them in LDS:
// planes[(p * B + b) * 4 + k], ub[b] = u_b.  Each lane then loads its own
// block's five planes into registers once.
template <int XG>
struct StStage {
    float v[XG][8];

    __device__ __forceinline__ void load(const float *__restrict__ x, int B) {
#pragma unroll
        for (int it = 0; it < XG; ++it) {
            const int i = min(static_cast<int>(threadIdx.x + it * blockDim.x), 4 * B - 1);
            const float *xb = x + 32 * static_cast<int64_t>(i >> 2) + 4 * (i & 3);
            const float4 lo = *reinterpret_cast<const float4 *>(xb);
            const float4 hi = *reinterpret_cast<const float4 *>(xb + 16);
            v[it][0] = lo.x; v[it][1] = lo.y; v[it][2] = lo.z; v[it][3] = lo.w;
            v[it][4] = hi.x; v[it][5] = hi.y; v[it][6] = hi.z; v[it][7] = hi.w;
        }
    }

    // The math runs for every thread (groups past the row repeat the last
    // group, so every quad is complete); only the LDS stores are predicated.
    __device__ __forceinline__ void store(int B, uint32_t *planes, float *ub) const {
#pragma unroll
        for (int it = 0; it < XG; ++it) {
            const int i = threadIdx.x + it * blockDim.x;
            const int ic = min(i, 4 * B - 1);
            const int b = ic >> 2, k = ic & 3;
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[it][e]));
            m = fmaxf(m, dpp_mov<0xB1>(m));  // the block's 4 groups form a quad
            m = fmaxf(m, dpp_mov<0x4E>(m));
            const int ex = __builtin_amdgcn_frexp_expf(m);  // m in [2^(ex-1), 2^ex); 0 for 0, inf, NaN
            const int e0 = max(ex - 18, -126);
            const float sc = __builtin_amdgcn_ldexpf(1.0f, -e0);
            uint32_t maxbits = 0;
            uint32_t w[kStPlanes];
            const float L[4] = {v[it][0], v[it][1], v[it][2], v[it][3]};
            const float H[4] = {v[it][4], v[it][5], v[it][6], v[it][7]};
            st_group(L, H, sc, w, maxbits);
            maxbits = max(maxbits, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                                       0, static_cast<int>(maxbits), 0xB1, 0xF, 0xF, false)));
            maxbits = max(maxbits, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                                       0, static_cast<int>(maxbits), 0x4E, 0xF, 0xF, false)));
            if (i < 4 * B) {
#pragma unroll
                for (int p = 0; p < kStPlanes; ++p) planes[(p * B + b) * 4 + k] = w[p];
                // u is NaN when the block holds an inf or NaN: the block then
                // poisons its rows the way f32 arithmetic would
                if (k == 0)
                    ub[b] = maxbits > kStFiniteMax ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(1.0f, e0);
            }
        }
    }
};

// sum_j (q_j - 8) * Z_j of one block in each of G rows: Horner over the
// planes inside the dot8 accumulators.  The G chains are interleaved
// instruction by instruction, so each v_dot8 has G-1 independent ones
// between it and the result it accumulates.
template <int G>
__device__ __forceinline__ void st_block_dots(const u32x4 *qs, const uint4 P[kStPlanes], int T[G]) {
#pragma unroll
    for (int r = 0; r < G; ++r) T[r] = 0;
#pragma unroll
    for (int p = kStPlanes - 1; p >= 0; --p) {
#pragma unroll
        for (int r = 0; r < G; ++r)
            T[r] = __builtin_amdgcn_sdot8(static_cast<int>(qs[r][0]), static_cast<int>(P[p].x), T[r] * 16, false);
#pragma unroll
        for (int r = 0; r < G; ++r)
            T[r] = __builtin_amdgcn_sdot8(static_cast<int>(qs[r][1]), static_cast<int>(P[p].y), T[r], false);
#pragma unroll
        for (int r = 0; r < G; ++r)
            T[r] = __builtin_amdgcn_sdot8(static_cast<int>(qs[r][2]), static_cast<int>(P[p].z), T[r], false);
#pragma unroll
        for (int r = 0; r < G; ++r)
            T[r] = __builtin_amdgcn_sdot8(static_cast<int>(qs[r][3]), static_cast<int>(P[p].w), T[r], false);
    }
}

// Code and scale bytes of one lane's block in S consecutive rows, through
// one buffer descriptor whose range ends with the last row that exists:
// buffer range checks include the scalar offset, so rows past it read 0
// without touching memory.
template <int S>
struct StStep {
    u32x4 q[S];
    uint32_t d[S];

    __device__ __forceinline__ void load(const uint8_t *__restrict__ W, int64_t row0, int rows, int64_t row_bytes,
                                         int qv, int dv) {
        const uint32_t records = static_cast<uint32_t>(rows * row_bytes);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(rows > 0 ? W + row0 * row_bytes : W), 0, records, kBufferWord3);
#pragma unroll
        for (int r = 0; r < S; ++r) {
            const int roff = r * static_cast<int>(row_bytes);
            d[r] = __builtin_amdgcn_raw_buffer_load_b16(rs, dv, roff, 0);
            q[r] = __builtin_amdgcn_raw_buffer_load_b128(rs, qv, roff, kNonTemporal);
        }
    }
};

// One step: the S rows of `st` against this lane's block, reduced across the
// wavefront, column partials through LDS buffer `buf` ([T][S][NBL]), then
// the team sums in column order and stores its rows.
template <int S>
__device__ __forceinline__ void st_step(const StStep<S> &st, const uint4 P[kStPlanes], float u, bool live, int lane,
                                        float *buf, int t, int c, int teams, int nbl, int64_t row0_of_step,
                                        int rows_per_team, int N, float *__restrict__ y) {
    constexpr int lgS = S == 4 ? 2 : (S == 8 ? 3 : 4);
    constexpr int G = 4;  // rows whose dot chains run interleaved
    float part[S];
#pragma unroll
    for (int g = 0; g < S; g += G) {
        int T[G];
        st_block_dots<G>(st.q + g, P, T);
#pragma unroll
        for (int r = 0; r < G; ++r) {
            const float d = half_bits_to_float(static_cast<uint16_t>(st.d[g + r]));
            part[g + r] = (d * u) * static_cast<float>(T[r]);
        }
    }
    const float tot = st_reduce<S>(part, lane);
    if ((lane & ((64 >> lgS) - 1)) == 0) buf[(t * S + (lane >> (6 - lgS))) * nbl + c] = tot;
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < teams * S) {
        const int tt = threadIdx.x / S;
        const int r = threadIdx.x - tt * S;
        const int64_t team0 = (static_cast<int64_t>(blockIdx.x) * teams + tt) * rows_per_team;
        const int64_t row = team0 + row0_of_step + r;
        const int64_t lim = min<int64_t>(N, team0 + rows_per_team);
        const float *src = buf + (tt * S + r) * nbl;
        float acc = src[0];
        for (int j = 1; j < nbl; ++j) acc += src[j];
        if (row < lim) y[row] = acc;
    }
}

// rows of step s that exist in a team holding team_rows rows
template <int S>
__device__ __forceinline__ int st_rows(int64_t team_rows, int s) {
    return static_cast<int>(max<int64_t>(0, min<int64_t>(S, team_rows - static_cast<int64_t>(s) * S)));
}

// LDS: the digit planes (dynamic: B uint4 per plane, then B block scales)
// and two [T][S][NBL] buffers of column partials, alternating by step.
// 16 rows per step need more than 128 registers: those kernels run at most
// 8 wavefronts per workgroup.
template <int S>
constexpr int st_max_threads() { return S == 16 ? 512 : 64 * kStMaxWaves; }

template <int S, int XG>
__global__ __launch_bounds__(st_max_threads<S>()) void gemv_q4_0_st_kernel(
    const uint8_t *__restrict__ W, const float *__restrict__ x, float *__restrict__ y, int N, int B,
    int64_t row_bytes, int nbl, int rows_per_team, int steps) {
    extern __shared__ uint4 st_planes[];
    float *st_ub = reinterpret_cast<float *>(st_planes + kStPlanes * B);
    __shared__ float red[2 * kStMaxWaves * S];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int teams = (blockDim.x >> 6) / nbl;
    const int t = wave / nbl;
    const int c = wave - t * nbl;
    const int64_t first = (static_cast<int64_t>(blockIdx.x) * teams + t) * rows_per_team;
    const int64_t team_rows = max<int64_t>(0, min<int64_t>(rows_per_team, N - first));

    const int braw = 64 * c + lane;
    const bool live = braw < B;
    const int bb = live ? braw : B - 1;
    const int qv = 16 * bb;
    const int dv = 16 * B + 2 * static_cast<int>(q4_0_d_slot(static_cast<uint64_t>(bb), static_cast<uint64_t>(B)));

    // Issue order: activation loads, the first rows' weights, then the
    // digit math, which waits only for the activations (loads retire in
    // order).  The empty asm statements keep IR passes from sinking the loads
    // towards their uses; the sched barriers do the same for the machine
    // scheduler.
    StStage<XG> xs;
    xs.load(x, B);
    asm volatile("" ::"s"(x), "s"(W) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    StStep<S> A, Bs;
    A.load(W, first, st_rows<S>(team_rows, 0), row_bytes, qv, dv);
    asm volatile("" ::"s"(x), "s"(W) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    xs.store(B, reinterpret_cast<uint32_t *>(st_planes), st_ub);
    __syncthreads();
    uint4 P[kStPlanes];
#pragma unroll
    for (int p = 0; p < kStPlanes; ++p) P[p] = st_planes[p * B + bb];
    // a lane past the row end contributes 0 whatever its (repeated) block holds
    const float u = live ? st_ub[bb] : 0.0f;

    const int stride = teams * S * nbl;
    // Steps alternate between the register sets A and Bs; the loads of step
    // s+1 are issued before step s is computed.  The steady-state loop runs
    // while at least three steps remain, the last one or two steps are
    // peeled, so no path issues a load for a step that does not exist and
    // every path has a fixed number of loads in flight (exact waits).
    int s = 0;
    for (; s + 2 < steps; s += 2) {
        Bs.load(W, first + static_cast<int64_t>(s + 1) * S, st_rows<S>(team_rows, s + 1), row_bytes, qv, dv);
        asm volatile("" ::"s"(x), "s"(W) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        st_step<S>(A, P, u, live, lane, red + (s & 1) * stride, t, c, teams, nbl, static_cast<int64_t>(s) * S,
                   rows_per_team, N, y);
        A.load(W, first + static_cast<int64_t>(s + 2) * S, st_rows<S>(team_rows, s + 2), row_bytes, qv, dv);
        asm volatile("" ::"s"(x), "s"(W) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        st_step<S>(Bs, P, u, live, lane, red + ((s + 1) & 1) * stride, t, c, teams, nbl,
                   static_cast<int64_t>(s + 1) * S, rows_per_team, N, y);
    }
    if (s + 1 < steps) {
        Bs.load(W, first + static_cast<int64_t>(s + 1) * S, st_rows<S>(team_rows, s + 1), row_bytes, qv, dv);
        asm volatile("" ::"s"(x), "s"(W) : "memory");
        __builtin_amdgcn_sched_barrier(0);
        st_step<S>(A, P, u, live, lane, red + (s & 1) * stride, t, c, teams, nbl, static_cast<int64_t>(s) * S,
                   rows_per_team, N, y);
        st_step<S>(Bs, P, u, live, lane, red + ((s + 1) & 1) * stride, t, c, teams, nbl,
                   static_cast<int64_t>(s + 1) * S, rows_per_team, N, y);
    } else {
        st_step<S>(A, P, u, live, lane, red + (s & 1) * stride, t, c, teams, nbl, static_cast<int64_t>(s) * S,
                   rows_per_team, N, y);
    }
}

typedef void (*st_kernel_t)(const uint8_t *, const float *, float *, int, int, int64_t, int, int, int);

template <int S>
st_kernel_t pick_st(int xg) {
    switch (xg) {
    case 1: return gemv_q4_0_st_kernel<S, 1>;
    case 2: return gemv_q4_0_st_kernel<S, 2>;
    default: return gemv_q4_0_st_kernel<S, 4>;
    }
}

size_t st_lds_bytes(int64_t B) { return static_cast<size_t>(B) * (kStPlanes * sizeof(uint4) + sizeof(float)); }

}  // namespace

// K up to 64 blocks per wavefront x 8 wavefronts; the activation row must be
// 16-byte aligned (it is read in float4s).
bool q4_0_st_supports(const mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    return !a.x_bf16 && B > 0 && B <= 64 * 8 && reinterpret_cast<uintptr_t>(a.x) % 16 == 0 &&
           st_lds_bytes(B) + 2 * kStMaxWaves * 16 * sizeof(float) <= ctx->max_lds_per_block && a.N <= INT32_MAX &&
           static_cast<int64_t>(a.N) * 18 * B < (int64_t(1) << 40);
}

int launch_gemv_q4_0_st(mi355x_ctx *ctx, const GemvArgs &a) {
    const int64_t B = a.K / 32;
    const int64_t row_bytes = 18 * B;
    const int nbl = static_cast<int>((B + 63) / 64);
    // wavefronts per workgroup: 16 (four per SIMD, rows per step <= 8) or 8
    const int max_waves = ctx->waves_override == 8 ? 8 : 16;
    const int teams = std::max(1, max_waves / nbl);
    const int threads = 64 * teams * nbl;
    // staging groups per thread, rounded up to a compiled count
    const int64_t need = (4 * B + threads - 1) / threads;
    const int xg = need <= 1 ? 1 : (need <= 2 ? 2 : 4);  // need <= 4: B <= 64 * nbl, threads >= 64 * nbl
    // one workgroup per CU, fewer when there are under 4 rows per team
    int64_t grid = std::min<int64_t>(ctx->num_cus, (a.N + 4 * teams - 1) / (4 * teams));
    // MI355X_OPT_GRID sets the workgroup count (at least one row per team)
    if (ctx->grid_override > 0) grid = std::min<int64_t>(ctx->grid_override, (a.N + teams - 1) / teams);
    grid = std::max<int64_t>(grid, 1);
    const int64_t rpt = (a.N + grid * teams - 1) / (grid * teams);
    // rows per step: the smallest of 4/8/16 that covers rpt in the fewest
    // steps; 16 only with 8 wavefronts (register budget)
    const int smax = threads > 512 ? 8 : 16;
    const int64_t nsteps = (rpt + smax - 1) / smax;
    const int64_t per = (rpt + nsteps - 1) / nsteps;
    int S = per <= 4 ? 4 : (per <= 8 ? 8 : 16);
    if ((ctx->rows_override == 4 || ctx->rows_override == 8 || ctx->rows_override == 16) && ctx->rows_override <= smax)
        S = ctx->rows_override;
    const int steps = static_cast<int>((rpt + S - 1) / S);
    const st_kernel_t k = S == 4 ? pick_st<4>(xg) : (S == 8 ? pick_st<8>(xg) : pick_st<16>(xg));
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(grid)), dim3(threads), st_lds_bytes(B), ctx->stream, a.W,
                       static_cast<const float *>(a.x), a.y, static_cast<int>(a.N), static_cast<int>(B), row_bytes, nbl,
                       static_cast<int>(rpt), steps);
    MI355X_HIP(hipGetLastError());
    return MI355X_OK;
}

}  // namespace mi355x
