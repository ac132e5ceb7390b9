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
// Work split.  A 512-thread workgroup stages the activations of one K chunk
// in LDS once, with their sums over every 8 values, and (IQ types) the
// codebook; each thread converts one 8-value run per pass, so the staging
// work is spread evenly over the workgroup whatever the chunk length.  Each
// wavefront owns R rows at a time; its 64 lanes cover 8 superblocks per
// step, 8 lanes per superblock, one 32-value slice per lane, NIT steps per
// row (NIT = ceil(superblocks / 8), a template parameter).  A lane reads its
// slices' codes and scales from the field planes with buffer loads
// (out-of-range reads return 0) and forms
//     sum_i scale_g * (code_i - offset_g) * x_i
//       = sum_g scale_g * (sum_i code_i * x_i - offset_g * sum_i x_i)
// so the per-value work is one byte convert and one FMA (f32 rows) or a
// share of two v_dot4 on 16-bit activation digits (digit rows); the offsets
// (Q6_K 32, Q3_K 4, IQ4_XS codebook bias 128, Q4_K/Q5_K mins) use the staged
// sums.
//
// Latency.  Every load a row group needs (R rows x NIT steps) is in flight
// before the group's decode starts: the prologue issues the first group's,
// and each step's registers are reloaded with the next group's step right
// after that step is decoded, so the next group's loads travel while the
// rest of the current one decodes.  In the prologue the activation loads are
// issued first, then the first group's weight loads, and only then are the
// activations written to LDS: loads retire in order, so the LDS writes wait
// for the activations alone while the weight stream is already under way.
#include "internal.h"
#include "kq_device.h"

#include <algorithm>
#include <cstdint>
#include <mutex>

namespace mi355x {
namespace {

// ---- kernel ------------------------------------------------------------------
// Buffer views of the R rows of group g; with live == false an empty range
// (loads through it return zeros and read nothing).
template <int TYPE, int R>
__device__ __forceinline__ void make_rows(const KqArgs &a, int64_t g, Row (&rows)[R], bool live = true) {
    constexpr KqLayout L = kq_layout(TYPE);
    const uint32_t records = live ? static_cast<uint32_t>(a.row_bytes) : 0u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = g * R + r < a.N ? g * R + r : a.N - 1;
        const uint8_t *base = a.W + row * a.row_bytes;
        rows[r].rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, records, kBufferWord3);
        const bool flipped = kq_row_flipped(reinterpret_cast<uintptr_t>(base));
        if constexpr (L.grouped) {
            rows[r].P[0] = static_cast<uint32_t>(a.B);
            rows[r].P[1] = flipped ? 1u : 0u;
        } else {
#pragma unroll
            for (int i = 0; i < 5; ++i)
                rows[r].P[i] = i < L.nfields ? static_cast<uint32_t>(kq_plane_start(L, i, a.B, flipped)) : 0u;
        }
    }
}

// Every launch of the row kernels has NIT = ceil(nb / 8) (at most 8), so the
// superblocks of steps before the last lie inside the chunk for every lane:
// only the last step needs the lane's bounds check.
template <int NIT>
__device__ __forceinline__ bool step_in_chunk(int t, int bloc, int nb) {
    return t < NIT - 1 || bloc < nb;
}

// a + b, never fused with the multiply that formed b: the forms that share a
// decode (row, pipelined, K-split) round every step's product alike.
__device__ __forceinline__ float add_unfused(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}

// Loads of row group g: regs[r][t] for step t (superblock it = 8t + lane/8,
// clamped into the chunk; lanes past the chunk's end are masked at use).
template <int TYPE, int R, int NIT>
__device__ __forceinline__ void load_group(const KqArgs &a, int64_t g, int s, int bl,
                                           typename Kq<TYPE>::Regs (&regs)[R][NIT], bool live = true) {
    Row rows[R];
    make_rows<TYPE, R>(a, g, rows, live);
#pragma unroll
    for (int t = 0; t < NIT; ++t) {
        const int bloc = kBlocksPerStep * t + bl;
        const int bc = step_in_chunk<NIT>(t, bloc, a.nb) ? bloc : a.nb - 1;
        const uint32_t babs = static_cast<uint32_t>(a.b0 + bc);
#pragma unroll
        for (int r = 0; r < R; ++r) regs[r][t] = Kq<TYPE>::load(rows[r], babs, s);
    }
}

// runs of a chunk each thread of an NT-thread row kernel stages, at most
constexpr int runs_per_thread(int nt) { return (32 * kChunkBlocks + nt - 1) / nt; }

// One row group: its NIT steps against the staged activations, then the
// wavefront sums and the stores of its R outputs.  With RF the registers of
// step t are refilled, right after its decode, with step t of row group gn
// (an empty range when `next` is false: such loads read nothing), so the
// next group's loads are in flight while the rest of this group decodes.
// With XR (digit rows) the lane's activation slices come from xr, read from
// LDS once per kernel, instead of from LDS at every step.
template <int TYPE, int R, int NIT, bool DG, bool RF, bool XR = false>
__device__ __forceinline__ void kq_row_group(const KqArgs &a, int64_t g, typename Kq<TYPE>::Regs (&regs)[R][NIT],
                                             const uint8_t *lds, const uint32_t *grid, int s, int bl, int lane,
                                             int64_t gn = 0, bool next = false, const XDig *xr = nullptr) {
    using K = Kq<TYPE>;
    constexpr int SH = slice_shape(TYPE);
    Row nrows[RF ? R : 1];
    if constexpr (RF) make_rows<TYPE, R>(a, gn, nrows, next);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
    for (int t = 0; t < NIT; ++t) {
        const int bloc = kBlocksPerStep * t + bl;
        const bool valid = step_in_chunk<NIT>(t, bloc, a.nb);
        const int bc = valid ? bloc : a.nb - 1;
        if constexpr (DG && XR) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float p = KqDg<TYPE>::compute(regs[r][t], s, xr[t], grid);
                acc[r] = add_unfused(acc[r], valid ? p : 0.f);
            }
        } else if constexpr (DG) {
            XDig x;
            dg_slice_lm<SH>(lds + lm_record(kDgGroupBytes, bc, s), x);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float p = KqDg<TYPE>::compute(regs[r][t], s, x, grid);
                acc[r] = add_unfused(acc[r], valid ? p : 0.f);
            }
        } else {
            XSlice x;
            x_slice_lm<SH>(lds + lm_record(kXGroupBytes, bc, s), x);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float p = K::compute(regs[r][t], s, x, grid);
                acc[r] = add_unfused(acc[r], valid ? p : 0.f);
            }
        }
        if constexpr (RF) {
            // after the decode, so the loads reuse its registers
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t babs = static_cast<uint32_t>(a.b0 + bc);
#pragma unroll
            for (int r = 0; r < R; ++r) regs[r][t] = K::load(nrows[r], babs, s);
        }
        // one step's activations live at a time (no hoisting of the
        // next step's LDS reads into this one)
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float tot = wave_sum(acc[r]);
        const int64_t row = g * R + r;
        if (lane == 0 && row < a.N) a.y[row] = a.accumulate ? a.y[row] + tot : tot;
    }
}

// PF: a wavefront's next row group is requested before the current one's
// decode (two register sets, alternating), so its loads travel while the
// current group computes; requests past the last group read nothing.
// NT = kThreads: wavefront w of workgroup b takes row groups b * 8 + w,
// stepping by the grid's wavefront count.  NT = kWideThreads (twelve
// wavefronts, one workgroup per CU): workgroup b takes a contiguous block of
// ceil(groups / grid) row groups, its wavefronts interleaved in it, so every
// SIMD gets the same number of rows within one.
template <int TYPE, int R, int NIT, bool DG, bool PF, int NT>
__global__ __launch_bounds__(NT) void gemv_kq_kernel(KqArgs a) {
    using K = Kq<TYPE>;
    // the codebook in static LDS (its address is known when the lookups are
    // compiled, so no base is added per lookup), the lane-major records (f32
    // or digit) in the dynamic LDS
    extern __shared__ float4 lds_kq[];
    constexpr int kTableWords = DG ? dg_table_words(TYPE) : Kq<TYPE>::kGrid;
    __shared__ uint32_t table_kq[kTableWords > 0 ? kTableWords : 1];
    constexpr int SH = slice_shape(TYPE);
    uint32_t *grid = table_kq;
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds_kq);

    constexpr int kNW = NT / 64;
    constexpr int kRuns = runs_per_thread(NT);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int s = lane / kBlocksPerStep;
    const int bl = lane % kBlocksPerStep;
    const int64_t n_groups = (a.N + R - 1) / R;
    int64_t g, g_end, stride;
    if constexpr (NT == kThreads) {
        stride = static_cast<int64_t>(gridDim.x) * kNW;
        g = static_cast<int64_t>(blockIdx.x) * kNW + wave;
        g_end = n_groups;
    } else {
        const int64_t per_wg = (n_groups + gridDim.x - 1) / gridDim.x;
        const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per_wg;
        stride = kNW;
        g = b0 + wave;
        g_end = b0 + per_wg < n_groups ? b0 + per_wg : n_groups;
    }

    // 1. activation loads for staging: runs r = threadIdx.x + NT k of
    // the chunk (8 values each)
    const int nruns = 32 * a.nb;
    const float *xc = a.x + static_cast<int64_t>(a.b0) * 256;
    float4 xv[kRuns][2];
#pragma unroll
    for (int k = 0; k < kRuns; ++k) {
        if (k == 0 || NT * k < nruns) {
            const int r = static_cast<int>(threadIdx.x) + NT * k;
            const float4 *src = reinterpret_cast<const float4 *>(xc + 8 * (r < nruns ? r : nruns - 1));
            xv[k][0] = src[0];
            xv[k][1] = src[1];
        }
    }
    GridRegs<TYPE, NT> gr;
    gr.fetch(a, threadIdx.x, NT);
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads of the first row group (waves without one read nothing)
    typename K::Regs regs[R][NIT];
    load_group<TYPE, R, NIT>(a, g < g_end ? g : n_groups - 1, s, bl, regs, g < g_end);
    __builtin_amdgcn_sched_barrier(0);

    // 3. the runs' record fields into LDS (nruns is a multiple of 32, so the
    // quads of stage_run_dg are all in or all out); codebook
#pragma unroll
    for (int k = 0; k < kRuns; ++k) {
        const int r = static_cast<int>(threadIdx.x) + NT * k;
        if (NT * k < nruns && r < nruns) {
            if constexpr (DG) stage_run_dg<SH>(lds, xv[k][0], xv[k][1], r >> 5, r & 31);
            else stage_run_f32<SH>(lds, xv[k][0], xv[k][1], r >> 5, r & 31);
        }
    }
    if constexpr (DG) gr.put_dg(grid, threadIdx.x, NT);
    else gr.put(grid, threadIdx.x, NT);
    __syncthreads();

    // 4. row groups
    if constexpr (PF) {
        typename K::Regs nxt[R][NIT];
        if (g < g_end) {
            for (;;) {
                const int64_t g1 = g + stride;
                load_group<TYPE, R, NIT>(a, g1 < g_end ? g1 : n_groups - 1, s, bl, nxt, g1 < g_end);
                kq_row_group<TYPE, R, NIT, DG, false>(a, g, regs, lds, grid, s, bl, lane);
                if (g1 >= g_end) break;
                const int64_t g2 = g1 + stride;
                load_group<TYPE, R, NIT>(a, g2 < g_end ? g2 : n_groups - 1, s, bl, regs, g2 < g_end);
                kq_row_group<TYPE, R, NIT, DG, false>(a, g1, nxt, lds, grid, s, bl, lane);
                if (g2 >= g_end) break;
                g = g2;
            }
        }
    } else {
        // refill per step, except where two rows of four steps are at the
        // register limit already (IQ3_S's digit rows, the f32 rows), and for
        // Q5_K's short rows (0.2-0.3 us slower with the refill at 14336x4096)
        constexpr bool RF = !(TYPE == MI355X_TYPE_Q5_K && NIT <= 2) &&
                            !(R == 2 && NIT >= 4 && (TYPE == MI355X_TYPE_IQ3_S || !DG));
        // one digit row per step: the lane's activation slices stay in
        // registers for all its row groups, up to the step counts whose
        // registers fit without spilling (six steps of the K6 slices' 24
        // words, seven of the others')
        constexpr bool XR = DG && RF && R == 1 && (NIT <= 6 || (NIT == 7 && SH != kK6));
        XDig xr[XR ? NIT : 1];
        if constexpr (XR) {
#pragma unroll
            for (int t = 0; t < NIT; ++t) {
                const int bloc = kBlocksPerStep * t + bl;
                const int bc = step_in_chunk<NIT>(t, bloc, a.nb) ? bloc : a.nb - 1;
                dg_slice_lm<SH>(lds + lm_record(kDgGroupBytes, bc, s), xr[t]);
            }
        }
        for (; g < g_end; g += stride) {
            const int64_t gn = g + stride;
            if constexpr (RF) {
                kq_row_group<TYPE, R, NIT, DG, true, XR>(a, g, regs, lds, grid, s, bl, lane,
                                                         gn < g_end ? gn : n_groups - 1, gn < g_end, xr);
            } else {
                kq_row_group<TYPE, R, NIT, DG, false>(a, g, regs, lds, grid, s, bl, lane);
                if (gn < g_end) load_group<TYPE, R, NIT>(a, gn, s, bl, regs);
            }
        }
    }
}

// ---- pipelined form -----------------------------------------------------------
// The kernel above re-reads each lane's activation slice from LDS for every
// row and stages the activations once per workgroup, with several
// workgroups per CU: measured on MI355X, its time hardly depends on the
// weight bytes (12-16 us from 21 to 48 MB), i.e. LDS and VALU, not HBM, set
// it.  This form applies what the Q4_0 pipelined form does:
//  * one workgroup of four wavefronts per CU (grid <= CU count); wavefront v
//    owns the consecutive rows [v*rows, v*rows + rows) of the launch;
//  * activations as 16-bit digits (the digit path's arithmetic, v_dot4 on
//    two signed-byte planes), staged once per CU; with XREG each lane then
//    copies the digit slices of its NIT steps into registers once, so the
//    row loop reads no LDS (24 VGPRs per step; NIT <= 4);
//  * a row's loads are issued kPlqDepth rows ahead of its decode, the first
//    two rows' before the staging math;
//  * loads of rows past the wavefront's range use an empty buffer range and
//    read nothing.
// Per row the arithmetic is the digit kernel's (R = 1): same slices, same
// step order, same expressions.
constexpr int kPlqWaves = 4;
constexpr int kPlqThreads = 64 * kPlqWaves;
constexpr int kPlqDepth = 3;
constexpr int kPlqStageBlocks = 2;  // records staged per thread
static_assert(kChunkBlocks <= kBlocksPerStep * kPlqWaves * kPlqStageBlocks, "staging covers a chunk");

template <int TYPE, int NIT, bool XREG>
__global__ __launch_bounds__(kPlqThreads) void gemv_kq_pl_kernel(KqArgs a, int rows) {
    using K = Kq<TYPE>;
    using KD = KqDg<TYPE>;
    constexpr int SH = slice_shape(TYPE);
    constexpr int D = kPlqDepth;
    extern __shared__ float4 lds_plq[];
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds_plq);
    uint32_t *grid = reinterpret_cast<uint32_t *>(lds + dg_lds_bytes(a.nb));
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int s = lane / kBlocksPerStep;
    const int bl = lane % kBlocksPerStep;
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kPlqWaves + wave) * rows;
    const int64_t lim = row0 + rows < a.N ? row0 + rows : a.N;
    const int nrows = lim > row0 ? static_cast<int>(lim - row0) : 0;

    // 1. activation loads: the records of groups wave + 4 j (superblocks
    // clamped into the chunk)
    float4 xv[kPlqStageBlocks][8];
#pragma unroll
    for (int j = 0; j < kPlqStageBlocks; ++j) {
        const int bc = kBlocksPerStep * (wave + kPlqWaves * j) + bl;
        load_record<SH>(a.x + static_cast<int64_t>(a.b0) * 256, bc < a.nb ? bc : a.nb - 1, s, xv[j]);
    }
    GridRegs<TYPE, kPlqThreads> gr;
    gr.fetch(a, threadIdx.x, kPlqThreads);
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads of the first two rows
    typename K::Regs regs[D][NIT];
    auto load_row = [&](int slot, int64_t row) {
        const Row rr = make_row_pl<TYPE>(a, row, lim);
#pragma unroll
        for (int t = 0; t < NIT; ++t) {
            const int bloc = kBlocksPerStep * t + bl;
            const int bc = bloc < a.nb ? bloc : a.nb - 1;
            regs[slot][t] = K::load(rr, static_cast<uint32_t>(a.b0 + bc), s);
        }
    };
    load_row(0, row0);
    load_row(1, row0 + 1);
    __builtin_amdgcn_sched_barrier(0);

    // 3. digits into LDS (waits for the activation loads only); codebook
#pragma unroll
    for (int j = 0; j < kPlqStageBlocks; ++j) {
        const int rt = wave + kPlqWaves * j;
        if (kBlocksPerStep * rt < a.nb)
            put_record_dg<SH>(lds + kDgGroupBytes * rt + 16 * lm_chunk(lane), xv[j], kBlocksPerStep * rt + bl < a.nb);
    }
    gr.put_dg(grid, threadIdx.x, kPlqThreads);
    __builtin_amdgcn_sched_barrier(0);
    load_row(2, row0 + 2);
    __syncthreads();

    // 4. this lane's digit slices (registers with XREG)
    bool valid[NIT];
    int bcs[NIT];
#pragma unroll
    for (int t = 0; t < NIT; ++t) {
        const int bloc = kBlocksPerStep * t + bl;
        valid[t] = bloc < a.nb;
        bcs[t] = valid[t] ? bloc : a.nb - 1;
    }
    XDig xr[XREG ? NIT : 1];
    if constexpr (XREG) {
#pragma unroll
        for (int t = 0; t < NIT; ++t) dg_slice_lm<SH>(lds + lm_record(kDgGroupBytes, bcs[t], s), xr[t]);
    }

    // 5. rows, D loads ahead
    for (int r0 = 0; r0 < nrows; r0 += D) {
#pragma unroll
        for (int slot = 0; slot < D; ++slot) {
            const int r = r0 + slot;
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < NIT; ++t) {
                float p;
                if constexpr (XREG) {
                    p = KD::compute(regs[slot][t], s, xr[t], grid);
                } else {
                    XDig x;
                    dg_slice_lm<SH>(lds + lm_record(kDgGroupBytes, bcs[t], s), x);
                    p = KD::compute(regs[slot][t], s, x, grid);
                    // one step's activations live at a time
                    __builtin_amdgcn_sched_barrier(0);
                }
                acc += valid[t] ? p : 0.f;
            }
            __builtin_amdgcn_sched_barrier(0);
            load_row(slot, row0 + r + D);
            __builtin_amdgcn_sched_barrier(0);
            const float tot = wave_sum(acc);
            if (lane == 0 && r < nrows) {
                const int64_t row = row0 + r;
                a.y[row] = a.accumulate ? a.y[row] + tot : tot;
            }
        }
    }
}

typedef void (*kq_pl_fn)(KqArgs, int);

template <int TYPE>
kq_pl_fn pick_pl_type(int nit) {
    switch (nit) {
    case 1: return gemv_kq_pl_kernel<TYPE, 1, true>;
    case 2: return gemv_kq_pl_kernel<TYPE, 2, true>;
    case 3: return gemv_kq_pl_kernel<TYPE, 3, true>;
    case 4: return gemv_kq_pl_kernel<TYPE, 4, true>;
    case 5: return gemv_kq_pl_kernel<TYPE, 5, false>;
    case 6: return gemv_kq_pl_kernel<TYPE, 6, false>;
    case 7: return gemv_kq_pl_kernel<TYPE, 7, false>;
    default: return gemv_kq_pl_kernel<TYPE, 8, false>;
    }
}

kq_pl_fn pick_pl_kernel(int type, int nit) {
    switch (type) {
    case MI355X_TYPE_Q4_K: return pick_pl_type<MI355X_TYPE_Q4_K>(nit);
    case MI355X_TYPE_Q5_K: return pick_pl_type<MI355X_TYPE_Q5_K>(nit);
    case MI355X_TYPE_Q3_K: return pick_pl_type<MI355X_TYPE_Q3_K>(nit);
    case MI355X_TYPE_Q6_K: return pick_pl_type<MI355X_TYPE_Q6_K>(nit);
    case MI355X_TYPE_IQ4_XS: return pick_pl_type<MI355X_TYPE_IQ4_XS>(nit);
    case MI355X_TYPE_IQ3_S: return pick_pl_type<MI355X_TYPE_IQ3_S>(nit);
    case MI355X_TYPE_IQ3_XXS: return pick_pl_type<MI355X_TYPE_IQ3_XXS>(nit);
    case MI355X_TYPE_IQ2_S: return pick_pl_type<MI355X_TYPE_IQ2_S>(nit);
    default: return nullptr;
    }
}

// ---- activation-stationary form ------------------------------------------------
// The forms above give each wavefront whole rows, so every row re-reads its
// activation slices from LDS and, at N = 4096 over 256 CUs, a wavefront has
// a single row: its load latency is exposed and each workgroup stages the
// whole activation chunk for a few rows.  Here the steps of a row are split
// over wavefronts instead:
//  * one workgroup per CU of G groups of S = ceil(nb / 8) wavefronts;
//    wavefront (g, t) owns step t (superblocks 8t..8t+7 of the chunk) and,
//    once the digit planes are staged, copies its lanes' slices of that step
//    into registers for good;
//  * the workgroup's rows (a contiguous range) go in tiles of G * RB; group g
//    takes RB consecutive rows of a tile, each wavefront of the group loads
//    and decodes its step of them and writes its lane partials to LDS;
//    loads run two tiles ahead (two register sets), so the tile barrier
//    never waits for memory;
//  * after the barrier, each row's lane partials are summed in step order
//    and across the wavefront: the digit row kernel's slices, expressions and
//    order, so the two forms agree bit for bit.
// Partials are double-buffered by tile parity: the barrier of tile i+1 sits
// between the reads of tile i and the writes of tile i+2.
constexpr int kXsMaxWaves = 16;
constexpr int kXsThreads = 64 * kXsMaxWaves;
constexpr int kXsMaxRows = 4096;   // rows per workgroup (one LDS float each)
constexpr int kXsMinThreads = 64 * 10;  // S * G >= 10 for every S = 1..8

template <int TYPE, int RB>
__global__ __launch_bounds__(kXsThreads) void gemv_kq_xs_kernel(KqArgs a, int G, int rows_per_wg) {
    using K = Kq<TYPE>;
    using KD = KqDg<TYPE>;
    constexpr int SH = slice_shape(TYPE);
    extern __shared__ float4 lds_xs[];
    const int S = (a.nb + kBlocksPerStep - 1) / kBlocksPerStep;
    const int W = S * G;
    const int nthr = 64 * W;
    const int tile = G * RB;
    uint8_t *lds = reinterpret_cast<uint8_t *>(lds_xs);
    uint32_t *grid = reinterpret_cast<uint32_t *>(lds + dg_lds_bytes(a.nb));
    float *part = reinterpret_cast<float *>(grid + dg_table_words(TYPE));  // 2 x tile x S x 64
    float *ybuf = part + 2 * tile * S * 64;                     // rows_per_wg results

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int g = wave / S, t = wave % S;
    const int s = lane / kBlocksPerStep;
    const int bloc = kBlocksPerStep * t + lane % kBlocksPerStep;
    const bool valid = bloc < a.nb;
    const uint32_t babs = static_cast<uint32_t>(a.b0 + (valid ? bloc : a.nb - 1));
    const int64_t row_begin = static_cast<int64_t>(blockIdx.x) * rows_per_wg;
    const int64_t row_end = row_begin + rows_per_wg < a.N ? row_begin + rows_per_wg : a.N;
    const int n_tiles = row_end > row_begin ? static_cast<int>((row_end - row_begin + tile - 1) / tile) : 0;

    // 1. activation loads: wavefront w < S stages the records of group w
    // (the others load group S - 1 again and store nothing; superblocks
    // clamped into the chunk)
    const int rt = wave < S ? wave : S - 1;
    const int rbc = kBlocksPerStep * rt + lane % kBlocksPerStep;
    float4 xv[8];
    load_record<SH>(a.x + static_cast<int64_t>(a.b0) * 256, rbc < a.nb ? rbc : a.nb - 1, s, xv);
    GridRegs<TYPE, kXsMinThreads> gr;
    gr.fetch(a, threadIdx.x, nthr);
    __builtin_amdgcn_sched_barrier(0);

    // 2. weight loads of the first two tiles (rows past the range read nothing)
    typename K::Regs regs[2][RB];
    auto load_tile = [&](int buf, int ti) {
        const int64_t r0 = row_begin + static_cast<int64_t>(ti) * tile + g * RB;
#pragma unroll
        for (int j = 0; j < RB; ++j) regs[buf][j] = K::load(make_row_pl<TYPE>(a, r0 + j, row_end), babs, s);
    };
    load_tile(0, 0);
    load_tile(1, 1);
    __builtin_amdgcn_sched_barrier(0);

    // 3. digit records into LDS (waits for the activation loads only); codebook
    if (wave < S) put_record_dg<SH>(lds + kDgGroupBytes * rt + 16 * lm_chunk(lane), xv, rbc < a.nb);
    gr.put_dg(grid, threadIdx.x, nthr);
    __syncthreads();

    // 4. this lane's slice of step t, kept in registers
    XDig xr;
    dg_slice_lm<SH>(lds + lm_record(kDgGroupBytes, valid ? bloc : a.nb - 1, s), xr);

    // 5. tiles: decode, next loads, barrier, per-row sums into LDS.  The
    // loop issues the same loads on every pass (the tiles past the range
    // read nothing) and stores nothing to memory, so each wait for a row's
    // loads counts exactly the loads issued after them and never waits for
    // the next tile's.
    const int n_rows = static_cast<int>(row_end - row_begin);
    auto do_tile = [&](int buf, int ti) {
        float *pb = part + buf * (tile * S * 64);
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const float p = KD::compute(regs[buf][j], s, xr, grid);
            pb[((g * RB + j) * S + t) * 64 + lane] = valid ? p : 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);
        load_tile(buf, ti + 2);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        for (int r = wave; r < tile; r += W) {
            const int lr = ti * tile + r;
            if (lr >= n_rows) break;
            float acc = 0.f;
            for (int u = 0; u < S; ++u) acc += pb[(r * S + u) * 64 + lane];
            const float tot = wave_sum(acc);
            if (lane == 0) ybuf[lr] = tot;
        }
    };
    // tiles in pairs, the last pair possibly half empty (its rows read
    // nothing and are not kept): both halves on every pass, so the waits
    // of the first half also count the second half's loads
    for (int ti = 0; ti < n_tiles; ti += 2) {
        do_tile(0, ti);
        do_tile(1, ti + 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n_rows; i += nthr) {
        const int64_t row = row_begin + i;
        a.y[row] = a.accumulate ? a.y[row] + ybuf[i] : ybuf[i];
    }
}

typedef void (*kq_xs_fn)(KqArgs, int, int);

template <int RB>
kq_xs_fn pick_xs_kernel(int type) {
    switch (type) {
    case MI355X_TYPE_Q4_K: return gemv_kq_xs_kernel<MI355X_TYPE_Q4_K, RB>;
    case MI355X_TYPE_Q5_K: return gemv_kq_xs_kernel<MI355X_TYPE_Q5_K, RB>;
    case MI355X_TYPE_Q3_K: return gemv_kq_xs_kernel<MI355X_TYPE_Q3_K, RB>;
    case MI355X_TYPE_Q6_K: return gemv_kq_xs_kernel<MI355X_TYPE_Q6_K, RB>;
    case MI355X_TYPE_IQ4_XS: return gemv_kq_xs_kernel<MI355X_TYPE_IQ4_XS, RB>;
    case MI355X_TYPE_IQ3_S: return gemv_kq_xs_kernel<MI355X_TYPE_IQ3_S, RB>;
    case MI355X_TYPE_IQ3_XXS: return gemv_kq_xs_kernel<MI355X_TYPE_IQ3_XXS, RB>;
    case MI355X_TYPE_IQ2_S: return gemv_kq_xs_kernel<MI355X_TYPE_IQ2_S, RB>;
    default: return nullptr;
    }
}

kq_xs_fn pick_xs(int type, int rb) { return rb == 2 ? pick_xs_kernel<2>(type) : pick_xs_kernel<4>(type); }

// Rows per group and tile: 4 where two register sets of 4 rows' loads fit
// in 128 VGPRs without spilling, else 2 (Q3_K, Q5_K, Q6_K).
int xs_default_rows(int type) {
    return type == MI355X_TYPE_Q3_K || type == MI355X_TYPE_Q5_K || type == MI355X_TYPE_Q6_K ? 2 : 4;
}

typedef void (*kq_kernel_fn)(KqArgs);

constexpr int kWideThreads = 768;
constexpr int kWideMaxNit = 4;

// R = 2 rows per wavefront only for short rows (NIT <= 2), where both rows'
// loads and decode stay within ~128 VGPRs.
constexpr int kMaxNitR2 = 2;
// Types whose loads of one step fit in at most 8 VGPRs take R = 2 up to
// four steps per row.
constexpr bool small_regs(int type) {
    return type == MI355X_TYPE_Q3_K || type == MI355X_TYPE_IQ3_S || type == MI355X_TYPE_IQ3_XXS ||
           type == MI355X_TYPE_IQ2_S || type == MI355X_TYPE_IQ4_XS || type == MI355X_TYPE_Q4_K;
}
constexpr int max_nit_r2(int type) { return small_regs(type) ? 4 : kMaxNitR2; }

// R = 2 only without prefetch (two rows' loads and decode already fill the
// registers); prefetch doubles the weight registers of R = 1.  `wide`: one
// digit row per step in twelve-wavefront workgroups (rows of at most four
// steps, whose registers allow three wavefronts per SIMD); IQ3_S and IQ2_S,
// the types it measured faster for (8192x8192, us: IQ3_S 9.3 against 9.7
// with eight wavefronts; IQ2_S with its 8-byte codebook 8.05-8.24, mean
// 8.13 over eight runs, against 8.22-8.26, mean 8.24; IQ3_XXS 7.99-8.07 against 7.77-7.93, IQ4_XS 9.7 against 8.8),
// and only for launches in order: with two
// overlapped launches in flight IQ3_S took 7.9-8.0 us per launch with it
// against 7.5 with eight wavefronts (one workgroup per CU leaves the next
// launch's workgroups no room until it drains).
template <int TYPE, bool DG, bool PF>
kq_kernel_fn pick_dg(int R, int nit, bool wide) {
    if constexpr (!PF) {
        if (R == 2 && nit <= max_nit_r2(TYPE)) {
            if constexpr (small_regs(TYPE)) {
                if (nit == 3) return gemv_kq_kernel<TYPE, 2, 3, DG, false, kThreads>;
                if (nit == 4) return gemv_kq_kernel<TYPE, 2, 4, DG, false, kThreads>;
            }
            return nit == 1 ? gemv_kq_kernel<TYPE, 2, 1, DG, false, kThreads>
                            : gemv_kq_kernel<TYPE, 2, 2, DG, false, kThreads>;
        }
    }
    if constexpr (DG && !PF && (TYPE == MI355X_TYPE_IQ3_S || TYPE == MI355X_TYPE_IQ2_S)) {
        if (wide && nit <= kWideMaxNit) {
            switch (nit) {
            case 1: return gemv_kq_kernel<TYPE, 1, 1, DG, PF, kWideThreads>;
            case 2: return gemv_kq_kernel<TYPE, 1, 2, DG, PF, kWideThreads>;
            case 3: return gemv_kq_kernel<TYPE, 1, 3, DG, PF, kWideThreads>;
            default: return gemv_kq_kernel<TYPE, 1, 4, DG, PF, kWideThreads>;
            }
        }
    }
    switch (nit) {
    case 1: return gemv_kq_kernel<TYPE, 1, 1, DG, PF, kThreads>;
    case 2: return gemv_kq_kernel<TYPE, 1, 2, DG, PF, kThreads>;
    case 3: return gemv_kq_kernel<TYPE, 1, 3, DG, PF, kThreads>;
    case 4: return gemv_kq_kernel<TYPE, 1, 4, DG, PF, kThreads>;
    case 5: return gemv_kq_kernel<TYPE, 1, 5, DG, PF, kThreads>;
    case 6: return gemv_kq_kernel<TYPE, 1, 6, DG, PF, kThreads>;
    case 7: return gemv_kq_kernel<TYPE, 1, 7, DG, PF, kThreads>;
    default: return gemv_kq_kernel<TYPE, 1, 8, DG, PF, kThreads>;
    }
}

template <int TYPE>
kq_kernel_fn pick(int R, int nit, bool dg, bool pf, bool wide) {
    if (pf) return dg ? pick_dg<TYPE, true, true>(R, nit, wide) : pick_dg<TYPE, false, true>(R, nit, wide);
    return dg ? pick_dg<TYPE, true, false>(R, nit, wide) : pick_dg<TYPE, false, false>(R, nit, wide);
}

kq_kernel_fn pick_kernel(int type, int R, int nit, bool dg, bool pf, bool wide) {
    switch (type) {
    case MI355X_TYPE_Q4_K: return pick<MI355X_TYPE_Q4_K>(R, nit, dg, pf, wide);
    case MI355X_TYPE_Q5_K: return pick<MI355X_TYPE_Q5_K>(R, nit, dg, pf, wide);
    case MI355X_TYPE_Q3_K: return pick<MI355X_TYPE_Q3_K>(R, nit, dg, pf, wide);
    case MI355X_TYPE_Q6_K: return pick<MI355X_TYPE_Q6_K>(R, nit, dg, pf, wide);
    case MI355X_TYPE_IQ4_XS: return pick<MI355X_TYPE_IQ4_XS>(R, nit, dg, pf, wide);
    case MI355X_TYPE_IQ3_S: return pick<MI355X_TYPE_IQ3_S>(R, nit, dg, pf, wide);
    case MI355X_TYPE_IQ3_XXS: return pick<MI355X_TYPE_IQ3_XXS>(R, nit, dg, pf, wide);
    case MI355X_TYPE_IQ2_S: return pick<MI355X_TYPE_IQ2_S>(R, nit, dg, pf, wide);
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

// BF16 activations widened to f32 (exact) ahead of the GEMV.
__global__ void bf16_to_f32_kernel(const uint16_t *__restrict__ in, float *__restrict__ out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = bf16_bits_to_float(in[i]);
}


// ---- ggml-cpu numerics: K/IQ weights x Q8_K activations ----------------------
// MI355X_VARIANT_GGML_Q8 for the eight 256-value types: the reference's live
// path whenever ggml-cpu is loaded is quantize_row_q8_K on the activation row
// and ggml_vec_dot_<type>_q8_K per output row (src/xdna-gemv-engine.cpp:
// 1382-1399, 1430-1453; ggml, llama.cpp 0ec4027a2).  This kernel computes
// the arithmetic of ggml's generic C path bit for bit:
//  * each workgroup quantizes the activation row to Q8_K in LDS (one wave per
//    superblock: the first value of largest |x| gives iscale = -127 / max,
//    q = min(127, round-half-even(iscale * x)), d = 1 / iscale, sums of 16);
//  * a wavefront takes one row at a time, 8 lanes per superblock (one
//    32-value slice each, the slices of the f32 kernel), and forms exact
//    integer partials; for Q3_K..Q6_K a reduce-scatter across the 8 lanes
//    leaves ggml's aux[l] (values p = l mod 8, times their scales) in lane l
//    of the superblock;
//  * the f32 terms of ggml's sums ((d_w * d_x) * aux[l], (dmin_w * d_x) *
//    sum(bsums * mins), ((d_w * d_x) * (ls - 32)) * sumi, (d_w * d_x) *
//    bsum) go to LDS, and after a batch of rows one lane per (row, chain)
//    adds each chain in ggml's order, then the chains meet as ggml's do.
// Rows of up to 64 superblocks (K <= 16384).
constexpr int kQ8kMaxBlocks = 64;
constexpr int kQ8kTermFloats = 1024;  // per wavefront: the terms of a batch of rows
constexpr int kQ8kMaxBatch = 16;      // rows per batch
// LDS bytes per staged superblock's codes: 256 + 16, so the 8 superblocks of
// a step (lanes of one slice) read 8 different bank groups
constexpr int kQ8kStride = 272;

// integer max / min / sum across the wavefront (all lanes active): dpp_i above

__device__ __forceinline__ float max_swap32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    const unsigned a = r[0], b = r[1];
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float max_swap16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                    false, false);
    const unsigned a = r[0], b = r[1];
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// maximum over the wavefront, in every lane: lane ^ 32, lane ^ 16 (permlane
// swaps), then row mirror, half-row mirror and quad swaps
__device__ __forceinline__ float wave_max_f(float v) {
    v = max_swap32(v);
    v = max_swap16(v);
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x140>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x141>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0x4E>(__builtin_bit_cast(int, v))));
    v = fmaxf(v, __builtin_bit_cast(float, dpp_i<0xB1>(__builtin_bit_cast(int, v))));
    return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
    {
        const auto r = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
        const unsigned a = r[0], b = r[1];
        v = min(static_cast<int>(a), static_cast<int>(b));
    }
    {
        const auto r = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
        const unsigned a = r[0], b = r[1];
        v = min(static_cast<int>(a), static_cast<int>(b));
    }
    v = min(v, dpp_i<0x140>(v));
    v = min(v, dpp_i<0x141>(v));
    v = min(v, dpp_i<0x4E>(v));
    v = min(v, dpp_i<0xB1>(v));
    return v;
}

// ggml's nearest_int: round half to even through + 1.5 * 2^23.  The ggml
// numerics here use plain operators in functions compiled with contraction
// off: hipcc contracts by default, and a product feeding this sum would
// otherwise fuse into one FMA (one rounding instead of ggml's two).  HIP's
// __fmul_rn / __fadd_rn do not prevent that: they are plain * and + defined
// where contraction is on.
__device__ __forceinline__ int nearest_int_rn(float f) {
#pragma clang fp contract(off)
    const float v = (f + 12582912.0f);
    return (__builtin_bit_cast(int, v) & 0x007fffff) - 0x00400000;
}

// Superblocks [0, nb) of x into Q8_K in LDS: codes qs[kQ8kStride * sb + p],
// bsums bs[16 * sb + j], scales dq[sb].  Wave w takes superblocks w, w + 8,
// ...; lane l holds values 4l..4l+3.
__device__ __forceinline__ void q8k_stage(const float *__restrict__ x, int nb, int8_t *qs, int16_t *bs, float *dq,
                                          int wave, int lane) {
#pragma clang fp contract(off)
    for (int sb = wave; sb < nb; sb += kWaves) {
        const float4 v4 = reinterpret_cast<const float4 *>(x + 256 * static_cast<int64_t>(sb))[lane];
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[e]));
        const float amax = wave_max_f(m);
        int first = 256;
#pragma unroll
        for (int e = 3; e >= 0; --e)
            if (fabsf(v[e]) == amax) first = 4 * lane + e;
        const int j = wave_min_i(first);
        int q[4] = {0, 0, 0, 0};
        float d = 0.0f;
        if (amax != 0.0f && j < 256) {
            // the value at j: element j % 4 (a uniform index) of lane j / 4
            const float sel = v[j & 3];
            const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sel), j >> 2));
            const float iscale = __fdiv_rn(-127.0f, mx);
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = min(127, nearest_int_rn((iscale * v[e])));
            d = __fdiv_rn(1.0f, iscale);
        }
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) packed |= (static_cast<uint32_t>(q[e]) & 0xFFu) << (8 * e);
        reinterpret_cast<uint32_t *>(qs + kQ8kStride * sb)[lane] = packed;
        int s4 = q[0] + q[1] + q[2] + q[3];
        s4 += dpp_i<0xB1>(s4);
        s4 += dpp_i<0x4E>(s4);
        if ((lane & 3) == 0) bs[16 * sb + (lane >> 2)] = static_cast<int16_t>(s4);
        if (lane == 0) dq[sb] = d;
    }
}

__device__ __forceinline__ int sext8(uint32_t w, int byte) { return static_cast<int>(w << (24 - 8 * byte)) >> 24; }

// (scale, min) integers of sub-blocks 2c and 2c+1 of a Q4_K/Q5_K block from
// its scale words (include/xdna/kquants.h:204-212 per sub-block)
__device__ __forceinline__ void scale_min_pair_k4_i(int c, uint32_t w0, uint32_t w1, uint32_t w2, int &sc0, int &m0,
                                                    int &sc1, int &m1) {
    const uint32_t sh = 16u * static_cast<uint32_t>(c & 1);
    const uint32_t a2 = (w0 >> sh) & 0xFFFFu, b2 = (w1 >> sh) & 0xFFFFu, c2 = (w2 >> sh) & 0xFFFFu;
    const uint32_t sc = c < 2 ? (a2 & 0x3F3Fu) : ((c2 & 0x0F0Fu) | ((a2 >> 2) & 0x3030u));
    const uint32_t mn = c < 2 ? (b2 & 0x3F3Fu) : (((c2 >> 4) & 0x0F0Fu) | ((b2 >> 2) & 0x3030u));
    sc0 = static_cast<int>(sc & 0xFFu);
    sc1 = static_cast<int>(sc >> 8);
    m0 = static_cast<int>(mn & 0xFFu);
    m1 = static_cast<int>(mn >> 8);
}

// sum over sub-blocks j of bsums[j] * min[j / 2] of a Q4_K/Q5_K superblock
__device__ __forceinline__ int k4_min_sum(const u32x4 &hd, const int16_t *bs) {
    int s = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int sc0, m0, sc1, m1;
        scale_min_pair_k4_i(c, hd[1], hd[2], hd[3], sc0, m0, sc1, m1);
        s += (bs[4 * c] + bs[4 * c + 1]) * m0 + (bs[4 * c + 2] + bs[4 * c + 3]) * m1;
    }
    return s;
}

// Lane partials of aux[0..7] for Q4_K / Q5_K slice s = (c, h): code byte i of
// the slice holds value 64c + 16h + i (low nibble, sub-block 2c) and 64c + 32
// + 16h + i (high nibble, 2c + 1); both sit at l = i mod 8.
template <bool Q5>
__device__ __forceinline__ void k45_partial(const u32x4 &q, const u32x4 &qh, const u32x4 &hd, int s,
                                            const int8_t *q8, int (&part)[8]) {
    const int c = s >> 1, h = s & 1;
    int sc0, m0, sc1, m1;
    scale_min_pair_k4_i(c, hd[1], hd[2], hd[3], sc0, m0, sc1, m1);
    const uint32_t *qa = reinterpret_cast<const uint32_t *>(q8 + 64 * c + 16 * h);
    const uint32_t *qb = reinterpret_cast<const uint32_t *>(q8 + 64 * c + 32 + 16 * h);
    int lo[8] = {0, 0, 0, 0, 0, 0, 0, 0}, hi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t A = qa[w], Bv = qb[w];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = 4 * w + e;
            int cl = static_cast<int>((q[w] >> (8 * e)) & 15u);
            int ch = static_cast<int>((q[w] >> (8 * e + 4)) & 15u);
            if constexpr (Q5) {
                cl += static_cast<int>((qh[w] >> (8 * e + 2 * c)) & 1u) << 4;
                ch += static_cast<int>((qh[w] >> (8 * e + 2 * c + 1)) & 1u) << 4;
            }
            lo[i & 7] += cl * sext8(A, e);
            hi[i & 7] += ch * sext8(Bv, e);
        }
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) part[l] = sc0 * lo[l] + sc1 * hi[l];
}

// Lane partials of aux[0..7] for Q6_K / Q3_K slice s = (hh, k): value
// 128hh + 32j + 8k + t (j = 0..3, t = 0..7) sits at l = t, scale group
// 8hh + 2j + k/2.
__device__ __forceinline__ void k6_partial(const Kq<MI355X_TYPE_Q6_K>::Regs &g, int s, const int8_t *q8,
                                           int (&part)[8]) {
    const int hh = s >> 2, k = s & 3;
#pragma unroll
    for (int t = 0; t < 8; ++t) part[t] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int sc = sext8(g.sw4, j);
        const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 128 * hh + 32 * j + 8 * k);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t A = g.qa[w], Bq = g.qb[w], H = g.qh[w], Q = qv[w];
            uint32_t code;
            if (j == 0) code = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
            else if (j == 1) code = (Bq & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
            else if (j == 2) code = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
            else code = ((Bq >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                part[4 * w + e] += sc * ((static_cast<int>((code >> (8 * e)) & 0xFFu) - 32) * sext8(Q, e));
        }
    }
}

__device__ __forceinline__ void k3_partial(const Kq<MI355X_TYPE_Q3_K>::Regs &g, int s, const int8_t *q8,
                                           int (&part)[8]) {
    const int hh = s >> 2, k = s & 3, kk = k >> 1;
    const u32x2 hm = Kq<MI355X_TYPE_Q3_K>::hmask(g);
#pragma unroll
    for (int t = 0; t < 8; ++t) part[t] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int lo_byte = 2 * j + kk;
        const int lo = static_cast<int>((Kq<MI355X_TYPE_Q3_K>::lo_scale_byte(g, kk, j) >> (4 * hh)) & 15u);
        const int hi = static_cast<int>((byte_u(g.sw2, lo_byte & 3) >> (2 * (2 * hh + (j >> 1)))) & 3u);
        const int sc = (lo | (hi << 4)) - 32;
        const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 128 * hh + 32 * j + 8 * k);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t code =
                ((g.q[w] >> (2 * j)) & 0x03030303u) | (((hm[w] >> (4 * hh + j)) & 0x01010101u) << 2);
            const uint32_t Q = qv[w];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                part[4 * w + e] += sc * ((static_cast<int>((code >> (8 * e)) & 0xFFu) - 4) * sext8(Q, e));
        }
    }
}

// Integer sums of one 32-value slice of the IQ types: IQ4_XS the codebook dot
// (its scale enters in f32), the grid types sumi times their integer scales.
__device__ __forceinline__ int iq4xs_sumi(const Kq<MI355X_TYPE_IQ4_XS>::Regs &g, int s, const int8_t *q8) {
    const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 32 * s);
    int sumi = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        sumi = sdot4(KqDg<MI355X_TYPE_IQ4_XS>::lookup(g.q[w] & 0x0F0F0F0Fu), qv[w], sumi);
        sumi = sdot4(KqDg<MI355X_TYPE_IQ4_XS>::lookup((g.q[w] >> 4) & 0x0F0F0F0Fu), qv[4 + w], sumi);
    }
    return sumi;
}

__device__ __forceinline__ int iq3s_bsum(const Kq<MI355X_TYPE_IQ3_S>::Regs &g, int s, const int8_t *q8,
                                         const uint32_t *grid) {
    const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 32 * s);
    int sumi = 0;
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        const uint32_t i0 = byte_u(g.qs[k >> 2], k & 3) | (((g.qh >> k) & 1u) << 8);
        const uint32_t i1 = byte_u(g.qs[k >> 2], (k & 3) + 1) | (((g.qh >> (k + 1)) & 1u) << 8);
        uint32_t v0, v1;
        signed8(grid[i0], grid[i1], byte_u(g.sg, k >> 1), v0, v1);
        sumi = sdot4(v0, qv[k], sumi);
        sumi = sdot4(v1, qv[k + 1], sumi);
    }
    return sumi * (1 + 2 * static_cast<int>((g.scb >> (4 * (s & 1))) & 15u));
}

__device__ __forceinline__ int iq3xxs_bsum(const Kq<MI355X_TYPE_IQ3_XXS>::Regs &g, int s, const int8_t *q8,
                                           const uint32_t *grid) {
    const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 32 * s);
    int sumi = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        uint32_t v0, v1;
        signed8(grid[byte_u(g.qs[l >> 1], 2 * (l & 1))], grid[byte_u(g.qs[l >> 1], 2 * (l & 1) + 1)],
                ksigns((g.aux >> (7 * l)) & 127u), v0, v1);
        sumi = sdot4(v0, qv[2 * l], sumi);
        sumi = sdot4(v1, qv[2 * l + 1], sumi);
    }
    return sumi * (1 + 2 * static_cast<int>(g.aux >> 28));
}

__device__ __forceinline__ int iq2s_bsum(const Kq<MI355X_TYPE_IQ2_S>::Regs &g, int s, const int8_t *q8,
                                         const uint32_t *grid) {
    const uint32_t *qv = reinterpret_cast<const uint32_t *>(q8 + 32 * s);
    int s1 = 0, s2 = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        const uint32_t idx = byte_u(g.qs, l) | (((g.qh >> (2 * l)) & 3u) << 8);
        uint32_t v0, v1;
        signed8(grid[2 * idx], grid[2 * idx + 1], byte_u(g.sg, l), v0, v1);
        int t = sdot4(v0, qv[2 * l], 0);
        t = sdot4(v1, qv[2 * l + 1], t);
        if (l < 2) s1 += t;
        else s2 += t;
    }
    return (1 + 2 * static_cast<int>(g.scb & 15u)) * s1 + (1 + 2 * static_cast<int>(g.scb >> 4)) * s2;
}

// Reduce-scatter of 8 per-lane partials across the 8 slice lanes of a
// superblock (lanes bl + 8 s): lane (s, bl) ends with the total of partial s.
// Partners: lane ^ 32 (permlane32 swap), lane ^ 16 (permlane16 swap),
// lane ^ 8 (DPP row rotate by 8).
__device__ __forceinline__ int fold32_i(int a, int b) {
    const auto r = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(a), static_cast<unsigned>(b), false, false);
    const unsigned lo = r[0], hi = r[1];
    return static_cast<int>(lo) + static_cast<int>(hi);
}
__device__ __forceinline__ int fold16_i(int a, int b) {
    const auto r = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(a), static_cast<unsigned>(b), false, false);
    const unsigned lo = r[0], hi = r[1];
    return static_cast<int>(lo) + static_cast<int>(hi);
}
__device__ __forceinline__ int scatter8(const int (&p)[8], int lane) {
    int v4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v4[i] = fold32_i(p[i], p[i + 4]);   // lanes s < 4: l 0..3; s >= 4: 4..7
    int v2[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) v2[i] = fold16_i(v4[i], v4[i + 2]); // then by s & 2
    const bool odd = (lane & 8) != 0;                                // s & 1
    const int own = odd ? v2[1] : v2[0];
    const int other = odd ? v2[0] : v2[1];
    return own + dpp_i<0x128>(other);  // row_ror:8 = lane ^ 8 within a 16-lane row
}
// full integer sum over the 8 slice lanes
__device__ __forceinline__ int sum8(int v) {
    v = fold32_i(v, v);
    v = fold16_i(v, v);
    return v + dpp_i<0x128>(v);
}

template <int TYPE, int NIT>
__global__ __launch_bounds__(kThreads) void gemv_kq_q8k_kernel(KqArgs a, int rb) {
#pragma clang fp contract(off)
    using K = Kq<TYPE>;
    constexpr bool EIGHT = TYPE == MI355X_TYPE_Q3_K || TYPE == MI355X_TYPE_Q4_K || TYPE == MI355X_TYPE_Q5_K ||
                           TYPE == MI355X_TYPE_Q6_K;
    constexpr bool MINS = TYPE == MI355X_TYPE_Q4_K || TYPE == MI355X_TYPE_Q5_K;
    constexpr bool IQ4 = TYPE == MI355X_TYPE_IQ4_XS;
    extern __shared__ float4 lds_q8k[];
    const int S = a.nb;  // superblocks per row (the whole row: b0 == 0)
    int8_t *qs = reinterpret_cast<int8_t *>(lds_q8k);
    int16_t *bs = reinterpret_cast<int16_t *>(qs + kQ8kStride * S);
    float *dq = reinterpret_cast<float *>(bs + 16 * S);
    float *terms = dq + S;  // kWaves x kQ8kTermFloats
    uint32_t *grid = reinterpret_cast<uint32_t *>(terms + kWaves * kQ8kTermFloats);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int s = lane / kBlocksPerStep;
    const int bl = lane % kBlocksPerStep;
    float *tw = terms + wave * kQ8kTermFloats;
    // terms per row: chains of S (8 lanes [+ mins]) or 8S (IQ4_XS) or S
    const int per_row = EIGHT ? (MINS ? 9 : 8) * S : (IQ4 ? 8 * S : S);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWaves;
    int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;

    // first row's weights in flight while the activations are quantized
    typename K::Regs regs[1][NIT];
    GridRegs<TYPE, kThreads> gr;
    gr.fetch(a, threadIdx.x, kThreads);
    load_group<TYPE, 1, NIT>(a, row < a.N ? row : a.N - 1, s, bl, regs);
    __builtin_amdgcn_sched_barrier(0);
    q8k_stage(a.x, S, qs, bs, dq, wave, lane);
    gr.put(grid, threadIdx.x, kThreads);
    __syncthreads();

    while (row < a.N) {
        // a batch of up to rb rows of this wavefront; their terms in tw
        const int64_t first = row;  // batch rows first + r * stride
        int nrow = 0;
        for (; nrow < rb && row < a.N; ++nrow, row += stride) {
            float *tr = tw + nrow * per_row;
#pragma unroll
            for (int t = 0; t < NIT; ++t) {
                const int i = kBlocksPerStep * t + bl;  // superblock
                const bool valid = i < S;
                const int ic = valid ? i : S - 1;
                const int8_t *q8 = qs + kQ8kStride * ic;
                const float dx = dq[ic];
                const auto &g = regs[0][t];
                if constexpr (EIGHT) {
                    int part[8];
                    float dw;
                    if constexpr (TYPE == MI355X_TYPE_Q4_K || TYPE == MI355X_TYPE_Q5_K) {
                        u32x4 qh{0u, 0u, 0u, 0u};
                        if constexpr (TYPE == MI355X_TYPE_Q5_K) qh = g.qh;
                        k45_partial<TYPE == MI355X_TYPE_Q5_K>(g.q, qh, g.hd, s, q8, part);
                        dw = half_f(g.hd[0] & 0xFFFF);
                    } else if constexpr (TYPE == MI355X_TYPE_Q6_K) {
                        k6_partial(g, s, q8, part);
                        dw = half_f(g.d);
                    } else {
                        k3_partial(g, s, q8, part);
                        dw = half_f(g.d);
                    }
                    const int aux = scatter8(part, lane);  // aux[s] of superblock i
                    if (valid) tr[s * S + i] = ((dw * dx) * static_cast<float>(aux));
                    if constexpr (MINS) {
                        if (valid && s == 0) {
                            const int msum = k4_min_sum(g.hd, bs + 16 * ic);
                            const float dmin = (half_f(g.hd[0] >> 16) * dx);
                            tr[8 * S + i] = (dmin * static_cast<float>(msum));
                        }
                    }
                } else if constexpr (IQ4) {
                    const int sumi = iq4xs_sumi(g, s, q8);
                    const uint32_t sh = g.hd[0] >> 16;
                    const int ls = static_cast<int>(((g.hd[1] >> (4 * s)) & 15u) | (((sh >> (2 * s)) & 3u) << 4));
                    const float d4d8 = (half_f(g.hd[0] & 0xFFFF) * dx);
                    const float dl = (d4d8 * static_cast<float>(ls - 32));
                    if (valid) tr[8 * i + s] = (dl * static_cast<float>(sumi));
                } else {
                    int part;
                    if constexpr (TYPE == MI355X_TYPE_IQ3_S) part = iq3s_bsum(g, s, q8, grid);
                    else if constexpr (TYPE == MI355X_TYPE_IQ3_XXS) part = iq3xxs_bsum(g, s, q8, grid);
                    else part = iq2s_bsum(g, s, q8, grid);
                    const int bsum = sum8(part);
                    const float d = (half_f(g.d) * dx);
                    if (valid && s == 0) tr[i] = (d * static_cast<float>(bsum));
                }
            }
            // the next row's loads before this row's terms are summed
            load_group<TYPE, 1, NIT>(a, row + stride < a.N ? row + stride : a.N - 1, s, bl, regs);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // chains: one lane per (row, chain), terms in ggml's order
        if constexpr (EIGHT) {
            constexpr int C = MINS ? 9 : 8;
            for (int task = lane; task < nrow * C; task += 64) {
                const int r = task / C, c = task % C;
                const float *src = tw + r * per_row + c * S;
                float acc = 0.0f;
                if (c < 8) {
                    acc = ordered_sum(src, S);
                } else {
                    for (int i = 0; i < S; ++i) acc = (acc - src[i]);
                }
                tw[r * per_row + c * S] = acc;  // the chain's first term is no longer needed
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (lane < nrow) {
                const float *cr = tw + lane * per_row;
                float sumf = MINS ? cr[8 * S] : 0.0f;
#pragma unroll
                for (int l = 0; l < 8; ++l) sumf = (sumf + cr[l * S]);
                a.y[first + lane * stride] = sumf;
            }
        } else {
            if (lane < nrow) {
                float sumf = ordered_sum(tw + lane * per_row, per_row);
                if constexpr (TYPE == MI355X_TYPE_IQ3_XXS) sumf = (0.25f * sumf);
                if constexpr (TYPE == MI355X_TYPE_IQ2_S) sumf = (0.125f * sumf);
                a.y[first + lane * stride] = sumf;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

typedef void (*kq_q8k_fn)(KqArgs, int);

template <int TYPE>
kq_q8k_fn pick_q8k_type(int nit) {
    switch (nit) {
    case 1: return gemv_kq_q8k_kernel<TYPE, 1>;
    case 2: return gemv_kq_q8k_kernel<TYPE, 2>;
    case 3: return gemv_kq_q8k_kernel<TYPE, 3>;
    case 4: return gemv_kq_q8k_kernel<TYPE, 4>;
    case 5: return gemv_kq_q8k_kernel<TYPE, 5>;
    case 6: return gemv_kq_q8k_kernel<TYPE, 6>;
    case 7: return gemv_kq_q8k_kernel<TYPE, 7>;
    default: return gemv_kq_q8k_kernel<TYPE, 8>;
    }
}

kq_q8k_fn pick_q8k_kernel(int type, int nit) {
    switch (type) {
    case MI355X_TYPE_Q4_K: return pick_q8k_type<MI355X_TYPE_Q4_K>(nit);
    case MI355X_TYPE_Q5_K: return pick_q8k_type<MI355X_TYPE_Q5_K>(nit);
    case MI355X_TYPE_Q3_K: return pick_q8k_type<MI355X_TYPE_Q3_K>(nit);
    case MI355X_TYPE_Q6_K: return pick_q8k_type<MI355X_TYPE_Q6_K>(nit);
    case MI355X_TYPE_IQ4_XS: return pick_q8k_type<MI355X_TYPE_IQ4_XS>(nit);
    case MI355X_TYPE_IQ3_S: return pick_q8k_type<MI355X_TYPE_IQ3_S>(nit);
    case MI355X_TYPE_IQ3_XXS: return pick_q8k_type<MI355X_TYPE_IQ3_XXS>(nit);
    case MI355X_TYPE_IQ2_S: return pick_q8k_type<MI355X_TYPE_IQ2_S>(nit);
    default: return nullptr;
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

    // activations as 16-byte aligned f32 (bf16 and unaligned inputs go
    // through the context's activation buffer; the context lock keeps the
    // buffer in place from the conversion to the last launch that reads it)
    const float *x = static_cast<const float *>(a.x);
    std::unique_lock<std::mutex> lk(ctx->mu, std::defer_lock);
    if (a.x_bf16 || (reinterpret_cast<uintptr_t>(a.x) & 15) != 0) {
        lk.lock();
        const size_t need = static_cast<size_t>(a.K) * sizeof(float);
        if (ctx->xconv_bytes < need) {
            const int rc = free_device(ctx, ctx->xconv);
            if (rc) return rc;
            ctx->xconv = nullptr;
            ctx->xconv_bytes = 0;
            MI355X_HIP(hipMalloc(&ctx->xconv, need));
            ctx->xconv_bytes = need;
        }
        float *dst = static_cast<float *>(ctx->xconv);
        if (a.x_bf16) {
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((a.K + 255) / 256, 1024));
            hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(blocks), dim3(256), 0, ctx->stream,
                               static_cast<const uint16_t *>(a.x), dst, a.K);
            MI355X_HIP(hipGetLastError());
        } else {
            MI355X_HIP(hipMemcpyAsync(dst, a.x, need, hipMemcpyDeviceToDevice, ctx->stream));
        }
        x = dst;
    }

    // ggml-cpu numerics: the whole row in one launch (ggml's sums run over
    // every superblock in order)
    if (ctx->kernel_variant == MI355X_VARIANT_GGML_Q8) {
        if (B > kQ8kMaxBlocks)
            return set_error(MI355X_EUNSUPPORTED,
                             "the ggml-cpu numerics variant takes K/IQ rows of up to 16384 values");
        const bool eight = a.type == MI355X_TYPE_Q3_K || a.type == MI355X_TYPE_Q4_K || a.type == MI355X_TYPE_Q5_K ||
                           a.type == MI355X_TYPE_Q6_K;
        const bool mins = a.type == MI355X_TYPE_Q4_K || a.type == MI355X_TYPE_Q5_K;
        const int64_t per_row = eight ? (mins ? 9 : 8) * B : (a.type == MI355X_TYPE_IQ4_XS ? 8 * B : B);
        const int rb = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kQ8kMaxBatch, kQ8kTermFloats / per_row)));
        const int nit = static_cast<int>((B + kBlocksPerStep - 1) / kBlocksPerStep);
        const kq_q8k_fn k = pick_q8k_kernel(a.type, nit);
        const size_t lds = static_cast<size_t>(B) * (kQ8kStride + 32 + 4) +
                           static_cast<size_t>(kWaves) * kQ8kTermFloats * sizeof(float) + grid_words(a.type) * 4u;
        if (lds > ctx->max_lds_per_block) return set_error(MI355X_EUNSUPPORTED, "activation row exceeds LDS");
        const int occ = occupancy(reinterpret_cast<const void *>(k), kThreads, lds);
        int64_t wgs = std::min<int64_t>((a.N + kWaves - 1) / kWaves, static_cast<int64_t>(ctx->num_cus) * occ);
        if (ctx->grid_override > 0) wgs = std::min<int64_t>(wgs, ctx->grid_override);
        KqArgs args{a.W, a.N, row_bytes, static_cast<int>(B), 0, static_cast<int>(B), x, a.y, 0, grid};
        hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(std::max<int64_t>(wgs, 1))), dim3(kThreads), lds,
                           ctx->stream, args, rb);
        MI355X_HIP(hipGetLastError());
        return MI355X_OK;
    }

    const bool grid_type = a.type == MI355X_TYPE_IQ3_S || a.type == MI355X_TYPE_IQ3_XXS || a.type == MI355X_TYPE_IQ2_S;
    const bool dg_forced = ctx->kernel_variant == MI355X_VARIANT_DIGITS;

    // equal chunks of at most kChunkBlocks superblocks
    const int64_t n_chunks = (B + kChunkBlocks - 1) / kChunkBlocks;
    const int64_t per_chunk = (B + n_chunks - 1) / n_chunks;
    // Default forms (variant and form AUTO), from sweeps of the BASELINE
    // shapes on MI355X (us, 14336x4096 / 4096x14336; 8192x8192 for IQ;
    // boxes differ by up to ~0.4 us):
    //  * every type: digit rows, one row per wavefront step, each step's
    //    registers refilled with the next row group's step right after its
    //    decode (Q3_K 9.1 / 10.9, Q4_K 7.9 / 9.3, Q5_K 9.8 / 11.1, Q6_K
    //    11.1 / 13.2, IQ4_XS 10.7, IQ3_S 11.4, IQ2_S 10.6, IQ3_XXS 9.8; the
    //    next group loaded after the whole decode: 10.2 / 11.5, 8.3 / 9.9,
    //    9.8 / 11.4, 11.2 / 13.3, 11.0, 11.6 (two rows per step), 10.8 (two
    //    rows), 10.0);
    //  * IQ4_XS only up to four steps and the codebook types only up to
    //    four steps and N >= 4096 (f32 rows otherwise): table-driven sign
    //    application and dot4 products cost fewer VALU instructions than the
    //    f32 decode (f32 14.0 / 12.2 / 12.7 for IQ3_S / IQ3_XXS / IQ2_S).
    // Prefetch (a second register set for the next row group, requested
    // before the current one's decode) is off by default: the refill gives
    // the loads the same head start without the second set (Q3_K 9.2 / 10.9
    // with prefetch).
    auto dg_rows_auto = [&](int nit) {
        switch (a.type) {
        case MI355X_TYPE_Q3_K:
        case MI355X_TYPE_Q4_K:
        case MI355X_TYPE_Q5_K:
        case MI355X_TYPE_Q6_K: return true;
        case MI355X_TYPE_IQ4_XS: return nit <= 4;
        default: return grid_type && nit <= max_nit_r2(a.type) && a.N >= 4096;
        }
    };
    for (int64_t b0 = 0; b0 < B; b0 += per_chunk) {
        const int nb = static_cast<int>(std::min<int64_t>(per_chunk, B - b0));
        const int nit = (nb + kBlocksPerStep - 1) / kBlocksPerStep;
        const bool pl = ctx->kernel_variant != MI355X_VARIANT_EXACT_F32 &&
                        ctx->form_override == MI355X_FORM_PIPE;
        const bool xs = ctx->kernel_variant != MI355X_VARIANT_EXACT_F32 && ctx->form_override == MI355X_FORM_KSPLIT;
        if (xs) {
            const int rb = ctx->rows_override == 2 || ctx->rows_override == 4 ? ctx->rows_override
                                                                                : xs_default_rows(a.type);
            const kq_xs_fn k = pick_xs(a.type, rb);
            const int S = nit;
            const int G = std::max(1, kXsMaxWaves / S);
            if (64 * S * G < kXsMinThreads)
                return set_error(MI355X_EUNSUPPORTED, "too few wavefronts for the codebook staging");
            // LDS: digits, codebook, two tiles of lane partials, then one
            // float per row of the workgroup (at most kXsMaxRows)
            const size_t lds0 = dg_lds_bytes(nb) + dg_table_words(a.type) * 4u +
                                2u * static_cast<size_t>(G) * rb * S * 64 * sizeof(float);
            const int occ = occupancy(reinterpret_cast<const void *>(k), 64 * S * G, lds0 + kXsMaxRows * sizeof(float));
            const int64_t tile = static_cast<int64_t>(G) * rb;
            int64_t wgs = std::min<int64_t>((a.N + tile - 1) / tile, static_cast<int64_t>(ctx->num_cus) * std::max(occ, 1));
            if (ctx->grid_override > 0) wgs = std::min<int64_t>(wgs, ctx->grid_override);
            wgs = std::max<int64_t>({wgs, 1, (a.N + kXsMaxRows - 1) / kXsMaxRows});
            const int64_t rows_per_wg = (a.N + wgs - 1) / wgs;
            wgs = (a.N + rows_per_wg - 1) / rows_per_wg;
            if (wgs >= (int64_t(1) << 31)) return set_error(MI355X_EUNSUPPORTED, "too many rows");
            const size_t lds = lds0 + static_cast<size_t>(rows_per_wg) * sizeof(float);
            if (lds > ctx->max_lds_per_block) return set_error(MI355X_EUNSUPPORTED, "activation chunk exceeds LDS");
            KqArgs args{a.W, a.N, row_bytes, static_cast<int>(B), static_cast<int>(b0), nb, x, a.y, b0 > 0 ? 1 : 0,
                        grid};
            hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(wgs)), dim3(64 * S * G), lds, ctx->stream, args, G,
                               static_cast<int>(rows_per_wg));
            MI355X_HIP(hipGetLastError());
            continue;
        }
        if (pl) {
            const kq_pl_fn k = pick_pl_kernel(a.type, nit);
            const size_t lds = dg_lds_bytes(nb) + dg_table_words(a.type) * 4u;
            if (lds > ctx->max_lds_per_block) return set_error(MI355X_EUNSUPPORTED, "activation chunk exceeds LDS");
            const int64_t slots = static_cast<int64_t>(ctx->num_cus) * kPlqWaves;
            const int64_t rows = (a.N + slots - 1) / slots;
            const int64_t wgs = (a.N + rows * kPlqWaves - 1) / (rows * kPlqWaves);
            KqArgs args{a.W, a.N, row_bytes, static_cast<int>(B), static_cast<int>(b0), nb, x, a.y, b0 > 0 ? 1 : 0,
                        grid};
            hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(wgs)), dim3(kPlqThreads), lds, ctx->stream, args,
                               static_cast<int>(rows));
            MI355X_HIP(hipGetLastError());
            continue;
        }
        const bool dg_auto = ctx->kernel_variant == MI355X_VARIANT_AUTO && dg_rows_auto(nit);
        const bool dg = dg_forced || dg_auto;
        int R = 1;
        if (ctx->rows_override == 1 || (ctx->rows_override == 2 && nit <= max_nit_r2(a.type))) R = ctx->rows_override;
        const bool pf = R == 1 && ctx->prefetch_override == 1;
        const bool wide = (a.type == MI355X_TYPE_IQ3_S || a.type == MI355X_TYPE_IQ2_S) && dg && !pf && R == 1 &&
                          nit <= kWideMaxNit && nb >= 32 &&
                          !ctx->ov_open;
        const int nt = wide ? kWideThreads : kThreads;
        const kq_kernel_fn k = pick_kernel(a.type, R, nit, dg, pf, wide);
        const int64_t n_groups = (a.N + R - 1) / R;
        // dynamic LDS: the records (the codebook is the kernel's static LDS)
        const size_t lds = dg ? dg_lds_bytes(nb) : x_lds_bytes(nb);
        if (lds + (dg ? dg_table_words(a.type) : grid_words(a.type)) * 4u > ctx->max_lds_per_block)
            return set_error(MI355X_EUNSUPPORTED, "activation chunk exceeds LDS");
        // Workgroups per CU: every workgroup stages the whole chunk, so long
        // chunks take one per CU (each wavefront then walks more row groups,
        // its refills overlapping them) and 16-31 superblocks at most two
        // (measured, us: 8192x8192 IQ2_S / IQ3_XXS / IQ4_XS 9.1 / 8.8 / 9.5
        // with one against 9.5 / 9.3 / 9.8 with two; 4096x14336 Q4_K 8.7 vs
        // 10.2; 14336x4096 Q3_K / Q4_K / Q6_K 8.4 / 7.5 / 11.0 with two
        // against 8.8 / 8.1 / 11.7 with three).
        const int occ = occupancy(reinterpret_cast<const void *>(k), nt, lds);
        const int per_cu = nb >= 32 ? 1 : nb >= 16 ? std::min(occ, 2) : occ;
        const int nw = nt / 64;
        int64_t wgs = std::min<int64_t>((n_groups + nw - 1) / nw, static_cast<int64_t>(ctx->num_cus) * per_cu);
        if (ctx->grid_override > 0) wgs = std::min<int64_t>(wgs, ctx->grid_override);
        KqArgs args{a.W, a.N, row_bytes, static_cast<int>(B), static_cast<int>(b0), nb, x, a.y, b0 > 0 ? 1 : 0,
                    grid};
        hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(std::max<int64_t>(wgs, 1))), dim3(nt), lds,
                           ctx->stream, args);
        MI355X_HIP(hipGetLastError());
    }
    return MI355X_OK;
}

}  // namespace mi355x
