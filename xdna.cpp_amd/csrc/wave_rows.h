// Cross-lane helpers for kernels in which each lane holds one partial per
// row of a step of S rows ("stream" work splits, where a lane owns a fixed
// slice of K and the wavefront walks rows).
#pragma once

#include "device_common.h"

namespace mi355x {

template <int CTRL>
__device__ __forceinline__ float st_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// a and b become (a_lo | b_lo) and (a_hi | b_hi) over the wave halves
// (v_permlane32_swap exchanges lanes 32-63 of a with lanes 0-31 of b)
__device__ __forceinline__ float st_fold32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    // copy the elements out before bit-casting: clang lowers a bit cast of a
    // vector element lvalue (r[1]) as a load from the vector's base address
    const unsigned lo = r[0], hi = r[1];
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
// same within each half (v_permlane16_swap exchanges the odd 16-lane rows of
// a with the even rows of b)
__device__ __forceinline__ float st_fold16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                    false, false);
    // copy the elements out before bit-casting: clang lowers a bit cast of a
    // vector element lvalue (r[1]) as a load from the vector's base address
    const unsigned lo = r[0], hi = r[1];
    return __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
}
// merge two rows across a DPP pairing that flips lane bit `bit`: lanes with
// the bit clear keep a's row, lanes with it set b's row
template <int CTRL>
__device__ __forceinline__ float st_fold_dpp(float a, float b, bool bit) {
    const float own = bit ? b : a;
    const float other = bit ? a : b;
    return own + st_dpp<CTRL>(other);
}

// Sum of S per-lane values across the wavefront.  On return, lane l holds
// the total of row l >> (6 - log2 S) (all 64/S lanes of a group agree).
// Partners per stage: lane ^ 32, lane ^ 16, row mirror (lane ^ 15), half-row
// mirror (lane ^ 7), quad swaps (lane ^ 2, lane ^ 1) -- together every lane.
template <int S>
__device__ __forceinline__ float st_reduce(float v[S], int lane) {
    static_assert(S == 4 || S == 8 || S == 16, "rows per step");
#pragma unroll
    for (int i = 0; i < S / 2; ++i) v[i] = st_fold32(v[i], v[i + S / 2]);
#pragma unroll
    for (int i = 0; i < S / 4; ++i) v[i] = st_fold16(v[i], v[i + S / 4]);
    float t;
    if constexpr (S == 16) {
        v[0] = st_fold_dpp<0x140>(v[0], v[2], lane & 8);
        v[1] = st_fold_dpp<0x140>(v[1], v[3], lane & 8);
        t = st_fold_dpp<0x141>(v[0], v[1], lane & 4);
    } else if constexpr (S == 8) {
        t = st_fold_dpp<0x140>(v[0], v[1], lane & 8);
        t += st_dpp<0x141>(t);
    } else {
        t = v[0];
        t += st_dpp<0x140>(t);
        t += st_dpp<0x141>(t);
    }
    t += st_dpp<0x4E>(t);  // quad_perm [2,3,0,1]
    t += st_dpp<0xB1>(t);  // quad_perm [1,0,3,2]
    return t;
}

}  // namespace mi355x
