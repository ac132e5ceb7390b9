// Resident layout of a Q4_0 row, shared by host and device code.
//
// A ggml Q4_0 row is B blocks of [fp16 d][16 code bytes] (18*B bytes).  The
// resident row keeps the same bytes, reordered:
//   [code bytes of block 0 .. B-1 : 16*B][fp16 d plane : 2*B]
// Code bytes are stored XOR 0x88 (signed nibbles q - 8).  In the d plane the
// first 64*F blocks (F = B / 64 full columns of 64 blocks) are lane-major:
// block b sits at slot (b % 64) * F + b / 64, so the lane that owns blocks
// l, l+64, ..., l+64(F-1) finds their scales side by side and loads them with
// one wide load.  The last B % 64 blocks keep their natural slot b.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MI355X_HD __host__ __device__
#else
#define MI355X_HD
#endif

namespace mi355x {

MI355X_HD inline uint64_t q4_0_d_slot(uint64_t b, uint64_t B) {
    const uint64_t F = B >> 6;
    return b < 64 * F ? (b & 63) * F + (b >> 6) : b;
}

}  // namespace mi355x
