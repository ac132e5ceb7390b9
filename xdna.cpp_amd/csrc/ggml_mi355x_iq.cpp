// IQ3_XXS and IQ2_S grids taken from the host's ggml at run time.
//
// Both formats index a codebook (iq3xxs_grid: 256 x 4 bytes, iq2s_grid:
// 1024 x 8 bytes) that lives inside ggml and is not part of this library.
// When the host process exports ggml's dequantize_row_iq3_xxs /
// dequantize_row_iq2_s, the codebook is read back by dequantizing probe
// blocks whose every grid index is known, with d = 1, the smallest block
// scale and no sign flips, so each output is grid_byte * 2^-k exactly.
// Random blocks are then dequantized both by ggml and by the block formula
// below with the recovered grid; only a bit-exact match installs the grid.
//
// Block formulas: ggml dequantize_row_iq3_xxs / dequantize_row_iq2_s, as
// restated by the reference's kernels (src/xdna-gemv-engine.cpp:1388-1396
// selects them; ggml-quants.c holds the definitions).
#include "mi355x-gemv.h"

#include <dlfcn.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

namespace {

constexpr int kQK = 256;
constexpr int kIq3xxsBlock = 2 + 3 * kQK / 8;              // d, qs[96]
constexpr int kIq2sBlock = 2 + kQK / 4 + kQK / 32 + kQK / 32;  // d, qs[64], qh[8], scales[8]

float half_to_float(uint16_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    float f;
    if (exp == 0) {
        f = std::ldexp(static_cast<float>(man), -24);
    } else if (exp == 31) {
        f = man ? NAN : INFINITY;
    } else {
        f = std::ldexp(static_cast<float>(man | 0x400), static_cast<int>(exp) - 25);
    }
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    bits |= sign;
    std::memcpy(&f, &bits, 4);
    return f;
}

// ksigns_iq2xs[i]: the 7 stored sign bits plus an eighth bit that makes the
// number of set bits even.
uint8_t ksign(int i) { return static_cast<uint8_t>(i | ((__builtin_popcount(i) & 1) << 7)); }

typedef void (*dequant_fn)(const void *, float *, int64_t);

dequant_fn find(const char *name) { return reinterpret_cast<dequant_fn>(dlsym(RTLD_DEFAULT, name)); }

// Host restatement of one IQ3_XXS block with a candidate grid.
void iq3xxs_block(const uint8_t *blk, const uint32_t *grid, float *y) {
    uint16_t dh;
    std::memcpy(&dh, blk, 2);
    const float d = half_to_float(dh);
    const uint8_t *qs = blk + 2;
    const uint8_t *ss = blk + 2 + kQK / 4;
    for (int ib = 0; ib < kQK / 32; ++ib) {
        uint32_t aux;
        std::memcpy(&aux, ss + 4 * ib, 4);
        const float db = d * (0.5f + (aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; ++l) {
            const uint8_t s = ksign((aux >> (7 * l)) & 127);
            const uint8_t *g1 = reinterpret_cast<const uint8_t *>(&grid[qs[2 * l]]);
            const uint8_t *g2 = reinterpret_cast<const uint8_t *>(&grid[qs[2 * l + 1]]);
            for (int j = 0; j < 4; ++j) {
                y[j] = db * g1[j] * ((s >> j) & 1 ? -1.f : 1.f);
                y[j + 4] = db * g2[j] * ((s >> (j + 4)) & 1 ? -1.f : 1.f);
            }
            y += 8;
        }
        qs += 8;
    }
}

// Host restatement of one IQ2_S block with a candidate grid.
void iq2s_block(const uint8_t *blk, const uint64_t *grid, float *y) {
    uint16_t dh;
    std::memcpy(&dh, blk, 2);
    const float d = half_to_float(dh);
    const uint8_t *qs = blk + 2;
    const uint8_t *signs = qs + kQK / 8;
    const uint8_t *qh = blk + 2 + kQK / 4;
    const uint8_t *sc = qh + kQK / 32;
    for (int ib = 0; ib < kQK / 32; ++ib) {
        const float db[2] = {d * (0.5f + (sc[ib] & 0xf)) * 0.25f, d * (0.5f + (sc[ib] >> 4)) * 0.25f};
        for (int l = 0; l < 4; ++l) {
            const float dl = db[l / 2];
            const int idx = qs[l] | ((qh[ib] << (8 - 2 * l)) & 0x300);
            const uint8_t *g = reinterpret_cast<const uint8_t *>(&grid[idx]);
            for (int j = 0; j < 8; ++j) y[j] = dl * g[j] * ((signs[l] >> j) & 1 ? -1.f : 1.f);
            y += 8;
        }
        qs += 4;
        signs += 4;
    }
}

bool grid_byte(float v, float scale, uint8_t *out) {
    const float g = v * scale;
    if (!(g >= 0.f && g <= 255.f) || g != std::floor(g)) return false;
    *out = static_cast<uint8_t>(g);
    return true;
}

bool load_iq3xxs(dequant_fn dq) {
    // 4 probe blocks x 64 indices: block b, position p holds index 64b + p
    constexpr int kBlocks = 4;
    std::vector<uint8_t> probe(kBlocks * kIq3xxsBlock, 0);
    for (int b = 0; b < kBlocks; ++b) {
        uint8_t *blk = &probe[b * kIq3xxsBlock];
        blk[0] = 0x00;
        blk[1] = 0x3c;  // d = 1.0
        for (int p = 0; p < 64; ++p) blk[2 + p] = static_cast<uint8_t>(64 * b + p);
        // scales_and_signs all zero: db = 0.25, sign index 0 (no flips)
    }
    std::vector<float> y(kBlocks * kQK);
    dq(probe.data(), y.data(), kBlocks * kQK);
    uint32_t grid[256];
    for (int i = 0; i < 256; ++i) {
        uint8_t g[4];
        for (int j = 0; j < 4; ++j)
            if (!grid_byte(y[4 * i + j], 4.f, &g[j])) return false;
        std::memcpy(&grid[i], g, 4);
    }
    std::mt19937 rng(0x1A3);
    constexpr int kCheck = 16;
    std::vector<uint8_t> rnd(kCheck * kIq3xxsBlock);
    for (auto &c : rnd) c = static_cast<uint8_t>(rng());
    for (int b = 0; b < kCheck; ++b) {  // finite d in [2^-8, 2)
        rnd[b * kIq3xxsBlock + 1] = static_cast<uint8_t>(0x1c + (rng() % 32));
    }
    std::vector<float> want(kCheck * kQK), got(kCheck * kQK);
    dq(rnd.data(), want.data(), kCheck * kQK);
    for (int b = 0; b < kCheck; ++b) iq3xxs_block(&rnd[b * kIq3xxsBlock], grid, &got[b * kQK]);
    if (std::memcmp(want.data(), got.data(), want.size() * sizeof(float)) != 0) return false;
    return mi355x_set_iq_grid(MI355X_TYPE_IQ3_XXS, grid, sizeof grid) == MI355X_OK;
}

bool load_iq2s(dequant_fn dq) {
    // 32 probe blocks x 32 indices: block b, group ib, slot l holds 32b + 4ib + l
    constexpr int kBlocks = 32;
    std::vector<uint8_t> probe(kBlocks * kIq2sBlock, 0);
    for (int b = 0; b < kBlocks; ++b) {
        uint8_t *blk = &probe[b * kIq2sBlock];
        blk[0] = 0x00;
        blk[1] = 0x3c;  // d = 1.0
        uint8_t *qs = blk + 2;
        uint8_t *qh = blk + 2 + kQK / 4;
        for (int ib = 0; ib < 8; ++ib) {
            for (int l = 0; l < 4; ++l) {
                const int idx = 32 * b + 4 * ib + l;
                qs[4 * ib + l] = static_cast<uint8_t>(idx & 0xff);
                qh[ib] = static_cast<uint8_t>(qh[ib] | (((idx >> 8) & 3) << (2 * l)));
            }
        }
        // signs and scales zero: db = 0.125, no flips
    }
    std::vector<float> y(kBlocks * kQK);
    dq(probe.data(), y.data(), kBlocks * kQK);
    std::vector<uint64_t> grid(1024);
    for (int i = 0; i < 1024; ++i) {
        uint8_t g[8];
        for (int j = 0; j < 8; ++j)
            if (!grid_byte(y[8 * i + j], 8.f, &g[j])) return false;
        std::memcpy(&grid[i], g, 8);
    }
    std::mt19937 rng(0x25);
    constexpr int kCheck = 16;
    std::vector<uint8_t> rnd(kCheck * kIq2sBlock);
    for (auto &c : rnd) c = static_cast<uint8_t>(rng());
    for (int b = 0; b < kCheck; ++b) rnd[b * kIq2sBlock + 1] = static_cast<uint8_t>(0x1c + (rng() % 32));
    std::vector<float> want(kCheck * kQK), got(kCheck * kQK);
    dq(rnd.data(), want.data(), kCheck * kQK);
    for (int b = 0; b < kCheck; ++b) iq2s_block(&rnd[b * kIq2sBlock], grid.data(), &got[b * kQK]);
    if (std::memcmp(want.data(), got.data(), want.size() * sizeof(float)) != 0) return false;
    return mi355x_set_iq_grid(MI355X_TYPE_IQ2_S, grid.data(), grid.size() * sizeof(uint64_t)) == MI355X_OK;
}

}  // namespace

int mi355x_iq_grids_from_ggml_impl() {
    int n = 0;
    if (dequant_fn f = find("dequantize_row_iq3_xxs")) n += load_iq3xxs(f) ? 1 : 0;
    if (dequant_fn f = find("dequantize_row_iq2_s")) n += load_iq2s(f) ? 1 : 0;
    return n;
}
