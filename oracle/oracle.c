/*
 * CPU oracle for the quantized decode GEMV path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the numerics contract and the reference lines followed.
 * Build with -ffp-contract=off: the expression order below is the contract.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* src/xdna-q4-0-reference.cpp:207-242: sign | exponent rebias | mantissa,
 * subnormal halves renormalised, inf/nan payload widened. */
float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_to_f32(sign);
        int exp = -14;
        while (!(m & 0x400u)) {
            m <<= 1;
            exp -= 1;
        }
        m &= 0x3ffu;
        return bits_to_f32(sign | ((uint32_t)(exp + 127) << 23) | (m << 13));
    }
    if (e == 31) return bits_to_f32(sign | 0x7f800000u | (m << 13));
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

float orc_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

/* src/xdna-q4-0-reference.cpp:250-259: add 0x7fff + lsb, truncate. */
uint16_t orc_f32_to_bf16(float v) {
    uint32_t u = f32_to_bits(v);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------------ */
/* geometry                                                                  */
/* ------------------------------------------------------------------------ */

int64_t orc_block_values(int type) {
    switch (type) {
    case ORC_Q4_0: return 32;
    case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K:
    case ORC_IQ4_XS: case ORC_IQ3_S: case ORC_IQ3_XXS: case ORC_IQ2_S:
        return 256;
    default: return 0;
    }
}

/* include/xdna/kquants.h:182-194 */
int64_t orc_block_bytes(int type) {
    switch (type) {
    case ORC_Q4_0: return 18;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ4_XS: return 136;
    case ORC_IQ3_S: return 110;
    case ORC_IQ3_XXS: return 98;
    case ORC_IQ2_S: return 82;
    default: return 0;
    }
}

int64_t orc_row_bytes(int type, int64_t K) {
    int64_t bv = orc_block_values(type);
    if (bv == 0 || K < 0 || K % bv != 0) return -1;
    return (K / bv) * orc_block_bytes(type);
}

/* src/xdna-q4-0-reference.cpp:261-300 */
int orc_q4_0_validate_row(uint64_t value_count, uint64_t encoded_bytes) {
    if (value_count % 32u != 0) return ORC_EINVAL;
    uint64_t blocks = value_count / 32u;
    if (blocks > UINT64_MAX / 18u) return ORC_EINVAL;
    return encoded_bytes == blocks * 18u ? ORC_OK : ORC_EINVAL;
}

int orc_q4_0_validate_matrix(uint64_t rows, uint64_t values_per_row,
                             uint64_t encoded_bytes) {
    if (values_per_row % 32u != 0) return ORC_EINVAL;
    uint64_t row_bytes = (values_per_row / 32u) * 18u;
    if (rows != 0 && row_bytes > UINT64_MAX / rows) return ORC_EINVAL;
    return encoded_bytes == rows * row_bytes ? ORC_OK : ORC_EINVAL;
}

/* ------------------------------------------------------------------------ */
/* format tables                                                             */
/* ------------------------------------------------------------------------ */

/* IQ4_NL codebook (include/xdna/kquants.h:215-217). */
static const int8_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                   1,    13,   25,  38,  53,  69,  89,  113};

/* IQ3_S grid, 512 entries of four odd magnitudes 1..15 (include/xdna/kquants.h:220-285). */
static const uint32_t k_iq3s_grid[512] = {
    0x01010101u, 0x01010103u, 0x01010105u, 0x0101010bu, 0x0101010fu, 0x01010301u, 0x01010303u, 0x01010305u,
    0x01010309u, 0x0101030du, 0x01010501u, 0x01010503u, 0x0101050bu, 0x01010707u, 0x01010901u, 0x01010905u,
    0x0101090bu, 0x0101090fu, 0x01010b03u, 0x01010b07u, 0x01010d01u, 0x01010d05u, 0x01010f03u, 0x01010f09u,
    0x01010f0fu, 0x01030101u, 0x01030103u, 0x01030105u, 0x01030109u, 0x01030301u, 0x01030303u, 0x0103030bu,
    0x01030501u, 0x01030507u, 0x0103050fu, 0x01030703u, 0x0103070bu, 0x01030909u, 0x01030d03u, 0x01030d0bu,
    0x01030f05u, 0x01050101u, 0x01050103u, 0x0105010bu, 0x0105010fu, 0x01050301u, 0x01050307u, 0x0105030du,
    0x01050503u, 0x0105050bu, 0x01050701u, 0x01050709u, 0x01050905u, 0x0105090bu, 0x0105090fu, 0x01050b03u,
    0x01050b07u, 0x01050f01u, 0x01050f07u, 0x01070107u, 0x01070303u, 0x0107030bu, 0x01070501u, 0x01070505u,
    0x01070703u, 0x01070707u, 0x0107070du, 0x01070909u, 0x01070b01u, 0x01070b05u, 0x01070d0fu, 0x01070f03u,
    0x01070f0bu, 0x01090101u, 0x01090307u, 0x0109030fu, 0x01090503u, 0x01090509u, 0x01090705u, 0x01090901u,
    0x01090907u, 0x01090b03u, 0x01090f01u, 0x010b0105u, 0x010b0109u, 0x010b0501u, 0x010b0505u, 0x010b050du,
    0x010b0707u, 0x010b0903u, 0x010b090bu, 0x010b090fu, 0x010b0d0du, 0x010b0f07u, 0x010d010du, 0x010d0303u,
    0x010d0307u, 0x010d0703u, 0x010d0b05u, 0x010d0f03u, 0x010f0101u, 0x010f0105u, 0x010f0109u, 0x010f0501u,
    0x010f0505u, 0x010f050du, 0x010f0707u, 0x010f0b01u, 0x010f0b09u, 0x03010101u, 0x03010103u, 0x03010105u,
    0x03010109u, 0x03010301u, 0x03010303u, 0x03010307u, 0x0301030bu, 0x0301030fu, 0x03010501u, 0x03010505u,
    0x03010703u, 0x03010709u, 0x0301070du, 0x03010b09u, 0x03010b0du, 0x03010d03u, 0x03010f05u, 0x03030101u,
    0x03030103u, 0x03030107u, 0x0303010du, 0x03030301u, 0x03030309u, 0x03030503u, 0x03030701u, 0x03030707u,
    0x03030903u, 0x03030b01u, 0x03030b05u, 0x03030f01u, 0x03030f0du, 0x03050101u, 0x03050305u, 0x0305030bu,
    0x0305030fu, 0x03050501u, 0x03050509u, 0x03050705u, 0x03050901u, 0x03050907u, 0x03050b0bu, 0x03050d01u,
    0x03050f05u, 0x03070103u, 0x03070109u, 0x0307010fu, 0x03070301u, 0x03070307u, 0x03070503u, 0x0307050fu,
    0x03070701u, 0x03070709u, 0x03070903u, 0x03070d05u, 0x03070f01u, 0x03090107u, 0x0309010bu, 0x03090305u,
    0x03090309u, 0x03090703u, 0x03090707u, 0x03090905u, 0x0309090du, 0x03090b01u, 0x03090b09u, 0x030b0103u,
    0x030b0301u, 0x030b0307u, 0x030b0503u, 0x030b0701u, 0x030b0705u, 0x030b0b03u, 0x030d0501u, 0x030d0509u,
    0x030d050fu, 0x030d0909u, 0x030d090du, 0x030f0103u, 0x030f0107u, 0x030f0301u, 0x030f0305u, 0x030f0503u,
    0x030f070bu, 0x030f0903u, 0x030f0d05u, 0x030f0f01u, 0x05010101u, 0x05010103u, 0x05010107u, 0x0501010bu,
    0x0501010fu, 0x05010301u, 0x05010305u, 0x05010309u, 0x0501030du, 0x05010503u, 0x05010507u, 0x0501050fu,
    0x05010701u, 0x05010705u, 0x05010903u, 0x05010907u, 0x0501090bu, 0x05010b01u, 0x05010b05u, 0x05010d0fu,
    0x05010f01u, 0x05010f07u, 0x05010f0bu, 0x05030101u, 0x05030105u, 0x05030301u, 0x05030307u, 0x0503030fu,
    0x05030505u, 0x0503050bu, 0x05030703u, 0x05030709u, 0x05030905u, 0x05030b03u, 0x05050103u, 0x05050109u,
    0x0505010fu, 0x05050503u, 0x05050507u, 0x05050701u, 0x0505070fu, 0x05050903u, 0x05050b07u, 0x05050b0fu,
    0x05050f03u, 0x05050f09u, 0x05070101u, 0x05070105u, 0x0507010bu, 0x05070303u, 0x05070505u, 0x05070509u,
    0x05070703u, 0x05070707u, 0x05070905u, 0x05070b01u, 0x05070d0du, 0x05090103u, 0x0509010fu, 0x05090501u,
    0x05090507u, 0x05090705u, 0x0509070bu, 0x05090903u, 0x05090f05u, 0x05090f0bu, 0x050b0109u, 0x050b0303u,
    0x050b0505u, 0x050b070fu, 0x050b0901u, 0x050b0b07u, 0x050b0f01u, 0x050d0101u, 0x050d0105u, 0x050d010fu,
    0x050d0503u, 0x050d0b0bu, 0x050d0d03u, 0x050f010bu, 0x050f0303u, 0x050f050du, 0x050f0701u, 0x050f0907u,
    0x050f0b01u, 0x07010105u, 0x07010303u, 0x07010307u, 0x0701030bu, 0x0701030fu, 0x07010505u, 0x07010703u,
    0x07010707u, 0x0701070bu, 0x07010905u, 0x07010909u, 0x0701090fu, 0x07010b03u, 0x07010d07u, 0x07010f03u,
    0x07030103u, 0x07030107u, 0x0703010bu, 0x07030309u, 0x07030503u, 0x07030507u, 0x07030901u, 0x07030d01u,
    0x07030f05u, 0x07030f0du, 0x07050101u, 0x07050305u, 0x07050501u, 0x07050705u, 0x07050709u, 0x07050b01u,
    0x07070103u, 0x07070301u, 0x07070309u, 0x07070503u, 0x07070507u, 0x0707050fu, 0x07070701u, 0x07070903u,
    0x07070907u, 0x0707090fu, 0x07070b0bu, 0x07070f07u, 0x07090107u, 0x07090303u, 0x0709030du, 0x07090505u,
    0x07090703u, 0x07090b05u, 0x07090d01u, 0x07090d09u, 0x070b0103u, 0x070b0301u, 0x070b0305u, 0x070b050bu,
    0x070b0705u, 0x070b0909u, 0x070b0b0du, 0x070b0f07u, 0x070d030du, 0x070d0903u, 0x070f0103u, 0x070f0107u,
    0x070f0501u, 0x070f0505u, 0x070f070bu, 0x09010101u, 0x09010109u, 0x09010305u, 0x09010501u, 0x09010509u,
    0x0901050fu, 0x09010705u, 0x09010903u, 0x09010b01u, 0x09010f01u, 0x09030105u, 0x0903010fu, 0x09030303u,
    0x09030307u, 0x09030505u, 0x09030701u, 0x0903070bu, 0x09030907u, 0x09030b03u, 0x09030b0bu, 0x09050103u,
    0x09050107u, 0x09050301u, 0x0905030bu, 0x09050503u, 0x09050707u, 0x09050901u, 0x09050b0fu, 0x09050d05u,
    0x09050f01u, 0x09070109u, 0x09070303u, 0x09070307u, 0x09070501u, 0x09070505u, 0x09070703u, 0x0907070bu,
    0x09090101u, 0x09090105u, 0x09090509u, 0x0909070fu, 0x09090901u, 0x09090f03u, 0x090b010bu, 0x090b010fu,
    0x090b0503u, 0x090b0d05u, 0x090d0307u, 0x090d0709u, 0x090d0d01u, 0x090f0301u, 0x090f030bu, 0x090f0701u,
    0x090f0907u, 0x090f0b03u, 0x0b010105u, 0x0b010301u, 0x0b010309u, 0x0b010505u, 0x0b010901u, 0x0b010909u,
    0x0b01090fu, 0x0b010b05u, 0x0b010d0du, 0x0b010f09u, 0x0b030103u, 0x0b030107u, 0x0b03010bu, 0x0b030305u,
    0x0b030503u, 0x0b030705u, 0x0b030f05u, 0x0b050101u, 0x0b050303u, 0x0b050507u, 0x0b050701u, 0x0b05070du,
    0x0b050b07u, 0x0b070105u, 0x0b07010fu, 0x0b070301u, 0x0b07050fu, 0x0b070909u, 0x0b070b03u, 0x0b070d0bu,
    0x0b070f07u, 0x0b090103u, 0x0b090109u, 0x0b090501u, 0x0b090705u, 0x0b09090du, 0x0b0b0305u, 0x0b0b050du,
    0x0b0b0b03u, 0x0b0b0b07u, 0x0b0d0905u, 0x0b0f0105u, 0x0b0f0109u, 0x0b0f0505u, 0x0d010303u, 0x0d010307u,
    0x0d01030bu, 0x0d010703u, 0x0d010707u, 0x0d010d01u, 0x0d030101u, 0x0d030501u, 0x0d03050fu, 0x0d030d09u,
    0x0d050305u, 0x0d050709u, 0x0d050905u, 0x0d050b0bu, 0x0d050d05u, 0x0d050f01u, 0x0d070101u, 0x0d070309u,
    0x0d070503u, 0x0d070901u, 0x0d09050bu, 0x0d090907u, 0x0d090d05u, 0x0d0b0101u, 0x0d0b0107u, 0x0d0b0709u,
    0x0d0b0d01u, 0x0d0d010bu, 0x0d0d0901u, 0x0d0f0303u, 0x0d0f0307u, 0x0f010101u, 0x0f010109u, 0x0f01010fu,
    0x0f010501u, 0x0f010505u, 0x0f01070du, 0x0f010901u, 0x0f010b09u, 0x0f010d05u, 0x0f030105u, 0x0f030303u,
    0x0f030509u, 0x0f030907u, 0x0f03090bu, 0x0f050103u, 0x0f050109u, 0x0f050301u, 0x0f05030du, 0x0f050503u,
    0x0f050701u, 0x0f050b03u, 0x0f070105u, 0x0f070705u, 0x0f07070bu, 0x0f070b07u, 0x0f090103u, 0x0f09010bu,
    0x0f090307u, 0x0f090501u, 0x0f090b01u, 0x0f0b0505u, 0x0f0b0905u, 0x0f0d0105u, 0x0f0d0703u, 0x0f0f0101u,
};

uint8_t orc_ksigns_iq2xs(int i) {
    int parity = __builtin_popcount((unsigned)i) & 1;
    return (uint8_t)(i | (parity << 7));
}

/* ------------------------------------------------------------------------ */
/* per-type row dequantizers                                                 */
/* ------------------------------------------------------------------------ */

/* Q4_0: 18-byte block, fp16 d then 16 bytes; value j = (qs[j] & 15) - 8,
 * value j + 16 = (qs[j] >> 4) - 8; w = (float)q * d
 * (include/xdna/q4_0_reference.h:15-33, src/xdna-q4-0-reference.cpp:302-328). */
static void dq_q4_0(const uint8_t *row, int64_t K, float *y) {
    for (int64_t b = 0; b < K / 32; ++b) {
        const uint8_t *blk = row + 18 * b;
        float d = orc_fp16_to_f32(rd16(blk));
        const uint8_t *qs = blk + 2;
        for (int j = 0; j < 16; ++j) {
            y[32 * b + j] = (float)((int)(qs[j] & 15) - 8) * d;
            y[32 * b + 16 + j] = (float)((int)(qs[j] >> 4) - 8) * d;
        }
    }
}

/* 6-bit scale/min pair j of a Q4_K/Q5_K block (include/xdna/kquants.h:204-212). */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Integer form of one 256-value superblock: a[p] is the integer every value
 * multiplies (its code, or its signed grid magnitude), sc[g] the integer
 * scale of its group of `group` values (16 or 32), mn[] the Q4_K/Q5_K mins,
 * d/dmin the fp16 block scales.  Both the f32 dequantizers below and the
 * ggml Q8_K dot products further down read blocks through these, so the
 * dequantizers' golden vectors from the reference build also pin the
 * integers the dot products use. */
typedef struct {
    int a[256];
    uint8_t neg[256]; /* grid types: sign bit of value p (a zero magnitude keeps it) */
    int sc[16];
    int mn[8];
    int group;
    float d, dmin;
} kq_int;

/* Q4_K: d, dmin (fp16), 12 scale bytes, 128 quant bytes.  Each 64-value
 * chunk c uses two sub-blocks: low nibbles (sub-block 2c), high nibbles
 * (2c+1) (include/xdna/kquants.h:290-315). */
static void int_q4_k(const uint8_t *blk, kq_int *k) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = orc_fp16_to_f32(rd16(blk + 2));
    k->group = 32;
    for (int j = 0; j < 8; ++j) scale_min_k4(j, blk + 4, &k->sc[j], &k->mn[j]);
    const uint8_t *q = blk + 16;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) {
            k->a[64 * c + l] = q[32 * c + l] & 15;
            k->a[64 * c + 32 + l] = q[32 * c + l] >> 4;
        }
}

/* Q5_K: as Q4_K plus a fifth bit from qh[32]; chunk c takes bit 2c for the
 * low-nibble half and bit 2c+1 for the high half (include/xdna/kquants.h:317-348). */
static void int_q5_k(const uint8_t *blk, kq_int *k) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = orc_fp16_to_f32(rd16(blk + 2));
    k->group = 32;
    for (int j = 0; j < 8; ++j) scale_min_k4(j, blk + 4, &k->sc[j], &k->mn[j]);
    const uint8_t *qh = blk + 16;
    const uint8_t *ql = blk + 48;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) {
            k->a[64 * c + l] = (ql[32 * c + l] & 15) + (((qh[l] >> (2 * c)) & 1) ? 16 : 0);
            k->a[64 * c + 32 + l] = (ql[32 * c + l] >> 4) + (((qh[l] >> (2 * c + 1)) & 1) ? 16 : 0);
        }
}

/* Q3_K: hmask[32], qs[64], 12 packed bytes of sixteen 6-bit scales, fp16 d
 * at byte 108.  Scale s (0..15): low 4 bits from byte s%8 (nibble s/8), high
 * 2 bits from byte 8 + s%4 (bit pair s/4), minus 32.  Value = 2-bit q minus 4
 * when its hmask bit is clear (include/xdna/kquants.h:350-389). */
static void int_q3_k(const uint8_t *blk, kq_int *k) {
    const uint8_t *hm = blk;
    const uint8_t *q = blk + 32;
    const uint8_t *p = blk + 96;
    k->d = orc_fp16_to_f32(rd16(blk + 108));
    k->dmin = 0.0f;
    k->group = 16;
    for (int s = 0; s < 16; ++s) {
        int lo = (p[s % 8] >> (4 * (s / 8))) & 15;
        int hi = (p[8 + s % 4] >> (2 * (s / 4))) & 3;
        k->sc[s] = (lo | (hi << 4)) - 32;
    }
    /* position 128 half + 32 j + i: bits 2j of qs[32 half + i], hmask bit 4 half + j */
    for (int half = 0; half < 2; ++half)
        for (int j = 0; j < 4; ++j)
            for (int i = 0; i < 32; ++i) {
                int v = (q[32 * half + i] >> (2 * j)) & 3;
                k->a[128 * half + 32 * j + i] = v - (((hm[i] >> (4 * half + j)) & 1) ? 0 : 4);
            }
}

/* Q6_K: ql[128], qh[64], int8 scales[16], fp16 d at byte 208.  Per 128-value
 * half: four 32-value groups (ql low, ql+32 low, ql high, ql+32 high) with
 * qh bit pairs 0,2,4,6; q = 6-bit - 32 (include/xdna/kquants.h:391-419). */
static void int_q6_k(const uint8_t *blk, kq_int *k) {
    k->d = orc_fp16_to_f32(rd16(blk + 208));
    k->dmin = 0.0f;
    k->group = 16;
    for (int s = 0; s < 16; ++s) k->sc[s] = (int8_t)blk[192 + s];
    for (int half = 0; half < 2; ++half) {
        const uint8_t *ql = blk + 64 * half;
        const uint8_t *qh = blk + 128 + 32 * half;
        int *a = k->a + 128 * half;
        for (int l = 0; l < 32; ++l) {
            a[l] = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
            a[l + 32] = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            a[l + 64] = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            a[l + 96] = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        }
    }
}

/* IQ4_XS: fp16 d, scales_h (u16), scales_l[4], qs[128].  Sub-block ib of 32:
 * 6-bit ls = nibble ib of scales_l | 2 bits ib of scales_h, scale ls - 32;
 * first 16 values from low nibbles, next 16 from high nibbles through the
 * IQ4_NL codebook (include/xdna/kquants.h:421-441). */
static void int_iq4_xs(const uint8_t *blk, kq_int *k) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = 0.0f;
    k->group = 32;
    unsigned sh = rd16(blk + 2);
    const uint8_t *sl = blk + 4;
    const uint8_t *qs = blk + 8;
    for (int ib = 0; ib < 8; ++ib) {
        int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        k->sc[ib] = ls - 32;
        for (int j = 0; j < 16; ++j) {
            k->a[32 * ib + j] = k_iq4nl[qs[16 * ib + j] & 15];
            k->a[32 * ib + 16 + j] = k_iq4nl[qs[16 * ib + j] >> 4];
        }
    }
}

/* IQ3_S: fp16 d, qs[64], qh[8], signs[32], scales[4].  Eight groups of 32;
 * group g uses scale nibble g of scales (1 + 2 * nib), qh[g] supplies the 9th
 * index bit of its eight grid lookups (bit k for lookup k), signs bytes
 * 4g..4g+3 one bit per value (include/xdna/kquants.h:443-490). */
static void int_iq3_s(const uint8_t *blk, kq_int *k) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = 0.0f;
    k->group = 32;
    const uint8_t *qs = blk + 2;
    const uint8_t *qh = blk + 66;
    const uint8_t *signs = blk + 74;
    const uint8_t *scales = blk + 106;
    for (int g = 0; g < 8; ++g) {
        k->sc[g] = 1 + 2 * ((scales[g / 2] >> (4 * (g % 2))) & 15);
        for (int kk = 0; kk < 8; ++kk) {
            unsigned idx = qs[8 * g + kk] | (((unsigned)qh[g] >> kk & 1u) << 8);
            uint32_t gv = k_iq3s_grid[idx];
            uint8_t sb = signs[4 * g + kk / 2];
            for (int j = 0; j < 4; ++j) {
                int mag = (int)((gv >> (8 * j)) & 0xffu);
                int neg = (sb >> (4 * (kk & 1) + j)) & 1;
                k->neg[32 * g + 4 * kk + j] = (uint8_t)neg;
                k->a[32 * g + 4 * kk + j] = neg ? -mag : mag;
            }
        }
    }
}

/* IQ3_XXS (ggml, external): fp16 d, qs[64] grid indices, then eight u32
 * words (one per 32-value group): bits 0..27 four 7-bit sign indices (bit 7
 * of each sign byte: even parity), bits 28..31 the scale s (integer 2s + 1;
 * ggml's dequantizer computes (d*(0.5+s))*0.5). */
static void int_iq3_xxs(const uint8_t *blk, kq_int *k, const uint32_t *grid) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = 0.0f;
    k->group = 32;
    const uint8_t *qs = blk + 2;
    const uint8_t *ss = blk + 66;
    for (int g = 0; g < 8; ++g) {
        uint32_t aux = (uint32_t)ss[4 * g] | ((uint32_t)ss[4 * g + 1] << 8) |
                       ((uint32_t)ss[4 * g + 2] << 16) | ((uint32_t)ss[4 * g + 3] << 24);
        k->sc[g] = 1 + 2 * (int)(aux >> 28);
        for (int l = 0; l < 4; ++l) {
            uint8_t sg = orc_ksigns_iq2xs((aux >> (7 * l)) & 127);
            for (int h = 0; h < 2; ++h) {
                uint32_t gv = grid[qs[8 * g + 2 * l + h]];
                for (int j = 0; j < 4; ++j) {
                    int mag = (int)((gv >> (8 * j)) & 0xffu);
                    int neg = (sg >> (4 * h + j)) & 1;
                    k->neg[32 * g + 8 * l + 4 * h + j] = (uint8_t)neg;
                    k->a[32 * g + 8 * l + 4 * h + j] = neg ? -mag : mag;
                }
            }
        }
    }
}

/* IQ2_S (ggml, external): fp16 d, qs[32] low index bytes, signs[32], qh[8]
 * (two index bits per lookup), scales[8] (two nibbles per 32-value group:
 * low for the first 16 values, high for the next 16), scale 2s + 1 per 16
 * (ggml's dequantizer: (d*(0.5+s))*0.25). */
static void int_iq2_s(const uint8_t *blk, kq_int *k, const uint64_t *grid) {
    k->d = orc_fp16_to_f32(rd16(blk));
    k->dmin = 0.0f;
    k->group = 16;
    const uint8_t *qs = blk + 2;
    const uint8_t *signs = blk + 34;
    const uint8_t *qh = blk + 66;
    const uint8_t *scales = blk + 74;
    for (int g = 0; g < 8; ++g) {
        k->sc[2 * g] = 1 + 2 * (scales[g] & 15);
        k->sc[2 * g + 1] = 1 + 2 * (scales[g] >> 4);
        for (int l = 0; l < 4; ++l) {
            unsigned idx = qs[4 * g + l] | ((((unsigned)qh[g]) >> (2 * l) & 3u) << 8);
            uint64_t gv = grid[idx];
            uint8_t sg = signs[4 * g + l];
            for (int j = 0; j < 8; ++j) {
                int mag = (int)((gv >> (8 * j)) & 0xffu);
                int neg = (sg >> j) & 1;
                k->neg[32 * g + 8 * l + j] = (uint8_t)neg;
                k->a[32 * g + 8 * l + j] = neg ? -mag : mag;
            }
        }
    }
}

static int block_int(int type, const uint8_t *blk, kq_int *k, const void *grid) {
    switch (type) {
    case ORC_Q4_K: int_q4_k(blk, k); return ORC_OK;
    case ORC_Q5_K: int_q5_k(blk, k); return ORC_OK;
    case ORC_Q3_K: int_q3_k(blk, k); return ORC_OK;
    case ORC_Q6_K: int_q6_k(blk, k); return ORC_OK;
    case ORC_IQ4_XS: int_iq4_xs(blk, k); return ORC_OK;
    case ORC_IQ3_S: int_iq3_s(blk, k); return ORC_OK;
    case ORC_IQ3_XXS:
        if (!grid) return ORC_ENOGRID;
        int_iq3_xxs(blk, k, (const uint32_t *)grid);
        return ORC_OK;
    case ORC_IQ2_S:
        if (!grid) return ORC_ENOGRID;
        int_iq2_s(blk, k, (const uint64_t *)grid);
        return ORC_OK;
    default: return ORC_EINVAL;
    }
}

/* f32 dequantization of one superblock, in each reference expression's
 * order:
 *   Q4_K, Q5_K  (d*sc)*a - dmin*m       (include/xdna/kquants.h:290-348)
 *   Q3_K        (d*(sc-32))*a           (include/xdna/kquants.h:350-389)
 *   Q6_K        (d*sc)*a                (include/xdna/kquants.h:391-419)
 *   IQ4_XS      (d*(ls-32))*kvalue      (include/xdna/kquants.h:421-441)
 *   IQ3_S       (d*(1+2s))*(+-mag)      (include/xdna/kquants.h:443-490)
 *   IQ3_XXS     ((d*(0.5+s))*0.5)*(+-mag)   (ggml dequantize_row_iq3_xxs)
 *   IQ2_S       ((d*(0.5+s))*0.25)*(+-mag)  (ggml dequantize_row_iq2_s)
 * For the grid types the sign is applied after the product, as the
 * references do (a zero magnitude with its sign bit set gives -0.0). */
static void dq_superblock(int type, const kq_int *k, float *y) {
    for (int g = 0; g < 256 / k->group; ++g) {
        float dl, ml = 0.0f;
        switch (type) {
        case ORC_Q4_K: case ORC_Q5_K:
            dl = k->d * (float)k->sc[g];
            ml = k->dmin * (float)k->mn[g];
            break;
        case ORC_IQ3_XXS:
            dl = k->d * (0.5f + (float)((k->sc[g] - 1) / 2)) * 0.5f;
            break;
        case ORC_IQ2_S:
            dl = k->d * (0.5f + (float)((k->sc[g] - 1) / 2)) * 0.25f;
            break;
        default:
            dl = k->d * (float)k->sc[g];
            break;
        }
        const int grid_type = type == ORC_IQ3_S || type == ORC_IQ3_XXS || type == ORC_IQ2_S;
        for (int i = 0; i < k->group; ++i) {
            const int p = g * k->group + i;
            if (type == ORC_Q4_K || type == ORC_Q5_K) {
                y[p] = dl * (float)k->a[p] - ml;
            } else if (grid_type) {
                const float v = dl * (float)(k->a[p] < 0 ? -k->a[p] : k->a[p]);
                y[p] = k->neg[p] ? -v : v;
            } else {
                y[p] = dl * (float)k->a[p];
            }
        }
    }
}

static void dq_kquant(int type, const uint8_t *row, int64_t K, float *y, const void *grid) {
    const int64_t bb = orc_block_bytes(type);
    kq_int k;
    for (int64_t b = 0; b < K / 256; ++b) {
        block_int(type, row + bb * b, &k, grid);
        dq_superblock(type, &k, y + 256 * b);
    }
}

int orc_dequant_row(int type, const uint8_t *row, int64_t K, float *out, const void *grid) {
    if (orc_row_bytes(type, K) < 0 || (K > 0 && (!row || !out))) return ORC_EINVAL;
    switch (type) {
    case ORC_Q4_0: dq_q4_0(row, K, out); return ORC_OK;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q3_K: case ORC_Q6_K: case ORC_IQ4_XS: case ORC_IQ3_S:
        dq_kquant(type, row, K, out, NULL);
        return ORC_OK;
    case ORC_IQ3_XXS: case ORC_IQ2_S:
        if (!grid) return ORC_ENOGRID;
        dq_kquant(type, row, K, out, grid);
        return ORC_OK;
    default: return ORC_EINVAL;
    }
}

/* y[r] = sequential fp32 sum of fl(w*x): the order of
 * src/xdna-q4-0-reference.cpp:169-203 and include/xdna/kquants.h:495-577. */
int orc_gemv_f32(int type, const uint8_t *W, int64_t N, int64_t K,
                 const float *x, float *y, const void *grid) {
    int64_t rb = orc_row_bytes(type, K);
    if (rb < 0 || N < 0) return ORC_EINVAL;
    if ((type == ORC_IQ3_XXS || type == ORC_IQ2_S) && !grid) return ORC_ENOGRID;
    if (N == 0) return ORC_OK;
    if (!W || !y || (K > 0 && !x)) return ORC_EINVAL;
    int failed = 0;
    /* rows are independent: threads split them, each row's sum stays sequential */
#pragma omp parallel reduction(| : failed)
    {
        float *w = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
        if (!w) {
            failed = 1;
        } else {
#pragma omp for schedule(static)
            for (int64_t r = 0; r < N; ++r) {
                orc_dequant_row(type, W + r * rb, K, w, grid);
                float s = 0.0f;
                for (int64_t c = 0; c < K; ++c) {
                    float p = w[c] * x[c];
                    s = s + p;
                }
                y[r] = s;
            }
            free(w);
        }
    }
    return failed ? ORC_EINVAL : ORC_OK;
}

int orc_gemv_bf16(int type, const uint8_t *W, int64_t N, int64_t K,
                  const uint16_t *x_bf16, float *y, const void *grid) {
    if (K < 0) return ORC_EINVAL;
    float *x = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!x) return ORC_EINVAL;
    for (int64_t c = 0; c < K; ++c) x[c] = orc_bf16_to_f32(x_bf16[c]);
    int rc = orc_gemv_f32(type, W, N, K, x, y, grid);
    free(x);
    return rc;
}

int orc_row_norms(int type, const uint8_t *W, int64_t N, int64_t K, double *norms,
                  const void *grid) {
    int64_t rb = orc_row_bytes(type, K);
    if (rb < 0 || N < 0) return ORC_EINVAL;
    if ((type == ORC_IQ3_XXS || type == ORC_IQ2_S) && !grid) return ORC_ENOGRID;
    if (N == 0) return ORC_OK;
    float *w = (float *)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!w) return ORC_EINVAL;
    for (int64_t r = 0; r < N; ++r) {
        orc_dequant_row(type, W + r * rb, K, w, grid);
        double s = 0.0;
        for (int64_t c = 0; c < K; ++c) s += (double)w[c] * (double)w[c];
        norms[r] = sqrt(s);
    }
    free(w);
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* ggml-cpu's Q4_0 x Q8_0 numerics (EXTERNAL; pinned by known answers)       */
/* ------------------------------------------------------------------------ */
/* ggml's CPU backend does not multiply Q4_0 weights by f32 activations: it
 * first quantizes the activation row to Q8_0 (quantize_row_q8_0) and then
 * takes integer block dot products (ggml_vec_dot_q4_0_q8_0).  Restated here
 * from ggml's published generic C path (llama.cpp 0ec4027a2, the pinned
 * build of README.md:64; not vendored in the reference, so not comparable
 * against ggml itself in this container):
 *   block of 32: amax = max|x|, d = amax / 127, id = d ? 1/d : 0,
 *                q_j = roundf(x_j * id), d stored as fp16 (round to even);
 *   row:         sumf += (sum_j (q4_j - 8) * q8_j) * d_w * d_x, blocks in
 *                order, low nibbles against q8[0..15], high against [16..31].
 * The reference's own engines never take this path (src/cpu-q4-gemv-engine.cpp
 * and src/xdna-gemv-engine.cpp multiply by f32 activations).  Used only to
 * measure whether f32-activation decode and ggml-cpu-numerics decode pick
 * the same tokens. */

uint16_t orc_f32_to_fp16(float f) {
    uint32_t x = f32_to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (x > 0x7f800000u ? 0x200u : 0u));
    if (x >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: rounds to inf */
    if (x < 0x38800000u) {                                     /* result subnormal (or 0) */
        if (x < 0x33000000u) return (uint16_t)sign;           /* < 2^-25: rounds to 0 */
        uint32_t e = x >> 23, m = (x & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150) = (m >> shift) * 2^-24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t r = ((x >> 23) - 112u) << 10 | ((x >> 13) & 0x3ffu);
    uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

int orc_quantize_row_q8_0(const float *x, int64_t K, uint8_t *out) {
    if (K < 0 || K % 32 != 0 || (K > 0 && (!x || !out))) return ORC_EINVAL;
    for (int64_t b = 0; b < K / 32; ++b) {
        const float *xb = x + 32 * b;
        uint8_t *ob = out + 34 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            float a = fabsf(xb[j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = orc_f32_to_fp16(d);
        ob[0] = (uint8_t)(h & 0xff);
        ob[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) ob[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
    }
    return ORC_OK;
}

int orc_gemv_q4_0_q8_0(const uint8_t *W, int64_t N, int64_t K, const float *x, float *y) {
    const int64_t rb = orc_row_bytes(ORC_Q4_0, K);
    if (rb < 0 || N < 0) return ORC_EINVAL;
    if (N == 0) return ORC_OK;
    if (!W || !y || (K > 0 && !x)) return ORC_EINVAL;
    const int64_t nb = K / 32;
    uint8_t *xq = (uint8_t *)malloc((size_t)(nb > 0 ? nb : 1) * 34);
    if (!xq) return ORC_EINVAL;
    orc_quantize_row_q8_0(x, K, xq);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < N; ++r) {
        const uint8_t *row = W + r * rb;
        float sumf = 0.0f;
        for (int64_t b = 0; b < nb; ++b) {
            const uint8_t *wb = row + 18 * b;
            const uint8_t *qb = xq + 34 * b;
            int sumi0 = 0, sumi1 = 0;
            for (int j = 0; j < 16; ++j) {
                const int v0 = (wb[2 + j] & 0x0f) - 8;
                const int v1 = (wb[2 + j] >> 4) - 8;
                sumi0 += v0 * (int)(int8_t)qb[2 + j];
                sumi1 += v1 * (int)(int8_t)qb[2 + 16 + j];
            }
            const int sumi = sumi0 + sumi1;
            const float dw = orc_fp16_to_f32((uint16_t)(wb[0] | (wb[1] << 8)));
            const float dx = orc_fp16_to_f32((uint16_t)(qb[0] | (qb[1] << 8)));
            sumf += (float)sumi * dw * dx;
        }
        y[r] = sumf;
    }
    free(xq);
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* ggml-cpu's K-quant / IQ x Q8_K numerics (EXTERNAL; pinned by known answers) */
/* ------------------------------------------------------------------------ */
/* The reference's live path for the eight 256-value types, whenever
 * ggml-cpu is loaded (src/xdna-gemv-engine.cpp:1382-1399, 1430-1453):
 * quantize_row_q8_K on the activation row, then per output row
 * ggml_vec_dot_<type>_q8_K(K, &y[r], 0, row, 0, q8, 0, 1).  Restated from
 * ggml's published generic C path (llama.cpp 0ec4027a2, the pinned build of
 * README.md:64; not vendored in the reference):
 *   Q8_K block of 256: f32 d, int8 qs[256], int16 bsums[16] (292 bytes);
 *     max = the first value of largest |x|, iscale = -127 / max,
 *     q = min(127, nearest_int(iscale * x)) (round half to even through
 *     + 1.5 * 2^23), bsums = sums of 16 codes, d = 1 / iscale; an all-zero
 *     block stores d = 0 and zero codes (and, here, zero sums).
 *   Q4_K, Q5_K, Q3_K, Q6_K: per superblock the integers
 *     aux[l] = sum over values p = l (mod 8) of scale(p) * a[p] * q8[p],
 *     then lanes[l] += (d_w * d_x) * aux[l]; Q4_K / Q5_K also
 *     sumf -= (dmin_w * d_x) * sum_j bsums[j] * min[j / 2]; at the end
 *     sumf += lanes[0..7] in order.
 *   IQ4_XS: per 32-value sub-block sumf += ((d_w * d_x) * (ls - 32)) * sumi.
 *   IQ3_S, IQ3_XXS, IQ2_S: per superblock bsum = sum over groups of
 *     scale * sum(a * q8) (scales 2s + 1), sumf += (d_w * d_x) * bsum; the
 *     result is sumf (IQ3_S), 0.25 * sumf (IQ3_XXS) or 0.125 * sumf (IQ2_S).
 * Integers as ggml's generic code forms them (their order does not matter);
 * every f32 operation in ggml's order (build with -ffp-contract=off). */

static int nearest_int_q8(float f) {
    float v = f + 12582912.0f;
    int32_t i;
    memcpy(&i, &v, sizeof i);
    return (i & 0x007fffff) - 0x00400000;
}

int orc_quantize_row_q8_K(const float *x, int64_t K, uint8_t *out) {
    if (K < 0 || K % 256 != 0 || (K > 0 && (!x || !out))) return ORC_EINVAL;
    for (int64_t b = 0; b < K / 256; ++b) {
        const float *xb = x + 256 * b;
        uint8_t *ob = out + ORC_Q8K_BYTES * b;
        int8_t *qs = (int8_t *)(ob + 4);
        int16_t bsums[16];
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        float d = 0.0f;
        if (amax == 0.0f) {
            memset(qs, 0, 256);
        } else {
            const float iscale = -127.0f / max;
            for (int j = 0; j < 256; ++j) {
                const int v = nearest_int_q8(iscale * xb[j]);
                qs[j] = (int8_t)(v < 127 ? v : 127);
            }
            d = 1.0f / iscale;
        }
        for (int j = 0; j < 16; ++j) {
            int sum = 0;
            for (int i = 0; i < 16; ++i) sum += qs[16 * j + i];
            bsums[j] = (int16_t)sum;
        }
        memcpy(ob, &d, 4);
        memcpy(ob + 260, bsums, sizeof bsums);
    }
    return ORC_OK;
}

/* One output row: ggml_vec_dot_<type>_q8_K (generic) over nb superblocks. */
static float dot_row_q8_K(int type, const uint8_t *row, int64_t nb, const uint8_t *q8, const void *grid) {
    const int64_t bb = orc_block_bytes(type);
    const int eight_lanes = type == ORC_Q4_K || type == ORC_Q5_K || type == ORC_Q3_K || type == ORC_Q6_K;
    float lanes[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    float sumf = 0.0f;
    kq_int k;
    for (int64_t i = 0; i < nb; ++i) {
        block_int(type, row + bb * i, &k, grid);
        const uint8_t *yb = q8 + ORC_Q8K_BYTES * i;
        float yd;
        memcpy(&yd, yb, 4);
        const int8_t *yq = (const int8_t *)(yb + 4);
        int16_t bsums[16];
        memcpy(bsums, yb + 260, sizeof bsums);
        if (eight_lanes) {
            int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int p = 0; p < 256; ++p) aux[p & 7] += k.sc[p / k.group] * (k.a[p] * (int)yq[p]);
            const float d = k.d * yd;
            for (int l = 0; l < 8; ++l) lanes[l] += d * (float)aux[l];
            if (type == ORC_Q4_K || type == ORC_Q5_K) {
                int sumi = 0;
                for (int j = 0; j < 16; ++j) sumi += bsums[j] * k.mn[j / 2];
                const float dmin = k.dmin * yd;
                sumf -= dmin * (float)sumi;
            }
        } else if (type == ORC_IQ4_XS) {
            const float d4d8 = k.d * yd;
            for (int ib = 0; ib < 8; ++ib) {
                int sumi = 0;
                for (int p = 32 * ib; p < 32 * ib + 32; ++p) sumi += (int)yq[p] * k.a[p];
                const float dl = d4d8 * (float)k.sc[ib];
                sumf += dl * (float)sumi;
            }
        } else {
            const float d = k.d * yd;
            int bsum = 0;
            for (int g = 0; g < 256 / k.group; ++g) {
                int sumi = 0;
                for (int p = g * k.group; p < (g + 1) * k.group; ++p) sumi += k.a[p] * (int)yq[p];
                bsum += sumi * k.sc[g];
            }
            sumf += d * (float)bsum;
        }
    }
    if (eight_lanes)
        for (int l = 0; l < 8; ++l) sumf += lanes[l];
    if (type == ORC_IQ3_XXS) return 0.25f * sumf;
    if (type == ORC_IQ2_S) return 0.125f * sumf;
    return sumf;
}

int orc_gemv_q8_K(int type, const uint8_t *W, int64_t N, int64_t K, const float *x, float *y,
                  const void *grid) {
    const int64_t rb = orc_row_bytes(type, K);
    if (rb < 0 || N < 0 || orc_block_values(type) != 256) return ORC_EINVAL;
    if ((type == ORC_IQ3_XXS || type == ORC_IQ2_S) && !grid) return ORC_ENOGRID;
    if (N == 0) return ORC_OK;
    if (!W || !y || (K > 0 && !x)) return ORC_EINVAL;
    const int64_t nb = K / 256;
    uint8_t *q8 = (uint8_t *)malloc((size_t)(nb > 0 ? nb : 1) * ORC_Q8K_BYTES);
    if (!q8) return ORC_EINVAL;
    orc_quantize_row_q8_K(x, K, q8);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < N; ++r) y[r] = dot_row_q8_K(type, W + r * rb, nb, q8, grid);
    free(q8);
    return ORC_OK;
}
