/*
 * CPU oracle for the quantized decode GEMV path -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's scalar numerics, used by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the
 * checker.  The shipped library (xdna.cpp_amd/) never links, loads or calls
 * anything in this directory.
 *
 * Weight type ids are ggml's GGUF type ids (stable on-disk values).
 *
 * Numerics contract followed here (bit-for-bit, compile with
 * -ffp-contract=off):
 *   y[r] = sequential fp32 sum over c of fl(w[r][c] * x[c]),
 * with w[r][c] the dequantized weight, computed by the per-type expression
 * order of the reference:
 *   Q4_0      src/xdna-q4-0-reference.cpp:169-203 (dot_unchecked), 302-328
 *   Q4_K      include/xdna/kquants.h:290-315, 495-507
 *   Q5_K      include/xdna/kquants.h:317-348, 509-521
 *   Q3_K      include/xdna/kquants.h:350-389, 523-535
 *   Q6_K      include/xdna/kquants.h:391-419, 537-549
 *   IQ4_XS    include/xdna/kquants.h:421-441, 551-563
 *   IQ3_S     include/xdna/kquants.h:443-490, 565-577
 *   IQ3_XXS   ggml dequantize_row_iq3_xxs (external, llama.cpp 0ec4027a2;
 *             called by the reference only through ggml_vec_dot_iq3_xxs_q8_K,
 *             src/xdna-gemv-engine.cpp:1395)
 *   IQ2_S     ggml dequantize_row_iq2_s (external, same pin; reference call
 *             site src/xdna-gemv-engine.cpp:1396)
 * IQ3_XXS / IQ2_S grids are not in the reference; callers pass them in.  The
 * reference holds no vectors for these two decoders, so they are pinned by
 * encoders written from ggml's quantizer packing (the inverse direction, round
 * trip through the decoder), known answers for every sign index and its parity
 * bit, every IQ2_S sign bit, the scale nibbles, the index high bits and the
 * scale factors, and probe blocks that read a grid back
 * (tests/test_oracle_cpu.py, test_iq3_xxs_* and test_iq2_s_*).
 */
#ifndef XDNA_ORACLE_H
#define XDNA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_Q4_0 = 2,
    ORC_Q3_K = 11,
    ORC_Q4_K = 12,
    ORC_Q5_K = 13,
    ORC_Q6_K = 14,
    ORC_IQ3_XXS = 18,
    ORC_IQ3_S = 21,
    ORC_IQ2_S = 22,
    ORC_IQ4_XS = 23,
};

/* status codes */
enum {
    ORC_OK = 0,
    ORC_EINVAL = -1,     /* bad shape / size / type */
    ORC_ENOGRID = -2,    /* IQ3_XXS / IQ2_S requested without a grid */
};

/* Exact IEEE half -> float (src/xdna-q4-0-reference.cpp:207-242). */
float orc_fp16_to_f32(uint16_t bits);
/* BF16 <-> float (src/xdna-q4-0-reference.cpp:244-259): RNE rounding. */
float orc_bf16_to_f32(uint16_t bits);
uint16_t orc_f32_to_bf16(float value);

/* Values per block (32 or 256) and bytes per block; 0 for unknown types. */
int64_t orc_block_values(int type);
int64_t orc_block_bytes(int type);
/* Bytes of one row of K values, or -1 if K is not a multiple of the block. */
int64_t orc_row_bytes(int type, int64_t K);

/* Q4_0 validation helpers with the reference's rules
 * (src/xdna-q4-0-reference.cpp:261-300); 0 on success, ORC_EINVAL otherwise. */
int orc_q4_0_validate_row(uint64_t value_count, uint64_t encoded_bytes);
int orc_q4_0_validate_matrix(uint64_t rows, uint64_t values_per_row,
                             uint64_t encoded_bytes);

/* Dequantize one row of K values.  grid: IQ3_XXS -> uint32[256],
 * IQ2_S -> uint64[1024]; ignored (may be NULL) for other types. */
int orc_dequant_row(int type, const uint8_t *row, int64_t K, float *out,
                    const void *grid);

/* GEMV, f32 activations.  W is N contiguous rows of orc_row_bytes(type,K). */
int orc_gemv_f32(int type, const uint8_t *W, int64_t N, int64_t K,
                 const float *x, float *y, const void *grid);

/* GEMV, BF16 activations (raw bits), converted exactly to f32 first
 * (src/xdna-q4-0-reference.cpp:382-406). */
int orc_gemv_bf16(int type, const uint8_t *W, int64_t N, int64_t K,
                  const uint16_t *x_bf16, float *y, const void *grid);

/* Euclidean norm of every dequantized row (double accumulation), used for
 * the per-row error bound |y - y_ref| <= 1e-4 * ||w_r|| * ||x||. */
int orc_row_norms(int type, const uint8_t *W, int64_t N, int64_t K, double *norms,
                  const void *grid);

/* IQ2 sign table: 7 sign bits plus an even-parity 8th bit (ggml
 * ksigns_iq2xs, external).  Returns the byte for index i in [0,128). */
uint8_t orc_ksigns_iq2xs(int i);

/* ggml-cpu's Q4_0 x Q8_0 path (external restatement, see oracle.c; pinned by
 * the Q8_0 quantizer's invariants and hand-written known answers for its
 * tie rounding, product association and block order, tests/ggml_q8_cases.py):
 * f32 -> fp16 round to even, Q8_0 quantization of an activation row (K/32
 * blocks of [fp16 d][int8 q[32]]), and the Q4_0 x Q8_0 GEMV. */
uint16_t orc_f32_to_fp16(float f);
int orc_quantize_row_q8_0(const float *x, int64_t K, uint8_t *out);
int orc_gemv_q4_0_q8_0(const uint8_t *W, int64_t N, int64_t K, const float *x, float *y);

/* ggml-cpu's K-quant / IQ x Q8_K path (external restatement, see oracle.c;
 * pinned by the Q8_K quantizer's invariants, known answers and the float64 dot
 * of the dequantized operands, tests/test_oracle_cpu.py test_q8_K_* and
 * test_gemv_q8_K_*): Q8_K quantization of an activation row (K/256
 * blocks of [f32 d][int8 q[256]][int16 bsums[16]]) and the GEMV of any of
 * the eight 256-value types against it. */
#define ORC_Q8K_BYTES 292
int orc_quantize_row_q8_K(const float *x, int64_t K, uint8_t *out);
int orc_gemv_q8_K(int type, const uint8_t *W, int64_t N, int64_t K, const float *x, float *y,
                  const void *grid);

#ifdef __cplusplus
}
#endif

#endif
