"""Known-answer cases for ggml-cpu's Q4_0 x Q8_0 arithmetic, shared by the
oracle's CPU tests and the GPU kernels' tests.

ggml's generic C path (llama.cpp 0ec4027a2, the build the reference pins in
README.md:64; ggml itself is not in this build) does, per 32-value block:
  quantize_row_q8_0_ref:  d = amax / 127, id = d ? 1/d : 0,
                          q_j = roundf(x_j * id)  -- C's roundf: halves
                          round AWAY from zero (2.5 -> 3, -2.5 -> -3), not
                          to even;
  ggml_vec_dot_q4_0_q8_0: sumf += sumi * d_w * d_x, i.e. (sumi * d_w) * d_x
                          by C's left-to-right association, blocks added to
                          sumf one after another in block order.

The expected values below are written out by hand from those three rules.
Each case is chosen so that the plausible alternative gives a different
result: rintf (half to even), sumi * (d_w * d_x), and any other block order
(reverse, pairwise, or an exact sum).

One activation row of K = 256 (8 blocks) and a weight matrix of N = 68
rows:
- rows 0..63 read single activation codes: row r has weight +1 (code 9,
  d_w = 1) at value r of the row and 0 (code 8) everywhere else, so
  y_r = q_r * d_x of its block, exactly;
  - block 0 (d_x = 1: amax 127) holds exact halves k + 0.5 for odd and
    even k of both signs;
  - block 1 (d_x = 0.5: amax 63.5, id = 2) holds values whose x * id lands
    on k + 0.5;
- row 64 sums four block terms 2^24, 1, 1, -2^24 (blocks 2..5): in order
  (2^24 + 1) rounds back to 2^24 (tie to even), so does + 1, and the row is
  0; reverse order gives 2, pairwise 1, the exact sum 2;
- row 65 is one block (block 6, d_x = 0.75) with sumi = 27562 and
  d_w = fp16(0.3): (sumi * d_w) * d_x and sumi * (d_w * d_x) differ in f32;
- rows 66, 67 are all zero codes (y = 0).
"""
from __future__ import annotations

import numpy as np

K = 256
N = 68

# block 0: d_x = 1 (amax 127, id = 1), x * id = x
B0_X = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 126.5, -126.5, 64.5, -64.5, 100.5, 101.5, -101.5,
        0.49999997, -0.49999997, 7.5, -8.5, 0.0, 1.0, -1.0, 50.0, -50.0, 10.5, -11.5, 20.25, -20.75, 33.5, 34.5, -0.0]
# the same codes under half-away-from-zero rounding, written out
B0_Q = [127, 1, -1, 2, -2, 3, -3, 4, -4, 127, -127, 65, -65, 101, 102, -102,
        0, 0, 8, -9, 0, 1, -1, 50, -50, 11, -12, 20, -21, 34, 35, 0]
# block 1: amax 63.5, d_x = 0.5, id = 2, so x * id = 2x lands on k + 0.5
B1_X = [63.5, 0.25, -0.25, 0.75, -0.75, 1.25, -1.25, 1.75, -1.75, 31.75, -31.75, 62.25, -62.75, 5.0, -5.0, 0.125,
        10.25, 10.75, -10.25, -10.75, 0.0, 40.25, -40.25, 20.75, -20.75, 3.25, 3.75, -3.25, -3.75, 63.25, -63.25, 0.5]
B1_Q = [127, 1, -1, 2, -2, 3, -3, 4, -4, 64, -64, 125, -126, 10, -10, 0,
        21, 22, -21, -22, 0, 81, -81, 42, -42, 7, 8, -7, -8, 127, -127, 1]
# blocks 2..5 (order case): d_x = 1, codes as given
ORDER_X = [127.0, 127.0, 127.0, 127.0, 4.0, 1.0] + [0.0] * 26
# block 6 (association case): amax 95.25 -> d = 0.75 exactly (fp16 exact),
# id = fl(1 / 0.75); 31 values 95.25 -> 127, the last 2.25 -> 3
ASSOC_X = [95.25] * 31 + [2.25]
ASSOC_SUMI = 31 * 7 * 127 + 1 * 3          # 27562
ASSOC_DW_BITS = 0x34CD                     # fp16(0.3) = 0.300048828125
# block 7: small integers (d_x = 1), read by no row
TAIL_X = [127.0] + [float(v) for v in range(-15, 16)]


def activation() -> np.ndarray:
    x = np.array(B0_X + B1_X + ORDER_X * 4 + ASSOC_X + TAIL_X, dtype=np.float32)
    assert x.size == K
    return x


def expected_codes() -> list[list[int]]:
    """Q8_0 codes of blocks 0 and 1 under ggml's roundf."""
    return [B0_Q, B1_Q]


def _block(d_bits: int, values) -> np.ndarray:
    """One ggml Q4_0 block: fp16 d, then 16 bytes; value j < 16 is the low
    nibble of byte j, value j >= 16 the high nibble of byte j - 16; the
    nibble is the weight + 8."""
    v = np.asarray(values, dtype=np.int32) + 8
    assert v.size == 32 and v.min() >= 0 and v.max() <= 15
    b = np.empty(18, dtype=np.uint8)
    b[0], b[1] = d_bits & 0xFF, d_bits >> 8
    b[2:] = (v[:16] | (v[16:] << 4)).astype(np.uint8)
    return b


def weights() -> np.ndarray:
    """The N x K Q4_0 matrix in ggml's byte encoding (N rows of 8 blocks)."""
    one, zero = 0x3C00, 0x0000
    zb = _block(one, [0] * 32)
    rows = []
    for r in range(64):
        v = [0] * 32
        v[r % 32] = 1
        blocks = [zb] * 8
        blocks[r // 32] = _block(one, v)
        rows.append(np.concatenate(blocks))
    # row 64: 2^24, 1, 1, -2^24 from blocks 2..5 (codes 127,127,127,127,4,1)
    big = 0x7800                                            # fp16 32768
    small = 0x2000                                          # fp16 2^-7
    plus5 = [1, 1, 1, 1, 1] + [0] * 27                      # sumi = 4 * 127 + 4 = 512
    minus5 = [-1, -1, -1, -1, -1] + [0] * 27                # -512
    pair = [1, 0, 0, 0, 0, 1] + [0] * 26                    # 127 + 1 = 128
    rows.append(np.concatenate([zb, zb, _block(big, plus5), _block(small, pair), _block(small, pair),
                                _block(big, minus5), zb, zb]))
    # row 65: sumi = 31 * 7 * 127 + 3 with d_w = fp16(0.3), d_x = 0.75
    rows.append(np.concatenate([zb] * 6 + [_block(ASSOC_DW_BITS, [7] * 31 + [1]), zb]))
    rows.append(np.concatenate([_block(zero, [0] * 32)] * 8))
    rows.append(np.concatenate([zb] * 8))
    w = np.stack(rows)
    assert w.shape == (N, 18 * K // 32)
    return w


def _f32(v) -> np.float32:
    return np.float32(v)


def expected_y() -> np.ndarray:
    y = np.zeros(N, dtype=np.float32)
    y[:32] = np.array(B0_Q, dtype=np.float32) * np.float32(1.0)
    y[32:64] = np.array(B1_Q, dtype=np.float32) * np.float32(0.5)
    y[64] = 0.0                         # ((2^24 + 1) + 1) - 2^24 in f32
    dw = np.array([ASSOC_DW_BITS], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    y[65] = _f32(_f32(_f32(ASSOC_SUMI) * dw) * _f32(0.75))
    return y


def alternatives() -> dict[str, np.ndarray]:
    """What the plausible mistakes would give for rows 0..65 (each must
    differ from expected_y somewhere): rintf codes, the other product
    association, and other block orders for row 64."""
    e = expected_y()
    rint = e.copy()
    rint[:32] = np.rint(np.array(B0_X, dtype=np.float64)).astype(np.float32)
    rint[32:64] = np.rint(2.0 * np.array(B1_X, dtype=np.float64)).astype(np.float32) * np.float32(0.5)
    dw = np.array([ASSOC_DW_BITS], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    assoc = e.copy()
    assoc[65] = _f32(_f32(ASSOC_SUMI) * _f32(dw * _f32(0.75)))
    big, one = _f32(2.0 ** 24), _f32(1.0)
    rev = e.copy()
    rev[64] = _f32(_f32(_f32(-big + one) + one) + big)
    pairwise = e.copy()
    pairwise[64] = _f32(_f32(big + one) + _f32(one - big))
    return {"rintf": rint, "sumi*(dw*dx)": assoc, "reverse order": rev, "pairwise": pairwise}
