"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Four independent sources:
  1. golden vectors written by the reference's own compiled code
     (tests/golden/ref_vectors.npz, made by tests/golden/make_golden.py);
  2. the compiled reference itself (oracle/_ref), on fresh random inputs,
     when it is built in this checkout;
  3. the known answers the reference's tests hold
     (tests/test-q4-0-reference.cpp:49-54,128-143,157-210,
      tests/test-backend.cpp:58-98, tests/test-gemv-accuracy.cpp:128-153,184-217,
      tests/test-kquants-gemv.cpp:258-270);
  4. closed forms: exhaustive fp16/bf16 conversion against numpy, and each
     K/IQ format's decode against an independent *encoder* written from ggml's
     quantizer packing (the inverse direction), so a wrong shift, index or
     nibble order in the oracle's decoder fails.
IQ3_XXS / IQ2_S have no reference code, vectors or tests: their layouts are
pinned by encoders from ggml's quantizer packing and known answers for every
sign bit, parity bit, scale nibble and scale factor, on synthetic grids (the
grid contents themselves stay ggml's).
"""
import hashlib
import os

import numpy as np
import pytest

from oracle import (IQ2_S, IQ3_S, IQ3_XXS, IQ4_XS, Q3_K, Q4_0, Q4_K, Q5_K, Q6_K, TYPE_NAMES, RefLib)
import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")
REF_TYPES = (Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS, IQ3_S)


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def half(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


# ---- 1. golden vectors from the reference build -----------------------------

@pytest.mark.parametrize("t", REF_TYPES, ids=[TYPE_NAMES[t] for t in REF_TYPES])
def test_golden_vectors_bit_exact(oracle, golden, t):
    name = TYPE_NAMES[t]
    i = 0
    while f"{name}_{i}_W" in golden:
        k = f"{name}_{i}"
        N, K = (int(v) for v in golden[k + "_shape"])
        W, x = golden[k + "_W"], golden[k + "_x"]
        y = oracle.gemv(t, W, N, K, x)
        assert np.array_equal(bits(y), bits(golden[k + "_y"])), k
        d0 = oracle.dequant_row(t, W.reshape(N, -1)[0], K)
        assert np.array_equal(bits(d0), bits(golden[k + "_deq0"])), k
        if t == Q4_0:
            yb = oracle.gemv(t, W, N, K, golden[k + "_xbf16"])
            assert np.array_equal(bits(yb), bits(golden[k + "_ybf16"])), k
        i += 1
    assert i >= 1


def test_golden_validation_rules(oracle, golden):
    # src/xdna-q4-0-reference.cpp:261-300: same accept/reject decisions
    for (v, b), rc in zip(golden["validate_row_cases"], golden["validate_row_rc"]):
        assert (oracle.lib.orc_q4_0_validate_row(int(v), int(b)) == 0) == (rc == 0), (v, b)
    for (r, v, b), rc in zip(golden["validate_matrix_cases"], golden["validate_matrix_rc"]):
        assert (oracle.lib.orc_q4_0_validate_matrix(int(r), int(v), int(b)) == 0) == (rc == 0), (r, v, b)


def test_golden_bf16_rounding(oracle, golden):
    got = np.array([oracle.f32_to_bf16(float(v)) for v in golden["bf16_in"]], dtype=np.uint16)
    assert np.array_equal(got, golden["bf16_out"])


def test_golden_iq3s_grid_hash(oracle, golden):
    grid = extract_iq3s_grid(oracle)
    h = hashlib.sha256(grid.astype("<u4").tobytes()).digest()
    assert h == golden["iq3s_grid_sha256"].tobytes()


# ---- 2. the compiled reference on fresh inputs ------------------------------

@pytest.mark.parametrize("t", REF_TYPES, ids=[TYPE_NAMES[t] for t in REF_TYPES])
def test_oracle_matches_reference_build(oracle, reflib, t):
    rng = np.random.default_rng(t)
    for trial in range(6):
        bv = 32 if t == Q4_0 else 256
        N = int(rng.integers(1, 9))
        K = bv * int(rng.integers(1, 7))
        if t == Q4_0:
            W = synth.random_q4_0(N, K, seed=trial)
        else:
            d = int(rng.choice([0x2E66, 0x3C00, 0x1400, 0xB800]))
            W = synth.random_blocks(t, N, K, seed=trial, d_bits=d, dmin_bits=int(rng.choice([0x2A00, 0x0000, 0xB000])))
        x = (rng.standard_normal(K) * rng.choice([1e-3, 1.0, 100.0])).astype(np.float32)
        assert np.array_equal(bits(oracle.gemv(t, W, N, K, x)), bits(reflib.gemv(t, W, N, K, x))), (trial, N, K)
        for r in range(N):
            row = W.reshape(N, -1)[r]
            assert np.array_equal(bits(oracle.dequant_row(t, row, K)), bits(reflib.dequant_row(t, row, K)))


def test_oracle_matches_reference_build_bf16(oracle, reflib):
    W = synth.random_q4_0(16, 512, seed=3)
    xb = np.random.default_rng(5).integers(0, 1 << 16, 512).astype(np.uint16)
    xb[(xb & 0x7F80) == 0x7F80] = 0x3F80  # no inf/NaN activations
    assert np.array_equal(bits(oracle.gemv(Q4_0, W, 16, 512, xb)), bits(reflib.gemv(Q4_0, W, 16, 512, xb)))


def test_iq3s_grid_matches_reference_build(oracle, reflib):
    assert np.array_equal(extract_iq3s_grid(oracle), reflib.iq3s_grid())


# ---- 3. the reference tests' known answers ----------------------------------

EDGE = np.array([0x00, 0x3c, 0xf0, 0xe1, 0xd2, 0xc3, 0xb4, 0xa5, 0x96,
                 0x87, 0x78, 0x69, 0x5a, 0x4b, 0x3c, 0x2d, 0x1e, 0x0f], dtype=np.uint8)


def test_q4_0_edge_block_order_and_dot(oracle):
    # tests/test-q4-0-reference.cpp:49-54,157-191
    d = oracle.dequant_row(Q4_0, EDGE, 32)
    assert d[:16].tolist() == [j - 8.0 for j in range(16)]
    assert d[16:].tolist() == [7.0 - j for j in range(16)]
    x = np.arange(1, 33, dtype=np.float32)
    assert oracle.gemv(Q4_0, EDGE, 1, 32, x).tolist() == [-264.0]
    xb = np.array([oracle.f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    assert oracle.gemv(Q4_0, EDGE, 1, 32, xb).tolist() == [-264.0]


def test_q4_0_two_row_gemv(oracle):
    # tests/test-q4-0-reference.cpp:128-143,193-210: 528 and -264
    W = np.zeros(36, dtype=np.uint8)
    W[0:2], W[2:18] = [0x00, 0x3c], 0x99
    W[18:20], W[20:36] = [0x00, 0x38], 0x77
    x = np.arange(1, 33, dtype=np.float32)
    assert oracle.gemv(Q4_0, W, 2, 32, x).tolist() == [528.0, -264.0]
    xb = np.array([oracle.f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    assert oracle.gemv(Q4_0, W, 2, 32, xb).tolist() == [528.0, -264.0]


def test_q4_0_uniform_weights(oracle):
    # tests/test-backend.cpp:58-98 (d=1, +1 codes, x=0.5, K=256 -> 128) and
    # tests/test-gemv-accuracy.cpp:128-153 (d=0.5, x=0.25, K=256 -> 32)
    for d, xv, want in ((0x3C00, 0.5, 128.0), (0x3800, 0.25, 32.0)):
        blk = np.array([d & 0xFF, d >> 8] + [0x99] * 16, dtype=np.uint8)
        W = np.tile(blk, 128 * 8)
        y = oracle.gemv(Q4_0, W, 128, 256, np.full(256, xv, np.float32))
        assert np.all(y == want)


@pytest.mark.parametrize("t", REF_TYPES, ids=[TYPE_NAMES[t] for t in REF_TYPES])
def test_zero_activations_give_exact_zero(oracle, t):
    # tests/test-gemv-accuracy.cpp:184-217, tests/test-kquants-gemv.cpp:258-270
    K = 512
    W = synth.random_q4_0(64, K, 505) if t == Q4_0 else synth.random_blocks(t, 64, K, 505)
    y = oracle.gemv(t, W, 64, K, np.zeros(K, np.float32))
    assert np.all(y == 0.0)


def test_fp16_known_values(oracle):
    # tests/test-q4-0-reference.cpp:163-172
    assert oracle.fp16_to_f32(0x3c00) == 1.0
    assert oracle.fp16_to_f32(0xc000) == -2.0
    assert oracle.fp16_to_f32(0x0001) == 2.0 ** -24
    assert oracle.fp16_to_f32(0x7bff) == 65504.0
    assert oracle.bf16_to_f32(0x3f80) == 1.0
    assert oracle.bf16_to_f32(0xc000) == -2.0


def test_q4_0_validation_messages_cases(oracle):
    # tests/test-q4-0-reference.cpp:212-222 and the row/matrix spans
    assert oracle.lib.orc_q4_0_validate_row(31, 18) != 0
    assert oracle.lib.orc_q4_0_validate_row(32, 17) != 0
    assert oracle.lib.orc_q4_0_validate_row(32, 19) != 0
    assert oracle.lib.orc_q4_0_validate_row(32, 18) == 0
    assert oracle.lib.orc_q4_0_validate_row(0, 0) == 0
    assert oracle.lib.orc_q4_0_validate_matrix(2, 32, 36) == 0
    assert oracle.row_bytes(Q4_0, 32) == 18 and oracle.row_bytes(Q4_0, 0) == 0


# ---- 4. closed forms ----------------------------------------------------------

def test_fp16_exhaustive(oracle):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_bf16_widen_exhaustive_and_round_to_nearest_even(oracle):
    b = np.arange(1 << 16, dtype=np.uint32)
    want = (b << 16).view(np.float32)
    got = np.array([oracle.bf16_to_f32(int(v)) for v in b], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan])) and np.isnan(got[nan]).all()
    # f32 -> bf16 is round-to-nearest-even on the dropped 16 bits
    for u, r in ((0x3F808000, 0x3F80), (0x3F818000, 0x3F82), (0x3F808001, 0x3F81), (0x3F807FFF, 0x3F80),
                 (0xBF808000, 0xBF80)):
        assert oracle.f32_to_bf16(float(np.uint32(u).view(np.float32))) == r


def test_block_geometry(oracle):
    # include/xdna/kquants.h:182-200 and the ggml structs
    want = {Q4_0: (32, 18), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
            IQ3_XXS: (256, 98), IQ3_S: (256, 110), IQ2_S: (256, 82), IQ4_XS: (256, 136)}
    for t, (bv, bb) in want.items():
        assert oracle.block_values(t) == bv and oracle.block_bytes(t) == bb
        assert oracle.row_bytes(t, 3 * bv) == 3 * bb
        assert oracle.row_bytes(t, bv + 1) < 0


# Independent encoders, from ggml's quantizer packing (ggml-quants.c,
# quantize_row_*_ref): logical codes/scales in, block bytes out.

def pack_k4_scales(ls, lm):
    """Q4_K / Q5_K: eight 6-bit (scale, min) pairs into 12 bytes."""
    s = np.zeros(12, dtype=np.uint8)
    for j in range(8):
        if j < 4:
            s[j] = ls[j]
            s[j + 4] = lm[j]
        else:
            s[j + 4] = (ls[j] & 0xF) | ((lm[j] & 0xF) << 4)
            s[j - 4] |= (ls[j] >> 4) << 6
            s[j] |= (lm[j] >> 4) << 6
    return s


def enc_q4_k(d, dmin, ls, lm, L):
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2], blk[2:4] = half(d), half(dmin)
    blk[4:16] = pack_k4_scales(ls, lm)
    q = blk[16:]
    for j in range(0, 256, 64):
        for l in range(32):
            q[j // 2 + l] = L[j + l] | (L[j + l + 32] << 4)
    return blk


def enc_q5_k(d, dmin, ls, lm, L):
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2], blk[2:4] = half(d), half(dmin)
    blk[4:16] = pack_k4_scales(ls, lm)
    qh, ql = blk[16:48], blk[48:]
    m1, m2 = 1, 2
    for n in range(0, 256, 64):
        for j in range(32):
            l1, l2 = int(L[n + j]), int(L[n + j + 32])
            if l1 > 15:
                l1 -= 16
                qh[j] |= m1
            if l2 > 15:
                l2 -= 16
                qh[j] |= m2
            ql[n // 2 + j] = l1 | (l2 << 4)
        m1 <<= 2
        m2 <<= 2
    return blk


def enc_q3_k(d, Ls, L):
    """Ls: sixteen 6-bit scales (value + 32); L: 256 codes in 0..7 (value + 4)."""
    blk = np.zeros(110, dtype=np.uint8)
    hm, q, sc = blk[0:32], blk[32:96], blk[96:108]
    for j in range(16):
        lv = int(Ls[j])
        if j < 8:
            sc[j] = lv & 0xF
        else:
            sc[j - 8] |= (lv & 0xF) << 4
        sc[j % 4 + 8] |= (lv >> 4) << (2 * (j // 4))
    L = np.array(L, dtype=np.int64)
    m, bit = 0, 1
    for j in range(256):
        if L[j] > 3:
            hm[m] |= bit
            L[j] -= 4
        m += 1
        if m == 32:
            m, bit = 0, bit << 1
    for j in range(0, 256, 128):
        for l in range(32):
            q[j // 4 + l] = L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6)
    blk[108:110] = half(d)
    return blk


def enc_q6_k(d, sc, L):
    """sc: sixteen int8 scales; L: 256 codes in 0..63 (value + 32)."""
    blk = np.zeros(210, dtype=np.uint8)
    ql, qh = blk[0:128], blk[128:192]
    for j in range(0, 256, 128):
        for l in range(32):
            a, b, c, e = (int(L[j + l + 32 * i]) for i in range(4))
            ql[j // 2 + l] = (a & 0xF) | ((c & 0xF) << 4)
            ql[j // 2 + l + 32] = (b & 0xF) | ((e & 0xF) << 4)
            qh[j // 4 + l] = (a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6)
    blk[192:208] = np.array(sc, dtype=np.int8).view(np.uint8)
    blk[208:210] = half(d)
    return blk


def enc_iq4_xs(d, ls, L):
    """ls: eight 6-bit scales (value + 32); L: 256 codebook indices 0..15."""
    blk = np.zeros(136, dtype=np.uint8)
    blk[0:2] = half(d)
    sh = 0
    for ib in range(8):
        sh |= (int(ls[ib]) >> 4) << (2 * ib)
        blk[4 + ib // 2] |= (int(ls[ib]) & 0xF) << (4 * (ib % 2))
        for j in range(16):
            blk[8 + 16 * ib + j] = L[32 * ib + j] | (L[32 * ib + j + 16] << 4)
    blk[2:4] = np.array([sh], dtype=np.uint16).view(np.uint8)
    return blk


KVALUES_IQ4NL = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def f32(v):
    return np.float32(v)


@pytest.mark.parametrize("seed", range(4))
def test_q4_k_and_q5_k_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(seed)
    ls, lm = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    d, dmin = f32(0.03125), f32(0.0078125)  # exact in fp16
    for t, top in ((Q4_K, 16), (Q5_K, 32)):
        L = rng.integers(0, top, 256)
        blk = (enc_q4_k if t == Q4_K else enc_q5_k)(d, dmin, ls, lm, L)
        got = oracle.dequant_row(t, blk, 256)
        sub = np.arange(256) // 32
        want = (d * ls[sub].astype(np.float32)) * L.astype(np.float32) - dmin * lm[sub].astype(np.float32)
        assert np.array_equal(bits(got), bits(want.astype(np.float32))), TYPE_NAMES[t]


@pytest.mark.parametrize("seed", range(4))
def test_q3_k_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(seed)
    Ls, L = rng.integers(0, 64, 16), rng.integers(0, 8, 256)
    d = f32(0.25)
    got = oracle.dequant_row(Q3_K, enc_q3_k(d, Ls, L), 256)
    want = (d * (Ls[np.arange(256) // 16] - 32).astype(np.float32)) * (L - 4).astype(np.float32)
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))


@pytest.mark.parametrize("seed", range(4))
def test_q6_k_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(seed)
    sc, L = rng.integers(-128, 128, 16), rng.integers(0, 64, 256)
    d = f32(0.0625)
    got = oracle.dequant_row(Q6_K, enc_q6_k(d, sc, L), 256)
    want = (d * sc[np.arange(256) // 16].astype(np.float32)) * (L - 32).astype(np.float32)
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))


@pytest.mark.parametrize("seed", range(4))
def test_iq4_xs_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(seed)
    ls, L = rng.integers(0, 64, 8), rng.integers(0, 16, 256)
    d = f32(0.5)
    got = oracle.dequant_row(IQ4_XS, enc_iq4_xs(d, ls, L), 256)
    kv = np.array(KVALUES_IQ4NL, dtype=np.float32)
    want = (d * (ls[np.arange(256) // 32] - 32).astype(np.float32)) * kv[L]
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))


def extract_iq3s_grid(oracle):
    """Read the oracle's iq3s_grid back through its decoder: d = 1, scale
    nibble 0 (db = 1), no sign bits; lookup k of group g of block b holds
    index 64b + 8g + k (bit 8 from qh)."""
    grid = np.zeros(512, dtype=np.uint32)
    for b in range(8):
        blk = np.zeros(110, dtype=np.uint8)
        blk[0:2] = half(1.0)
        for g in range(8):
            for k in range(8):
                idx = 64 * b + 8 * g + k
                blk[2 + 8 * g + k] = idx & 0xFF
                blk[66 + g] |= ((idx >> 8) & 1) << k
        v = oracle.dequant_row(IQ3_S, blk, 256).astype(np.int64)
        assert np.all((v >= 0) & (v < 256))
        grid[64 * b:64 * (b + 1)] = (v.reshape(64, 4) << np.array([0, 8, 16, 24])).sum(axis=1)
    return grid


def test_iq3_s_signs_and_scales(oracle):
    # sign bit (4*(k&1)+j) of byte 4g + k/2 negates value j of lookup k;
    # scale nibble s gives db = d * (1 + 2s)
    rng = np.random.default_rng(1)
    blk = synth.random_blocks(IQ3_S, 1, 256, 9, d_bits=0x3C00)[0]
    base = blk.copy()
    base[74:106] = 0
    base[106:110] = 0
    mag = oracle.dequant_row(IQ3_S, base, 256)
    assert np.all(mag >= 0)
    signed = base.copy()
    signed[74:106] = rng.integers(0, 256, 32, dtype=np.uint8)
    s = np.unpackbits(signed[74:106], bitorder="little").astype(bool)
    assert np.array_equal(oracle.dequant_row(IQ3_S, signed, 256), np.where(s, -mag, mag))
    scaled = base.copy()
    scaled[106:110] = [0x21, 0x43, 0x65, 0x87]  # groups 0..7 -> nibbles 1..8
    nib = np.repeat(np.arange(1, 9), 32).astype(np.float32)
    assert np.array_equal(oracle.dequant_row(IQ3_S, scaled, 256), mag * (np.float32(1) + np.float32(2) * nib))


def test_ksigns_table_structure(oracle):
    k = oracle.ksigns()
    assert np.array_equal(k & 0x7F, np.arange(128))
    assert all(bin(int(v)).count("1") % 2 == 0 for v in k)


# ---- IQ3_XXS / IQ2_S ------------------------------------------------------------
# The reference reaches these two types only through ggml
# (src/xdna-gemv-engine.cpp:1395-1396), so their block layouts are pinned here
# from ggml's published quantizer packing (quantize_row_iq3_xxs_impl,
# quantize_row_iq2_s_impl of ggml-quants.c, llama.cpp 0ec4027a2): an encoder
# written in that direction must round-trip through the oracle's decoder, and
# known answers fix every sign bit, the parity bit, the scale nibbles and the
# scale factors.  The grid *contents* are ggml's and absent here; these tests
# use synthetic grids (the library checks the real ones against the host's
# ggml at run time).

def synthetic_grid(t, seed=0):
    rng = np.random.default_rng(seed)
    n, w = (256, 4) if t == IQ3_XXS else (1024, 8)
    g = rng.integers(0, 64, (n, w)).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


def test_iq_grid_types_require_a_grid(oracle):
    row = np.zeros(98, dtype=np.uint8)
    with pytest.raises(ValueError):
        oracle.dequant_row(IQ3_XXS, row, 256)
    with pytest.raises(ValueError):
        oracle.dequant_row(IQ2_S, np.zeros(82, dtype=np.uint8), 256)


def test_iq3_xxs_probe_reads_back_the_grid(oracle):
    grid = synthetic_grid(IQ3_XXS)
    for b in range(4):
        blk = np.zeros(98, dtype=np.uint8)
        blk[0:2] = half(1.0)
        blk[2:66] = np.arange(64 * b, 64 * (b + 1)) & 0xFF
        v = oracle.dequant_row(IQ3_XXS, blk, 256, grid=grid) * 4  # db = 0.25
        want = grid[64 * b:64 * (b + 1)].view(np.uint8).astype(np.float32)
        assert np.array_equal(v, want)


def test_iq2_s_probe_reads_back_the_grid(oracle):
    grid = synthetic_grid(IQ2_S)
    for b in range(32):
        blk = np.zeros(82, dtype=np.uint8)
        blk[0:2] = half(1.0)
        for g in range(8):
            for l in range(4):
                idx = 32 * b + 4 * g + l
                blk[2 + 4 * g + l] = idx & 0xFF
                blk[66 + g] |= ((idx >> 8) & 3) << (2 * l)
        v = oracle.dequant_row(IQ2_S, blk, 256, grid=grid) * 8  # db = 0.125
        want = grid[32 * b:32 * (b + 1)].view(np.uint8).astype(np.float32)
        assert np.array_equal(v, want)


def sign8(idx7):
    """Full 8-bit sign pattern of a 7-bit IQ3_XXS sign index: ggml's
    quantizer makes the number of negative values in a group of 8 even and
    stores the low 7 bits, so bit 7 is the parity of the other seven."""
    return idx7 | ((bin(idx7).count("1") & 1) << 7)


def enc_iq3_xxs(d, gidx, signs7, ls):
    """ggml's IQ3_XXS packing: gidx[8][8] grid indices (q3[8*ib + k]),
    signs7[8][4] 7-bit sign indices and ls[8] 4-bit scales per 32-value
    sub-block; scales_and_signs[ib] = s0 | s1 << 7 | s2 << 14 | s3 << 21 |
    ls << 28 (little-endian u32 after the 64 index bytes)."""
    blk = np.zeros(98, dtype=np.uint8)
    blk[0:2] = half(d)
    for ib in range(8):
        for k in range(8):
            blk[2 + 8 * ib + k] = gidx[ib][k]
        w = 0
        for l in range(4):
            w |= int(signs7[ib][l]) << (7 * l)
        w |= int(ls[ib]) << 28
        blk[66 + 4 * ib:70 + 4 * ib] = np.array([w], dtype=np.uint32).view(np.uint8)
    return blk


def want_iq3_xxs(d, gidx, signs7, ls, grid):
    """Values of a block built by enc_iq3_xxs: ggml's dequantize_row_iq3_xxs
    formula db = d * (0.5 + ls) * 0.5 on magnitude bytes of the grid entry,
    value 8l + j of sub-block ib negated where bit j of sign8(signs7[ib][l])
    is set; lookups 2l and 2l + 1 give values 8l..8l+3 and 8l+4..8l+7."""
    mags = grid.view(np.uint8).reshape(256, 4)
    out = np.zeros(256, dtype=np.float32)
    for ib in range(8):
        db = np.float32(d) * (np.float32(0.5) + np.float32(ls[ib])) * np.float32(0.5)
        for l in range(4):
            sg = sign8(int(signs7[ib][l]))
            for j in range(8):
                m = np.float32(mags[gidx[ib][2 * l + j // 4]][j % 4])
                v = db * m
                out[32 * ib + 8 * l + j] = -v if (sg >> j) & 1 else v
    return out


@pytest.mark.parametrize("seed", range(6))
def test_iq3_xxs_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    grid = synthetic_grid(IQ3_XXS, seed)
    gidx = rng.integers(0, 256, (8, 8))
    signs7 = rng.integers(0, 128, (8, 4))
    ls = rng.integers(0, 16, 8)
    d = f32(0.0625)
    got = oracle.dequant_row(IQ3_XXS, enc_iq3_xxs(d, gidx, signs7, ls), 256, grid=grid)
    assert np.array_equal(bits(got), bits(want_iq3_xxs(d, gidx, signs7, ls, grid)))


def test_iq3_xxs_every_sign_index_and_parity_bit(oracle):
    """All 128 sign indices in every one of the 32 groups of 8: value j of the
    group is negative exactly where bit j of idx | parity << 7 is set."""
    grid = np.full(256, 0x01010101, dtype=np.uint32)  # every magnitude 1
    gidx = np.zeros((8, 8), dtype=np.int64)
    ls = np.zeros(8, dtype=np.int64)  # db = 0.25 at d = 1
    for idx in range(128):
        for l in range(4):
            signs7 = np.zeros((8, 4), dtype=np.int64)
            signs7[:, l] = idx
            v = oracle.dequant_row(IQ3_XXS, enc_iq3_xxs(f32(1.0), gidx, signs7, ls), 256, grid=grid)
            want = np.full(256, 0.25, dtype=np.float32)
            for ib in range(8):
                for j in range(8):
                    if (sign8(idx) >> j) & 1:
                        want[32 * ib + 8 * l + j] = -0.25
            assert np.array_equal(v, want), (idx, l)


def test_iq3_xxs_scale_factor_known_answers(oracle):
    """db = d * (0.5 + s) * 0.5 for s = 0..15 (0.25, 0.75, ..., 7.75 at d = 1
    and magnitude 1), one scale per 32-value sub-block, from bits 28-31."""
    grid = np.full(256, 0x01010101, dtype=np.uint32)
    gidx = np.zeros((8, 8), dtype=np.int64)
    signs7 = np.zeros((8, 4), dtype=np.int64)
    for lo in (0, 8):
        ls = np.arange(lo, lo + 8)
        v = oracle.dequant_row(IQ3_XXS, enc_iq3_xxs(f32(1.0), gidx, signs7, ls), 256, grid=grid)
        assert np.array_equal(v, np.repeat(0.25 + 0.5 * ls, 32).astype(np.float32))
    # d scales everything: d = 2^-3 -> 1/8 of the values above (exact)
    v = oracle.dequant_row(IQ3_XXS, enc_iq3_xxs(f32(0.125), gidx, signs7, np.full(8, 15)), 256, grid=grid)
    assert np.array_equal(v, np.full(256, 7.75 / 8, dtype=np.float32))


def enc_iq2_s(d, gidx, signs, l1, l2):
    """ggml's IQ2_S packing: per group of 8 values i8 = 0..31, qs[i8] = grid
    index & 255, qh[i8 / 4] |= (index >> 8) << 2 * (i8 % 4), signs at
    qs[32 + i8] (8 free bits); scales[ib] = l1 | l2 << 4 (l1 for the first 16
    values of 32-value sub-block ib, l2 for the next 16)."""
    blk = np.zeros(82, dtype=np.uint8)
    blk[0:2] = half(d)
    for i8 in range(32):
        g = int(gidx[i8])
        blk[2 + i8] = g & 0xFF
        blk[66 + i8 // 4] |= (g >> 8) << (2 * (i8 % 4))
        blk[34 + i8] = signs[i8]
    for ib in range(8):
        blk[74 + ib] = int(l1[ib]) | (int(l2[ib]) << 4)
    return blk


def want_iq2_s(d, gidx, signs, l1, l2, grid):
    mags = grid.view(np.uint8).reshape(1024, 8)
    out = np.zeros(256, dtype=np.float32)
    for i8 in range(32):
        ib, half16 = i8 // 4, (i8 % 4) // 2
        s = (l1 if half16 == 0 else l2)[ib]
        db = np.float32(d) * (np.float32(0.5) + np.float32(s)) * np.float32(0.25)
        for j in range(8):
            v = db * np.float32(mags[gidx[i8]][j])
            out[8 * i8 + j] = -v if (int(signs[i8]) >> j) & 1 else v
    return out


@pytest.mark.parametrize("seed", range(6))
def test_iq2_s_decode_inverts_ggml_packing(oracle, seed):
    rng = np.random.default_rng(200 + seed)
    grid = synthetic_grid(IQ2_S, seed)
    gidx = rng.integers(0, 1024, 32)
    signs = rng.integers(0, 256, 32)
    l1, l2 = rng.integers(0, 16, 8), rng.integers(0, 16, 8)
    d = f32(0.5)
    got = oracle.dequant_row(IQ2_S, enc_iq2_s(d, gidx, signs, l1, l2), 256, grid=grid)
    assert np.array_equal(bits(got), bits(want_iq2_s(d, gidx, signs, l1, l2, grid)))


def test_iq2_s_every_sign_bit(oracle):
    grid = np.full(1024, 0x0101010101010101, dtype=np.uint64)
    z = np.zeros(32, dtype=np.int64)
    zs = np.zeros(8, dtype=np.int64)
    for i8 in range(32):
        for j in range(8):
            signs = np.zeros(32, dtype=np.int64)
            signs[i8] = 1 << j
            v = oracle.dequant_row(IQ2_S, enc_iq2_s(f32(1.0), z, signs, zs, zs), 256, grid=grid)
            want = np.full(256, 0.125, dtype=np.float32)
            want[8 * i8 + j] = -0.125
            assert np.array_equal(v, want), (i8, j)


def test_iq2_s_scale_nibbles_known_answers(oracle):
    """db = d * (0.5 + s) * 0.25: the low nibble of scales[ib] scales values
    32ib..32ib+15, the high nibble 32ib+16..32ib+31, for s = 0..15 each."""
    grid = np.full(1024, 0x0101010101010101, dtype=np.uint64)
    z = np.zeros(32, dtype=np.int64)
    for rot in range(16):
        l1 = (np.arange(8) + rot) % 16
        l2 = (np.arange(8) * 3 + rot + 5) % 16
        v = oracle.dequant_row(IQ2_S, enc_iq2_s(f32(1.0), z, z, l1, l2), 256, grid=grid)
        want = np.concatenate([np.concatenate([np.full(16, 0.125 + 0.25 * a), np.full(16, 0.125 + 0.25 * b)])
                               for a, b in zip(l1, l2)]).astype(np.float32)
        assert np.array_equal(v, want), rot


def test_iq2_s_index_high_bits(oracle):
    """The two high index bits of lookup i8 sit at bits 2 * (i8 % 4) of
    qh[i8 / 4]: indices 256 apart read different grid entries."""
    grid = np.zeros(1024, dtype=np.uint64)
    for q in range(4):  # entry 256 q + 7 has every magnitude q + 1
        grid[256 * q + 7] = np.uint64(0x0101010101010101 * (q + 1))
    zs = np.zeros(8, dtype=np.int64)
    rng = np.random.default_rng(9)
    hi = rng.integers(0, 4, 32)
    v = oracle.dequant_row(IQ2_S, enc_iq2_s(f32(1.0), 256 * hi + 7, np.zeros(32, np.int64), zs, zs), 256, grid=grid)
    assert np.array_equal(v, np.repeat(0.125 * (hi + 1), 8).astype(np.float32))


# ---- the Q4_0 quantizer used to build the BASELINE configs ------------------

def test_quantize_q4_0_invariants(oracle):
    w = synth.normal_weights(64, 512, seed=1)
    raw = synth.quantize_q4_0(w)
    deq = np.stack([oracle.dequant_row(Q4_0, raw[r], 512) for r in range(64)])
    blk = w.reshape(64, 16, 32)
    dq = deq.reshape(64, 16, 32)
    d = raw.reshape(64, 16, 18)[..., :2].copy().view(np.float16)[..., 0].astype(np.float32)
    # every value is within half a step of its input (plus the fp16 rounding
    # of d, at most 8 * 2^-11 * |d|), except where the code clamps at 15
    # (+7 d: the side opposite the absmax reaches only 7/8 of it), where the
    # error stays within one step
    err = np.abs(blk - dq)
    ad = np.broadcast_to(np.abs(d)[..., None], err.shape)
    clamped = dq == 7 * d[..., None]
    slack = np.float32(8 * 2.0 ** -11)
    assert np.all(err[~clamped] <= ad[~clamped] * (np.float32(0.5) + slack))
    assert np.all(err[clamped] <= ad[clamped] * (np.float32(1.0) + slack))
    assert clamped.any()
    # the signed absmax element maps to code 0 (value -8 d)
    idx = np.argmax(np.abs(blk), axis=2)
    at = np.take_along_axis(dq, idx[..., None], axis=2)[..., 0]
    assert np.array_equal(at, -8 * d)


# ---- the K/IQ quantizers used to build the BASELINE configs ------------------
# synth.quantize_kq encodes f32 weights per type; decoding its blocks through
# the (pinned) oracle must give back the weights up to each format's
# quantization error.  A wrong nibble order, shift or sign in the encoder gives
# errors of the order of the weights themselves (relative RMS ~1), far above
# these bounds (about 1.25 x what the encoder reaches on these inputs).

KQ_RMS_BOUND = {  # (N(0, 0.02), N(0, 0.02) with 1% x8 outliers)
    "Q3_K": (0.19, 0.24), "Q4_K": (0.10, 0.12), "Q5_K": (0.048, 0.059), "Q6_K": (0.024, 0.033),
    "IQ4_XS": (0.10, 0.133), "IQ3_S": (0.172, 0.218),
    # synthetic grids (random odd magnitudes) fit the weights far worse than ggml's
    "IQ3_XXS": (0.32, 0.61), "IQ2_S": (0.39, 0.68)}
KQ_TYPE_IDS = {"Q3_K": Q3_K, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K, "IQ4_XS": IQ4_XS, "IQ3_S": IQ3_S,
               "IQ3_XXS": IQ3_XXS, "IQ2_S": IQ2_S}


def quant_grid(t):
    if t == IQ3_S:
        return synth.iq3s_grid()
    rng = np.random.default_rng(t)
    n, w = (256, 4) if t == IQ3_XXS else (1024, 8)
    g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


def test_iq3s_grid_table_matches_oracle(oracle):
    # the quantizer reads the kernels' compiled-in table; the oracle's is
    # pinned against the reference build by hash
    assert np.array_equal(synth.iq3s_grid(), extract_iq3s_grid(oracle))


def test_heavy_tail_weights_recipe():
    base = synth.normal_weights(256, 1024, seed=5)
    w = synth.heavy_tail_weights(256, 1024, seed=5)
    changed = w != base
    assert 0.008 < changed.mean() < 0.012
    assert np.array_equal(w[changed], base[changed] * np.float32(8))


@pytest.mark.parametrize("recipe", ["normal", "heavy_tail"])
@pytest.mark.parametrize("name", list(KQ_RMS_BOUND))
def test_kq_quantizer_round_trip(oracle, name, recipe):
    t = KQ_TYPE_IDS[name]
    N, K = 16, 2048
    w = synth.normal_weights(N, K, 3) if recipe == "normal" else synth.heavy_tail_weights(N, K, 3)
    grid = quant_grid(t) if t in (IQ3_S, IQ3_XXS, IQ2_S) else None
    raw = synth.quantize_kq(t, w, grid)
    assert raw.shape == (N, K // 256 * oracle.block_bytes(t))
    deq = np.stack([oracle.dequant_row(t, raw[r], K, grid=grid if t != IQ3_S else None) for r in range(N)])
    assert np.all(np.isfinite(deq))
    rel = np.sqrt(np.mean((deq - w) ** 2) / np.mean(w ** 2))
    assert rel < KQ_RMS_BOUND[name][recipe != "normal"], (name, recipe, rel)
    # row by row the same (rows are quantized independently, on threads)
    one = synth.quantize_kq(t, w[5:6], grid)
    assert np.array_equal(one[0], raw[5])


def test_kq_quantizer_zero_and_constant_blocks(oracle):
    # an all-zero superblock encodes to zero for every type; a constant block
    # is reproduced to within the format's step (grid types: to within the
    # spacing of the grid's entries, which holds no constant entry at the
    # top of its range, and with every sign right)
    for name, t in KQ_TYPE_IDS.items():
        grid = quant_grid(t) if t in (IQ3_S, IQ3_XXS, IQ2_S) else None
        g = grid if t in (IQ3_XXS, IQ2_S) else None
        z = synth.quantize_kq(t, np.zeros((1, 256), np.float32), grid)
        assert np.all(oracle.dequant_row(t, z[0], 256, grid=g) == 0), name
        c = synth.quantize_kq(t, np.full((1, 256), -0.03, np.float32), grid)
        v = oracle.dequant_row(t, c[0], 256, grid=g)
        tol = 0.6 if grid is not None else 0.15
        assert np.all(v < 0) and np.all(np.abs(v + 0.03) <= 0.03 * tol), (name, v[:4])


# ---- ggml-cpu Q4_0 x Q8_0 numerics (external restatement) -------------------
# ggml is not vendored in the reference, so this path cannot be compared with
# ggml itself here; it is pinned by what the mathematics fixes and by
# hand-written known answers for ggml's rounding, product association and
# block order (ggml_q8_cases.py).

def test_f32_to_fp16_matches_numpy_round_to_even(oracle):
    # every fp16 value round-trips, and every midpoint between neighbours
    # rounds to the even one -- numpy's float16 conversion is independent
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    got = np.array([oracle.f32_to_fp16(float(v)) for v in f[finite]], dtype=np.uint16)
    assert np.array_equal(got, h[finite])
    pos = np.arange(0x0000, 0x7bff, dtype=np.uint16)
    lo = pos.view(np.float16).astype(np.float64)
    hi = (pos + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in f32
    want = mid.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_fp16(float(v)) for v in mid], dtype=np.uint16)
    assert np.array_equal(got, want)
    for v, bits in ((65520.0, 0x7C00), (65519.0, 0x7BFF), (-1e30, 0xFC00), (2.0 ** -25, 0x0000),
                    (2.0 ** -24, 0x0001), (float("inf"), 0x7C00)):
        assert oracle.f32_to_fp16(v) == bits, v


def test_q8_0_quantization_invariants(oracle):
    rng = np.random.default_rng(77)
    x = (rng.standard_normal(32 * 64) * np.repeat(10.0 ** rng.uniform(-6, 6, 64), 32)).astype(np.float32)
    x[32:64] = 0.0
    q = oracle.quantize_q8_0(x).reshape(-1, 34)
    codes = q[:, 2:].view(np.int8).astype(np.int32)
    d16 = q[:, 0:2].copy().view(np.uint16).reshape(-1)
    xb = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(xb).max(axis=1)
    d = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)
    assert np.all(np.abs(codes) <= 127)
    # the absmax element is +-127; every value within half a step of q * d
    for b in range(len(xb)):
        if amax[b] == 0:
            assert np.all(codes[b] == 0) and d16[b] == 0
            continue
        j = int(np.argmax(np.abs(xb[b])))
        assert codes[b, j] == (127 if xb[b, j] > 0 else -127)
        assert np.all(np.abs(xb[b] - codes[b] * d[b]) <= 0.5 * d[b] * (1 + 1e-6))
        assert d16[b] == np.float32(d[b]).astype(np.float16).view(np.uint16)


def test_gemv_q4_0_q8_0_against_f32_path_on_dequantized_activation(oracle):
    # the blocked integer form equals the f32 GEMV of the same weights against
    # the dequantized Q8_0 activation, up to f32 rounding of the two orders
    N, K = 96, 2048
    raw = synth.random_q4_0(N, K, seed=31)
    x = synth.activations(K, seed=32)
    y8 = oracle.gemv_q4_0_q8_0(raw, N, K, x)
    q = oracle.quantize_q8_0(x).reshape(-1, 34)
    dx = np.array([oracle.fp16_to_f32(int(v)) for v in q[:, 0:2].copy().view(np.uint16).reshape(-1)], np.float32)
    xd = (q[:, 2:].view(np.int8).astype(np.float32) * dx[:, None]).reshape(-1)
    yf = oracle.gemv(2, raw, N, K, xd)
    norms = oracle.row_norms(2, raw, N, K)
    assert np.all(np.abs(y8 - yf) <= 1e-5 * norms * np.linalg.norm(xd))
    # and both are close to the f32-activation GEMV (what Q8_0 costs)
    y32 = oracle.gemv(2, raw, N, K, x)
    assert np.all(np.abs(y8 - y32) <= 2e-2 * norms * np.linalg.norm(x))


def test_q8_0_ties_round_half_away_from_zero(oracle):
    # exact halves of odd and even k, both signs, at d_x = 1 and d_x = 0.5:
    # ggml's quantize_row_q8_0 uses roundf (2.5 -> 3, -2.5 -> -3), so a
    # round-half-to-even quantizer (rintf) fails here
    import ggml_q8_cases as gq

    q = oracle.quantize_q8_0(gq.activation()).reshape(-1, 34)
    codes = q[:, 2:].view(np.int8).astype(np.int32)
    d16 = q[:, 0:2].copy().view(np.uint16).reshape(-1)
    for b, want in enumerate(gq.expected_codes()):
        assert list(codes[b]) == want, (b, list(codes[b]))
    assert list(d16[:7]) == [0x3C00, 0x3800, 0x3C00, 0x3C00, 0x3C00, 0x3C00, 0x3A00]  # 1, 0.5, 1 x 4, 0.75
    assert list(codes[6]) == [127] * 31 + [3]
    rint = np.rint(np.array(gq.B0_X, np.float64)).astype(np.int32)
    assert not np.array_equal(rint, codes[0])       # the case tells the two rules apart


def test_gemv_q4_0_q8_0_product_order_and_block_order(oracle):
    """ggml_vec_dot_q4_0_q8_0 forms sumi * d_w * d_x = (sumi * d_w) * d_x and
    adds the blocks to one f32 sum in block order.  Rows 0..63 read single
    Q8_0 codes, row 64 has block terms 2^24, 1, 1, -2^24 (0 in order; 2
    reversed, 1 pairwise), row 65 a product whose two associations differ
    in f32 (tests/ggml_q8_cases.py)."""
    import ggml_q8_cases as gq

    y = oracle.gemv_q4_0_q8_0(gq.weights(), gq.N, gq.K, gq.activation())
    want = gq.expected_y()
    bad = np.nonzero(y.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, (bad, y[bad], want[bad])
    # every plausible mistake gives a different row somewhere
    for name, alt in gq.alternatives().items():
        assert not np.array_equal(alt.view(np.uint32), want.view(np.uint32)), name


def test_gemv_q4_0_q8_0_known_answer(oracle):
    # codes 9 (+1) with d = 1 against x = 1: Q8_0 gives d_x = fp16(1/127),
    # q = 127, so each block adds 32 * 127 * fp16(1/127)
    N, K = 3, 96
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:] = 0x99
    raw = np.tile(blk, N * K // 32)
    y = oracle.gemv_q4_0_q8_0(raw, N, K, np.ones(K, dtype=np.float32))
    dx = np.float32(np.float32(1.0) / np.float32(127)).astype(np.float16).astype(np.float32)
    per = np.float32(4064) * np.float32(1.0) * dx
    want = np.float32(0)
    for _ in range(K // 32):
        want = np.float32(want + per)
    assert np.array_equal(y, np.full(N, want, dtype=np.float32))


# ---- ggml-cpu K-quant / IQ x Q8_K numerics (external restatement) -----------
# The reference's live path for the 256-value types (src/xdna-gemv-engine.cpp:
# 1382-1399, 1430-1453).  ggml itself is not in this build, so the f32 order
# of ggml's generic code is restated, not compared with ggml; the quantizer,
# the integers and the sums are pinned here by invariants, known answers and
# the float64 dot of the dequantized operands.

KQ_ALL = (Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS, IQ3_S, IQ3_XXS, IQ2_S)


def test_q8_K_quantization_invariants(oracle):
    rng = np.random.default_rng(5)
    nb = 48
    x = (rng.standard_normal(256 * nb) * np.repeat(10.0 ** rng.uniform(-8, 8, nb), 256)).astype(np.float32)
    x[256:512] = 0.0                                   # an all-zero block
    x[1024 + 3], x[1024 + 9] = 7.0, -7.0               # a tie of |x|: the first wins
    x[1024:1024 + 256][np.abs(x[1024:1280]) > 6.0] = 0.0
    x[1024 + 3], x[1024 + 9] = 7.0, -7.0
    d, qs, bs = oracle.quantize_q8_K(x)
    xb = x.reshape(nb, 256).astype(np.float64)
    q = qs.astype(np.int64)
    assert np.array_equal(bs.astype(np.int64), q.reshape(nb, 16, 16).sum(axis=2))
    for b in range(nb):
        if not np.any(xb[b]):
            assert d[b] == 0 and not np.any(q[b])
            continue
        j = int(np.argmax(np.abs(xb[b])))           # first index of the largest |x|
        mx = np.float32(xb[b, j])
        iscale = np.float32(-127.0) / mx
        assert d[b] == np.float32(1.0) / iscale
        assert q[b, j] == -127                         # the largest value maps to -127 * sign
        assert np.all(np.abs(q[b]) <= 127)
        # every value within half a step (plus f32 rounding of iscale * x)
        assert np.all(np.abs(xb[b] - q[b] * np.float64(d[b])) <= 0.5 * abs(d[b]) * (1 + 1e-5))
    assert q[4, 3] == -127 and q[4, 9] == 127          # the tie: +7 first, so d < 0


def test_q8_K_known_answers(oracle):
    # x = (127, 64, -32, 0.5, 0, ...): max 127, iscale -1, codes (-127, -64,
    # 32, 0) (0.5 rounds to even), d = -1
    x = np.zeros(256, np.float32)
    x[:4] = [127.0, 64.0, -32.0, 0.5]
    d, qs, bs = oracle.quantize_q8_K(x)
    assert d[0] == -1.0 and list(qs[0, :4]) == [-127, -64, 32, 0] and not np.any(qs[0, 4:])
    assert bs[0, 0] == -159 and not np.any(bs[0, 1:])
    # a Q6_K superblock with d = 1, every scale 1 and every code 33 (+1):
    # aux = (-127, -64, 32, 0, ...), lanes = d_w * d_x * aux = (127, 64, -32),
    # summed in lane order: 159 (the f32 dot is 159.5: 0.5 quantized to 0)
    blk = np.zeros(210, np.uint8)
    blk[0:128] = 0x11                                   # low nibbles 1
    blk[128:192] = 0xAA                                 # high 2-bit fields 2 -> code 33
    blk[192:208] = 1
    blk[208:210] = half(1.0)
    assert np.array_equal(oracle.dequant_row(Q6_K, blk, 256), np.ones(256, np.float32))
    assert oracle.gemv_q8_K(Q6_K, blk, 1, 256, x)[0] == np.float32(159.0)
    # Q4_K with dmin: codes 1, scale 1, min 1 -> every weight 1*1 - 1*1 = 0:
    # sumf -= dmin_w * d_x * sum(bsums * min) cancels the lanes exactly
    b4 = np.zeros(144, np.uint8)
    b4[0:2], b4[2:4] = half(1.0), half(1.0)
    b4[4:12] = 1                                        # scales and mins of sub-blocks 0..3 = 1
    b4[12:16] = 0x11                                    # sub-blocks 4..7: low nibbles 1
    b4[16:] = 0x11
    assert np.array_equal(oracle.dequant_row(Q4_K, b4, 256), np.zeros(256, np.float32))
    assert oracle.gemv_q8_K(Q4_K, b4, 1, 256, x)[0] == 0.0


@pytest.mark.parametrize("t", KQ_ALL, ids=[TYPE_NAMES[t] for t in KQ_ALL])
def test_gemv_q8_K_against_f64_dot_on_dequantized_operands(oracle, t):
    """The integer blocks and their scales form the same number as the f64
    dot of the dequantized weights (the reference-pinned dequantizers) with
    the dequantized Q8_K activation, up to f32 rounding of ggml's sums: a
    wrong code, scale, sign, min or final factor fails."""
    N, K = 64, 2048
    grid = synthetic_grid(t, 3) if t in (IQ3_XXS, IQ2_S) else None
    raw = synth.random_blocks(t, N, K, seed=11)
    x = synth.activations(K, seed=12)
    y = oracle.gemv_q8_K(t, raw, N, K, x, grid=grid)
    d, qs, _ = oracle.quantize_q8_K(x)
    xq = (qs.astype(np.float64) * d.astype(np.float64)[:, None]).reshape(-1)
    rows = raw.reshape(N, -1)
    for r in range(N):
        w = oracle.dequant_row(t, rows[r], K, grid=grid).astype(np.float64)
        want = float(np.dot(w, xq))
        scale = float(np.dot(np.abs(w), np.abs(xq)))
        assert abs(float(y[r]) - want) <= 2e-6 * scale + 1e-30, (TYPE_NAMES[t], r, float(y[r]), want)


def test_gemv_q8_K_rows_independent_of_threads_and_shape(oracle):
    # a row's result depends only on its bytes and x (OpenMP split, row count)
    N, K = 37, 1024
    raw = synth.random_blocks(Q5_K, N, K, seed=2)
    x = synth.activations(K, seed=3)
    y = oracle.gemv_q8_K(Q5_K, raw, N, K, x)
    rb = raw.reshape(N, -1)
    for r in (0, 17, 36):
        assert oracle.gemv_q8_K(Q5_K, rb[r], 1, K, x)[0] == y[r]
