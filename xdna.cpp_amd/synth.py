"""Seeded synthetic inputs for the decode GEMV path (numpy).

These generate *inputs* -- weight bytes in ggml encodings and activation rows
-- for tests and the benchmark; they compute no GEMV.

* ``quantize_q4_0`` follows ggml's reference Q4_0 quantizer (the recipe the
  BASELINE configs name): per 32-value block, the signed value of largest
  magnitude ``m`` gives ``d = m / -8``; codes are
  ``min(15, trunc(x / d + 8.5))``; d is stored as IEEE half (RNE).
* ``random_q4_0`` mirrors the reference tests' generator: uniform nibbles and
  a scale drawn from {1/16, 1/8, 1/4, 1/2, 1} (tests/test-gemv-accuracy.cpp:59-79).
* ``random_blocks`` fills any block type with random bytes and sane fp16
  scales, the way tests/test-kquants-gemv.cpp:81-217 builds its inputs.
"""
from __future__ import annotations

import numpy as np

Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS = 2, 11, 12, 13, 14, 18, 21, 22, 23
BLOCK_VALUES = {Q4_0: 32, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256, IQ3_S: 256,
                IQ2_S: 256, IQ4_XS: 256}
BLOCK_BYTES = {Q4_0: 18, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110,
               IQ2_S: 82, IQ4_XS: 136}
# byte offsets of fp16 scale fields inside each block (d, and dmin where present)
HALF_FIELDS = {Q4_0: (0,), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,), IQ3_XXS: (0,),
               IQ3_S: (0,), IQ2_S: (0,), IQ4_XS: (0,)}


def normal_weights(N: int, K: int, seed: int, sigma: float = 0.02, chunk_rows: int = 4096) -> np.ndarray:
    """f32 [N, K] ~ N(0, sigma^2) from numpy's PCG64 stream `seed`."""
    rng = np.random.default_rng(seed)
    out = np.empty((N, K), dtype=np.float32)
    for r0 in range(0, N, chunk_rows):
        r1 = min(N, r0 + chunk_rows)
        out[r0:r1] = rng.standard_normal((r1 - r0, K), dtype=np.float32)
    out *= np.float32(sigma)
    return out


def activations(K: int, seed: int) -> np.ndarray:
    """f32 [K] ~ N(0, 1)."""
    return np.random.default_rng(seed).standard_normal(K, dtype=np.float32)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """ggml Q4_0 encoding of f32 rows w[N, K] (K % 32 == 0) -> uint8 [N, 18*K/32]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    nb = K // 32
    out = np.empty((N, nb, 18), dtype=np.uint8)
    step = max(1, (1 << 22) // max(K, 1))
    for r0 in range(0, N, step):
        r1 = min(N, r0 + step)
        blk = w[r0:r1].reshape(r1 - r0, nb, 32)
        idx = np.argmax(np.abs(blk), axis=2)
        m = np.take_along_axis(blk, idx[..., None], axis=2)[..., 0]
        d = (m / np.float32(-8.0)).astype(np.float32)
        with np.errstate(divide="ignore"):
            inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
        v = blk * inv[..., None] + np.float32(8.5)
        q = np.minimum(15, v.astype(np.int8)).astype(np.uint8)
        out[r0:r1, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(r1 - r0, nb, 2)
        out[r0:r1, :, 2:] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(N, nb * 18)


def random_q4_0(N: int, K: int, seed: int) -> np.ndarray:
    """Uniform nibbles, d in {2^-4 .. 1} (the reference tests' generator)."""
    rng = np.random.default_rng(seed)
    nb = K // 32
    blocks = np.empty((N, nb, 18), dtype=np.uint8)
    cand = np.array([0x2C00, 0x3000, 0x3400, 0x3800, 0x3C00], dtype=np.uint16)
    d = cand[rng.integers(0, 5, size=(N, nb))]
    blocks[..., 0:2] = d.view(np.uint8).reshape(N, nb, 2)
    blocks[..., 2:] = rng.integers(0, 256, size=(N, nb, 16), dtype=np.uint8)
    return blocks.reshape(N, nb * 18)


def random_blocks(t: int, N: int, K: int, seed: int, d_bits: int = 0x3800, dmin_bits: int = 0x3000) -> np.ndarray:
    """Random bytes of type t with every fp16 scale field set to finite values."""
    bv, bb = BLOCK_VALUES[t], BLOCK_BYTES[t]
    if K % bv:
        raise ValueError(f"K must be a multiple of {bv}")
    nb = K // bv
    rng = np.random.default_rng(seed)
    blocks = rng.integers(0, 256, size=(N, nb, bb), dtype=np.uint8)
    fields = HALF_FIELDS[t]
    for i, off in enumerate(fields):
        val = d_bits if i == 0 else dmin_bits
        blocks[..., off] = val & 0xFF
        blocks[..., off + 1] = val >> 8
    return blocks.reshape(N, nb * bb)
