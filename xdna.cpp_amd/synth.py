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

import concurrent.futures
import os
import re

import numpy as np
import threadpoolctl

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


# ---------------------------------------------------------------------------
# Per-type quantizers for the K-quant and IQ formats.
#
# Each takes f32 weights w[N, K] (K % 256 == 0) and returns the ggml block
# bytes uint8[N, K/256 * block_bytes].  They are simple, deterministic
# quantizers written from the block formats (the byte layouts are ggml's,
# ggml-common.h block_q3_K .. block_iq4_xs; the packing follows ggml-quants.c
# quantize_row_*_ref), not ggml's error-minimising searches: sub-block scales
# come from each sub-block's extreme value, the superblock scale from the
# largest sub-block scale, codes by rounding (grid types: the nearest grid
# entry in L2).  Every fp16 scale is rounded first and the codes are chosen
# against the rounded value.  What matters for the decode kernels is that the
# blocks are well-formed encodings of realistic weights (scale fields spread
# the way quantized N(0, s^2) weights spread them); the kernels' work per
# block does not depend on the values.

KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                         dtype=np.float32)


def iq3s_grid() -> np.ndarray:
    """IQ3_S codebook (uint32[512], four byte magnitudes per entry), read from
    the table the kernels compile in (csrc/iq3s_grid.h)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "iq3s_grid.h")
    with open(path) as f:
        text = f.read()
    body = text[text.index("kIq3sGrid[kIq3sGridSize] = {"):]
    body = body[body.index("{") + 1:body.index("};")]
    vals = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", body)], dtype=np.uint32)
    if vals.size != 512:
        raise ValueError(f"iq3s_grid.h: {vals.size} entries, expected 512")
    return vals


def heavy_tail_weights(N: int, K: int, seed: int, sigma: float = 0.02, frac: float = 0.01,
                       factor: float = 8.0) -> np.ndarray:
    """N(0, sigma^2) weights with a fraction `frac` of entries scaled by
    `factor` (the heavy-tail recipe of the IQ benchmark configuration)."""
    w = normal_weights(N, K, seed, sigma)
    rng = np.random.default_rng(seed + 0x5EED)
    for r0 in range(0, N, 4096):
        r1 = min(N, r0 + 4096)
        m = rng.random((r1 - r0, K), dtype=np.float32) < frac
        w[r0:r1][m] *= np.float32(factor)
    return w


def _half(v: np.ndarray):
    """float32 -> (fp16 bytes [..., 2], the rounded value as float32)."""
    h = np.minimum(v, np.float32(65504.0)).astype(np.float16)
    return h.view(np.uint8).reshape(*v.shape, 2), h.astype(np.float32)


def _div(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a / b with 0 where b == 0."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(b != 0, a / np.where(b != 0, b, 1), np.float32(0)).astype(np.float32)


def _extreme(x: np.ndarray) -> np.ndarray:
    """Signed value of largest magnitude along the last axis."""
    idx = np.argmax(np.abs(x), axis=-1)
    return np.take_along_axis(x, idx[..., None], axis=-1)[..., 0]


def _rint_clip(v: np.ndarray, lo: int, hi: int) -> np.ndarray:
    return np.clip(np.rint(v), lo, hi).astype(np.int32)


def _quant_k4(x: np.ndarray, nmax: int):
    """Q4_K / Q5_K scales: x[B, 8, 32] -> (d, dmin fp16 bytes, ls, lm, codes)."""
    lo = np.minimum(x.min(-1), 0)
    scale = (x.max(-1) - lo) / np.float32(nmax)
    mins = -lo
    hd, d = _half(scale.max(-1) / np.float32(63))
    hm, dmin = _half(mins.max(-1) / np.float32(63))
    ls = _rint_clip(_div(scale, d[:, None]), 0, 63)
    lm = _rint_clip(_div(mins, dmin[:, None]), 0, 63)
    de = d[:, None] * ls
    dm = dmin[:, None] * lm
    q = _rint_clip(_div(x + dm[..., None], np.broadcast_to(de[..., None], x.shape)), 0, nmax)
    return hd, hm, ls, lm, q


def _pack_k4_scales(ls: np.ndarray, lm: np.ndarray) -> np.ndarray:
    s = np.empty((ls.shape[0], 12), dtype=np.uint8)
    s[:, 0:4] = ls[:, 0:4] | ((ls[:, 4:8] >> 4) << 6)
    s[:, 4:8] = lm[:, 0:4] | ((lm[:, 4:8] >> 4) << 6)
    s[:, 8:12] = (ls[:, 4:8] & 15) | ((lm[:, 4:8] & 15) << 4)
    return s


def _q4_k(x):
    B = x.shape[0]
    hd, hm, ls, lm, q = _quant_k4(x.reshape(B, 8, 32), 15)
    L = q.reshape(B, 4, 2, 32)
    out = np.empty((B, 144), dtype=np.uint8)
    out[:, 0:2], out[:, 2:4], out[:, 4:16] = hd, hm, _pack_k4_scales(ls, lm)
    out[:, 16:] = (L[:, :, 0] | (L[:, :, 1] << 4)).reshape(B, 128)
    return out


def _q5_k(x):
    B = x.shape[0]
    hd, hm, ls, lm, q = _quant_k4(x.reshape(B, 8, 32), 31)
    L = q.reshape(B, 4, 2, 32)
    qh = np.zeros((B, 32), dtype=np.int32)
    for c in range(4):
        for h in range(2):
            qh |= (L[:, c, h] >> 4) << (2 * c + h)
    out = np.empty((B, 176), dtype=np.uint8)
    out[:, 0:2], out[:, 2:4], out[:, 4:16] = hd, hm, _pack_k4_scales(ls, lm)
    out[:, 16:48] = qh
    out[:, 48:] = ((L[:, :, 0] & 15) | ((L[:, :, 1] & 15) << 4)).reshape(B, 128)
    return out


def _signed_scales(x: np.ndarray, nq: float, nsc: float, sc_lo: int, sc_hi: int):
    """Q3_K / Q6_K / IQ4_XS: per sub-block scale m / -nq (m the extreme
    value), superblock d = (extreme sub-block scale) / -nsc; returns (fp16
    bytes of d, integer sub-block scales, effective scales d * sc)."""
    scale = _extreme(x) / np.float32(-nq)
    hd, d = _half(_extreme(scale) / np.float32(-nsc))
    sc = _rint_clip(_div(scale, d[:, None]), sc_lo, sc_hi)
    return hd, sc, d[:, None] * sc


def _q3_k(x):
    B = x.shape[0]
    xs = x.reshape(B, 16, 16)
    hd, sc, de = _signed_scales(xs, 4, 32, -32, 31)
    L = (_rint_clip(_div(xs, np.broadcast_to(de[..., None], xs.shape)), -4, 3) + 4).reshape(B, 256)
    lv = sc + 32
    s = np.empty((B, 12), dtype=np.int32)
    s[:, 0:8] = (lv[:, 0:8] & 15) | ((lv[:, 8:16] & 15) << 4)
    s[:, 8:12] = sum((lv[:, 4 * k:4 * k + 4] >> 4) << (2 * k) for k in range(4))
    Lr = L.reshape(B, 8, 32)
    hm = sum(((Lr[:, b] >> 2) & 1) << b for b in range(8))
    Lq = (L & 3).reshape(B, 2, 4, 32)
    q = sum(Lq[:, :, i] << (2 * i) for i in range(4))
    out = np.empty((B, 110), dtype=np.uint8)
    out[:, 0:32], out[:, 32:96], out[:, 96:108], out[:, 108:110] = hm, q.reshape(B, 64), s, hd
    return out


def _q6_k(x):
    B = x.shape[0]
    xs = x.reshape(B, 16, 16)
    hd, sc, de = _signed_scales(xs, 32, 128, -128, 127)
    L = (_rint_clip(_div(xs, np.broadcast_to(de[..., None], xs.shape)), -32, 31) + 32).reshape(B, 2, 4, 32)
    a, b, c, e = (L[:, :, i] for i in range(4))
    out = np.empty((B, 210), dtype=np.uint8)
    ql = out[:, 0:128].reshape(B, 2, 2, 32)
    ql[:, :, 0] = (a & 15) | ((c & 15) << 4)
    ql[:, :, 1] = (b & 15) | ((e & 15) << 4)
    out[:, 128:192] = ((a >> 4) | ((b >> 4) << 2) | ((c >> 4) << 4) | ((e >> 4) << 6)).reshape(B, 64)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = hd
    return out


def _iq4_xs(x):
    B = x.shape[0]
    xs = x.reshape(B, 8, 32)
    hd, sc, de = _signed_scales(xs, 127, 32, -32, 31)
    mids = (KVALUES_IQ4NL[1:] + KVALUES_IQ4NL[:-1]) / 2
    L = np.searchsorted(mids, _div(xs, np.broadcast_to(de[..., None], xs.shape))).astype(np.int32)
    lv = sc + 32
    out = np.empty((B, 136), dtype=np.uint8)
    out[:, 0:2] = hd
    sh = sum((lv[:, ib] >> 4) << (2 * ib) for ib in range(8)).astype(np.uint16)
    out[:, 2:4] = sh.view(np.uint8).reshape(B, 2)
    out[:, 4:8] = (lv[:, 0::2] & 15) | ((lv[:, 1::2] & 15) << 4)
    out[:, 8:] = (L[:, :, :16] | (L[:, :, 16:] << 4)).reshape(B, 128)
    return out


def _nearest(mags: np.ndarray, table: np.ndarray, chunk: int = 1024) -> np.ndarray:
    """Index of the nearest row of table[E, w] (L2) for each row of mags[n, w]."""
    t = table.astype(np.float32)
    tn = (t * t).sum(1)
    out = np.empty(mags.shape[0], dtype=np.int32)
    for i in range(0, mags.shape[0], chunk):
        a = mags[i:i + chunk]
        out[i:i + chunk] = np.argmin(tn[None, :] - 2 * (a @ t.T), axis=1)
    return out


def _grid_bytes(grid: np.ndarray, width: int) -> np.ndarray:
    return np.ascontiguousarray(grid).view(np.uint8).reshape(-1, width)


def _odd_scale(amax: np.ndarray, gmax: float, div: float):
    """Scale nibble s with db = d * (2s + 1) / div ~ amax / gmax, d shared by
    the superblock (the largest sub-block takes s = 15)."""
    want = amax / np.float32(gmax)
    hd, d = _half(want.max(-1) * np.float32(div / 31))
    s = _rint_clip((_div(want * np.float32(div), d[:, None]) - 1) / 2, 0, 15)
    return hd, s, d[:, None] * (2 * s + 1).astype(np.float32) / np.float32(div)


def _iq3_s(x, grid):
    B = x.shape[0]
    g = _grid_bytes(grid, 4)
    xs = x.reshape(B, 8, 32)
    hd, s, db = _odd_scale(np.abs(xs).max(-1), float(g.max()), 1.0)
    mags = _div(np.abs(xs), np.broadcast_to(db[..., None], xs.shape)).reshape(-1, 4)
    idx = _nearest(mags, g).reshape(B, 8, 8)
    out = np.empty((B, 110), dtype=np.uint8)
    out[:, 0:2] = hd
    out[:, 2:66] = (idx & 255).reshape(B, 64)
    out[:, 66:74] = sum(((idx[:, :, k] >> 8) & 1) << k for k in range(8))
    out[:, 74:106] = np.packbits((x < 0).reshape(B, 32, 8), axis=-1, bitorder="little")[..., 0]
    out[:, 106:110] = s[:, 0::2] | (s[:, 1::2] << 4)
    return out


def _even_signs(x8: np.ndarray) -> np.ndarray:
    """Sign bits of groups of 8 with an even number of negatives: where the
    count is odd, the entry of smallest magnitude takes the other sign."""
    neg = x8 < 0
    odd = (neg.sum(-1) & 1).astype(bool)
    j = np.argmin(np.abs(x8), axis=-1)
    flip = np.zeros_like(neg)
    np.put_along_axis(flip, j[..., None], odd[..., None], axis=-1)
    return neg ^ flip


def _iq3_xxs(x, grid):
    B = x.shape[0]
    g = _grid_bytes(grid, 4)
    xs = x.reshape(B, 8, 32)
    hd, s, db = _odd_scale(np.abs(xs).max(-1), float(g.max()), 4.0)
    mags = _div(np.abs(xs), np.broadcast_to(db[..., None], xs.shape)).reshape(-1, 4)
    idx = _nearest(mags, g).reshape(B, 64)
    neg = _even_signs(xs.reshape(B, 8, 4, 8))
    s7 = np.packbits(neg, axis=-1, bitorder="little")[..., 0].astype(np.uint32) & 127
    words = sum(s7[:, :, l] << (7 * l) for l in range(4)) | (s.astype(np.uint32) << 28)
    out = np.empty((B, 98), dtype=np.uint8)
    out[:, 0:2] = hd
    out[:, 2:66] = idx
    out[:, 66:98] = words.astype(np.uint32).view(np.uint8).reshape(B, 32)
    return out


def _iq2_s(x, grid):
    B = x.shape[0]
    g = _grid_bytes(grid, 8)
    xs = x.reshape(B, 16, 16)
    hd, s, db = _odd_scale(np.abs(xs).max(-1), float(g.max()), 8.0)
    mags = _div(np.abs(xs), np.broadcast_to(db[..., None], xs.shape)).reshape(-1, 8)
    idx = _nearest(mags, g).reshape(B, 32)
    out = np.empty((B, 82), dtype=np.uint8)
    out[:, 0:2] = hd
    out[:, 2:34] = idx & 255
    out[:, 34:66] = np.packbits((x < 0).reshape(B, 32, 8), axis=-1, bitorder="little")[..., 0]
    hi = (idx >> 8).reshape(B, 8, 4)
    out[:, 66:74] = sum(hi[:, :, l] << (2 * l) for l in range(4))
    out[:, 74:82] = s[:, 0::2] | (s[:, 1::2] << 4)
    return out


_KQ_QUANT = {Q3_K: _q3_k, Q4_K: _q4_k, Q5_K: _q5_k, Q6_K: _q6_k, IQ4_XS: _iq4_xs}
_GRID_QUANT = {IQ3_S: _iq3_s, IQ3_XXS: _iq3_xxs, IQ2_S: _iq2_s}


def quantize_kq(t: int, w: np.ndarray, grid: np.ndarray | None = None) -> np.ndarray:
    """f32 rows w[N, K] (K % 256 == 0) -> ggml blocks of K-quant / IQ type t,
    uint8[N, K/256 * block_bytes].  The grid types (IQ3_S, IQ3_XXS, IQ2_S)
    need their codebook: uint32[512] / uint32[256] of four byte magnitudes,
    uint64[1024] of eight."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    if K % 256:
        raise ValueError("K must be a multiple of 256")
    if t in _GRID_QUANT:
        if grid is None:
            raise ValueError("grid types need their codebook")
        fn = lambda x: _GRID_QUANT[t](x, grid)  # noqa: E731
    elif t in _KQ_QUANT:
        fn = _KQ_QUANT[t]
    else:
        raise ValueError(f"no K/IQ quantizer for type {t}")
    nb = K // 256
    out = np.empty((N, nb * BLOCK_BYTES[t]), dtype=np.uint8)
    step = max(1, (1 << 18) // K)

    def part(r0):
        r1 = min(N, r0 + step)
        out[r0:r1] = fn(w[r0:r1].reshape(-1, 256)).reshape(r1 - r0, -1)

    # numpy releases the GIL in its array loops: row ranges run on threads,
    # each with a one-thread BLAS (nested BLAS threads oversubscribe the cores
    # and make the small grid products many times slower)
    workers = max(1, min(8, os.cpu_count() or 1))
    with threadpoolctl.threadpool_limits(1, user_api="blas"):
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            list(pool.map(part, range(0, N, step)))
    return out
