"""Writes tests/golden/ref_vectors.npz from the reference's own CPU code.

The reference's scalar Q4_0 oracle and header-only K/IQ refs are compiled
from /root/reference by oracle/Makefile into oracle/_ref/libxdna_ref.so
(target `ref`); this script feeds them seeded inputs and stores inputs and
outputs as plain arrays (no pickles), so the CPU oracle can be checked
against the reference where the reference is absent (the GPU box).

Functions captured (reference file:line):
  Q4_0 dequantize_row / gemv_f32 / gemv_bf16   src/xdna-q4-0-reference.cpp:302-406
  Q4_0 validate_row / validate_matrix          src/xdna-q4-0-reference.cpp:261-300
  K/IQ dequant + gemv_*_ref                    include/xdna/kquants.h:290-577
  iq3s_grid                                    include/xdna/kquants.h:220-285 (hash only)

Run:  make -C oracle ref && python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "xdna.cpp_amd"))

from oracle import IQ3_S, IQ4_XS, Q3_K, Q4_0, Q4_K, Q5_K, Q6_K, TYPE_NAMES, RefLib  # noqa: E402
import synth  # noqa: E402

REF_TYPES = (Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_XS, IQ3_S)
# (N, K) per type: a few rows, two or more blocks, one non-power-of-two K
SHAPES = {Q4_0: [(4, 96), (8, 1024)], Q3_K: [(4, 512)], Q4_K: [(4, 512)], Q5_K: [(4, 512)],
          Q6_K: [(4, 768)], IQ4_XS: [(4, 512)], IQ3_S: [(4, 512)]}


def main():
    if not RefLib.available():
        sys.exit("oracle/_ref/libxdna_ref.so is missing: run `make -C oracle ref` first")
    ref = RefLib()
    out = {}
    for t in REF_TYPES:
        name = TYPE_NAMES[t]
        for i, (N, K) in enumerate(SHAPES[t]):
            seed = 1000 * t + i
            if t == Q4_0:
                W = synth.random_q4_0(N, K, seed)
            else:
                # d / dmin spread over a few binades, random everything else
                W = synth.random_blocks(t, N, K, seed, d_bits=0x2E66, dmin_bits=0x2A00)
            x = np.random.default_rng(seed + 1).uniform(-0.5, 0.5, K).astype(np.float32)
            key = f"{name}_{i}"
            out[key + "_W"] = W.reshape(-1)
            out[key + "_x"] = x
            out[key + "_shape"] = np.array([N, K], dtype=np.int64)
            out[key + "_y"] = ref.gemv(t, W, N, K, x)
            out[key + "_deq0"] = ref.dequant_row(t, W.reshape(N, -1)[0], K)
            if t == Q4_0:
                xb = np.array([ref.lib.ref_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
                out[key + "_xbf16"] = xb
                out[key + "_ybf16"] = ref.gemv(t, W, N, K, xb)
    # Q4_0 validation outcomes on a grid of (values, bytes)
    cases = [(v, b) for v in (0, 1, 31, 32, 33, 64, 96) for b in (0, 17, 18, 19, 36, 54)]
    out["validate_row_cases"] = np.array(cases, dtype=np.uint64)
    out["validate_row_rc"] = np.array([ref.lib.ref_q4_0_validate_row(v, b) for v, b in cases], dtype=np.int32)
    mcases = [(r, v, b) for r in (0, 1, 2, 3) for v in (0, 31, 32, 64) for b in (0, 18, 36, 54, 72)]
    out["validate_matrix_cases"] = np.array(mcases, dtype=np.uint64)
    out["validate_matrix_rc"] = np.array([ref.lib.ref_q4_0_validate_matrix(r, v, b) for r, v, b in mcases],
                                         dtype=np.int32)
    # bf16 rounding of a spread of floats, specials included
    rng = np.random.default_rng(77)
    f = np.concatenate([rng.standard_normal(4096).astype(np.float32) * np.float32(3.0),
                        np.array([0.0, -0.0, 1.0, -2.0, 65504.0, 1e-40, -1e-40, 3.4e38, np.inf, -np.inf],
                                 dtype=np.float32),
                        # exact ties: low 16 bits 0x8000 with even and odd bf16 mantissa
                        np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], dtype=np.uint32).view(np.float32)])
    out["bf16_in"] = f
    out["bf16_out"] = np.array([ref.lib.ref_f32_to_bf16(float(v)) for v in f], dtype=np.uint16)
    g = ref.iq3s_grid()
    out["iq3s_grid_sha256"] = np.frombuffer(hashlib.sha256(g.astype("<u4").tobytes()).digest(), dtype=np.uint8)
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)
    print(f"wrote {len(out)} arrays to tests/golden/ref_vectors.npz")


if __name__ == "__main__":
    main()
