"""Batched Q4_0 GEMV (mi355x_gemv_batched): M activation rows against the same
resident weights, the M>1 case the reference admits for weights in its own
buffer type and computes as M sequential GEMVs (src/ggml-xdna.cpp:110-112,
287-296).  The batched forms read the weights once per launch.  Every output
must be within the GEMV tolerance of the oracle, and an activation's output
must agree across batch sizes and positions to float rounding (the form --
pipelined or K-split -- depends on the batch size, the arithmetic per block
does not)."""
import numpy as np
import pytest

import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0


def oracle_check(oracle, raw, N, K, xs, y, what):
    norms = oracle.row_norms(Q4_0, raw, N, K)
    for m in range(xs.shape[0]):
        check_gemv(y[m], oracle.gemv(Q4_0, raw, N, K, xs[m]), norms, xs[m], f"{what} activation {m}")


# row lengths cover 1-8 block columns per lane, with and without a partial
# last column; at K = 16384 LDS holds 3 activation tiles (staged in sets)
SHAPES = [(300, 2048), (1000, 4096), (777, 5120), (512, 8192), (96, 11008), (256, 14336), (128, 16384),
          (64, 256), (40, 1024), (3, 2048)]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [2, 3, 5, 8, 11])
def test_batched_matches_oracle(ctx, oracle, N, K, M):
    raw = synth.random_q4_0(N, K, seed=N + K + M)
    xs = np.stack([synth.activations(K, seed=100 + m) for m in range(M)])
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        y = ctx.gemv_batched(w, xs)
    finally:
        w.free()
    oracle_check(oracle, raw, N, K, xs, y, f"{N}x{K} M={M}")


@pytest.mark.parametrize("N,K", [(300, 2048), (777, 5120), (512, 8192), (128, 16384)])
def test_batched_output_independent_of_batch(ctx, N, K):
    """Activation j alone (a one-activation remainder), in a pair, in a batch
    of 4 and in a batch of 8 at another position: the same values."""
    raw = synth.random_q4_0(N, K, seed=11)
    xs = np.stack([synth.activations(K, seed=400 + m) for m in range(9)])
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        y8 = ctx.gemv_batched(w, xs[:8])
        y9 = ctx.gemv_batched(w, xs)  # a batch of 8, then a one-activation remainder
        y2 = ctx.gemv_batched(w, xs[6:8])
        y4 = ctx.gemv_batched(w, xs[4:8])
    finally:
        w.free()
    scale = np.abs(y8).max()
    for a, b in ((y9[:8], y8), (y2, y8[6:8]), (y4, y8[4:8])):
        np.testing.assert_allclose(a, b, rtol=2e-6, atol=2e-6 * scale)


def test_batched_strides_and_misaligned_rows(ctx, oracle):
    """Padded output rows, activation rows an odd number of floats apart
    (not 16-byte aligned), and a padded-but-aligned activation stride."""
    N, K, M = 513, 4096, 6
    raw = synth.random_q4_0(N, K, seed=5)
    xs = np.stack([synth.activations(K, seed=200 + m) for m in range(M)])
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        ref = ctx.gemv_batched(w, xs)
        for xst, yst in ((K + 1, N + 3), (K + 64, N), (K, N + 1)):
            y = ctx.gemv_batched(w, xs, x_stride=xst, y_stride=yst)
            assert np.array_equal(y, ref), (xst, yst)
    finally:
        w.free()
    oracle_check(oracle, raw, N, K, xs, ref, "strided")


def test_batched_known_answer_and_nonfinite(ctx):
    # codes 0x99 (+1, +1), d = 1 -> row sum of x; activation m is m+1 / 2
    N, K, M = 96, 2048, 4
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:] = 0x99
    raw = np.tile(blk, N * K // 32).reshape(N, -1)
    xs = np.stack([np.full(K, 0.5 * (m + 1), np.float32) for m in range(M)])
    xs[2, 7] = np.inf
    xs[3, 100] = np.nan
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        y = ctx.gemv_batched(w, xs)
    finally:
        w.free()
    assert np.all(y[0] == 1024.0) and np.all(y[1] == 2048.0)
    # a non-finite activation poisons its block (the digit path gives NaN
    # where a plain f32 sum would give inf), and only its own outputs
    assert not np.isfinite(y[2]).any() and np.all(np.isnan(y[3]))


def test_batched_fallbacks_match_oracle(ctx, oracle):
    """Shapes and variants the batched form does not take (row length not a
    multiple of 256 values, exact-f32 variant) run as sequential GEMVs."""
    cases = [(70, 96, mi355x.VARIANT_AUTO), (300, 4096, mi355x.VARIANT_EXACT_F32)]
    for N, K, var in cases:
        raw = synth.random_q4_0(N, K, seed=9)
        xs = np.stack([synth.activations(K, seed=300 + m) for m in range(3)])
        w = ctx.resident(Q4_0, raw, N, K)
        ctx.set_option(mi355x.OPT_VARIANT, var)
        try:
            y = ctx.gemv_batched(w, xs)
        finally:
            ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
            w.free()
        norms = oracle.row_norms(Q4_0, raw, N, K)
        for m in range(3):
            check_gemv(y[m], oracle.gemv(Q4_0, raw, N, K, xs[m]), norms, xs[m], f"{N}x{K} activation {m}")


def test_batched_rejects_bad_arguments(ctx):
    N, K = 64, 256
    raw = synth.random_q4_0(N, K, seed=1)
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        assert ctx.gemv_batched_ptr(Q4_0, w.ptr, N, K, 0, K, 0, N, -1) == mi355x.EINVAL
        assert ctx.gemv_batched_ptr(Q4_0, w.ptr, N, K, 16, K - 1, 16, N, 2) == mi355x.EINVAL
        assert ctx.gemv_batched_ptr(Q4_0, w.ptr, N, K, 16, K, 16, N - 1, 2) == mi355x.EINVAL
        assert ctx.gemv_batched_ptr(Q4_0, w.ptr, N, K + 1, 16, K + 1, 16, N, 2) == mi355x.EINVAL
        assert ctx.gemv_batched_ptr(Q4_0, w.ptr, N, K, 0, K, 0, N, 0) == mi355x.OK
    finally:
        w.free()
