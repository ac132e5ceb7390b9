"""mi355x_gemv_batched_noalloc: the allocation-free form of
mi355x_gemv_batched (activation tiles of the K-split batched form in the
library's static device scratch).  Called through the C-ABI and checked
against mi355x_gemv_batched -- the same kernels, so bit for bit -- and
against the oracle within the GEMV tolerance, on two calls in a row, the
second with a smaller input (the scratch keeps the first call's contents)."""
import ctypes

import numpy as np
import pytest

import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0


def batched(ctx, fn, w, xs):
    """M GEMVs through fn (a C entry point), device activation rows and outputs."""
    M, K = xs.shape
    xb = ctx.to_device(np.ascontiguousarray(xs, np.float32))
    yb = ctx.alloc(4 * M * w.N)
    try:
        mi355x.check(fn(ctx.h, w.t, w.ptr, w.N, w.K, xb.ptr, K, yb.ptr, w.N, M))
        ctx.sync()
        return yb.download(np.float32, M * w.N).reshape(M, w.N)
    finally:
        xb.free()
        yb.free()


# (N, K, M): first the largest tile set the static scratch holds (8
# activations of K = 16384, K-split form), then smaller inputs of the K-split
# form (rows of a partial 64-block column; 3 activations) and of the pipelined
# batched form (which needs no scratch)
CASES = [[(1000, 16384, 8), (300, 4352, 3)], [(777, 8192, 5), (128, 2048, 2)]]


@pytest.mark.parametrize("calls", CASES, ids=["16384x8_then_4352x3", "8192x5_then_2048x2"])
def test_noalloc_matches_batched_on_two_calls(ctx, oracle, calls):
    lib = ctx.lib
    for i, (N, K, M) in enumerate(calls):
        raw = synth.random_q4_0(N, K, seed=31 + 7 * i + N)
        xs = np.stack([synth.activations(K, seed=100 * i + m) for m in range(M)])
        w = ctx.resident(Q4_0, raw, N, K)
        try:
            got = batched(ctx, lib.mi355x_gemv_batched_noalloc, w, xs)
            ref = batched(ctx, lib.mi355x_gemv_batched, w, xs)
        finally:
            w.free()
        assert np.array_equal(got, ref), (i, N, K, M, np.abs(got - ref).max())
        norms = oracle.row_norms(Q4_0, raw, N, K)
        for m in range(M):
            check_gemv(got[m], oracle.gemv(Q4_0, raw, N, K, xs[m]), norms, xs[m], f"call {i} row {m}")


def test_noalloc_leaves_the_context_buffer_alone(ctx):
    """A fresh context (its stream warmed up by one fill): the
    allocation-free calls leave the device's free memory where it was."""
    N, K, M = 512, 16384, 8
    raw = synth.random_q4_0(N, K, seed=5)
    xs = np.stack([synth.activations(K, seed=m) for m in range(M)])
    with mi355x.Context(0) as c2:
        w = c2.resident(Q4_0, raw, N, K)
        xb = c2.to_device(xs)
        yb = c2.alloc(4 * M * N)
        try:
            mi355x.check(c2.lib.mi355x_fill(c2.h, yb.ptr, 0, 4 * M * N))
            c2.sync()
            free0, _ = c2.mem_info()
            for _ in range(3):
                mi355x.check(c2.lib.mi355x_gemv_batched_noalloc(c2.h, Q4_0, w.ptr, N, K, xb.ptr, K, yb.ptr, N, M))
            c2.sync()
            free1, _ = c2.mem_info()
            a = yb.download(np.float32, M * N)
            mi355x.check(c2.lib.mi355x_gemv_batched(c2.h, Q4_0, w.ptr, N, K, xb.ptr, K, yb.ptr, N, M))
            c2.sync()
            b = yb.download(np.float32, M * N)
        finally:
            yb.free()
            xb.free()
            w.free()
    assert free1 == free0
    assert np.array_equal(a, b)


def test_noalloc_rejects_what_would_allocate(ctx):
    N, K = 64, 512
    lib = ctx.lib
    raw = synth.random_blocks(mi355x.Q4_K, N, K, 3)
    w = ctx.resident(mi355x.Q4_K, raw, N, K)
    xb = ctx.alloc(4 * K + 64)
    yb = ctx.alloc(4 * N)
    try:
        # unaligned activation row for a K/IQ type: the K/IQ kernels would
        # copy it into a context buffer
        assert lib.mi355x_gemv_batched_noalloc(ctx.h, mi355x.Q4_K, w.ptr, N, K, xb.ptr + 4, K, yb.ptr, N, 1) \
            == mi355x.EINVAL
        assert "aligned" in mi355x.last_error()
        assert lib.mi355x_gemv_batched_noalloc(ctx.h, mi355x.Q4_K, w.ptr, N, K, xb.ptr, K, yb.ptr, N, 1) == mi355x.OK
        ctx.sync()
    finally:
        yb.free()
        xb.free()
        w.free()
