"""MI355X_OPT_OVERLAP: consecutive mi355x_gemv calls alternate between the
context's stream and a second one, so independent launches overlap; every
other call joins the second stream back.  Outputs are bit-identical to the
in-order launches (same kernels), and work queued after a join sees every
overlapped GEMV's result."""
import ctypes

import numpy as np
import pytest

import mi355x
import synth

pytestmark = pytest.mark.gpu

Q4_0, Q4_K, IQ4_XS, IQ2_S, IQ3_S = mi355x.Q4_0, mi355x.Q4_K, mi355x.IQ4_XS, mi355x.IQ2_S, mi355x.IQ3_S


def synthetic_grid(t, seed):
    # the same grid as the other K/IQ GPU tests install (process-wide table)
    rng = np.random.default_rng(seed)
    n, w = (256, 4) if t == 18 else (1024, 8)
    g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


class overlap:
    def __init__(self, ctx, streams=2):
        self.ctx, self.streams = ctx, streams

    def __enter__(self):
        self.ctx.set_option(mi355x.OPT_OVERLAP, self.streams)

    def __exit__(self, *exc):
        self.ctx.set_option(mi355x.OPT_OVERLAP, 0)


def weights(ctx, t, N, K, seed):
    raw = synth.random_q4_0(N, K, seed) if t == Q4_0 else synth.random_blocks(t, N, K, seed)
    return ctx.resident(t, raw, N, K)


@pytest.fixture(scope="module")
def mats(ctx):
    mi355x.set_iq_grid(IQ2_S, synthetic_grid(IQ2_S, IQ2_S))
    # IQ3_S at K = 8192: twelve-wavefront workgroups in order, eight when
    # overlapped (the same rows either way)
    spec = [(Q4_0, 4096, 4096), (Q4_0, 8192, 8192), (Q4_K, 1000, 4096), (IQ4_XS, 777, 8192), (Q4_0, 300, 2048),
            (IQ2_S, 4096, 8192), (IQ3_S, 1531, 8192)]
    ws = [(t, N, K, weights(ctx, t, N, K, seed=i + 1)) for i, (t, N, K) in enumerate(spec)]
    xs = {K: ctx.to_device(synth.activations(K, seed=K)) for K in {K for _, _, K in spec}}
    yield ws, xs
    for *_, w in ws:
        w.free()
    for b in xs.values():
        b.free()


@pytest.mark.parametrize("streams", [2, 3, 4])
def test_overlapped_gemvs_match_in_order(ctx, mats, streams):
    ws, xs = mats
    runs = [ws[i % len(ws)] for i in range(40)]
    ys = [ctx.alloc(4 * N) for _, N, _, _ in runs]
    try:
        refs = []
        for (t, N, K, w), y in zip(runs, ys):
            mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, y.ptr))
        refs = [y.download(np.float32, N) for (_, N, _, _), y in zip(runs, ys)]
        for y in ys:
            mi355x.check(ctx.lib.mi355x_fill(ctx.h, y.ptr, 0xFF, y.nbytes))
        with overlap(ctx, streams):
            for (t, N, K, w), y in zip(runs, ys):
                mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, y.ptr))
            ctx.sync()
            out = [y.download(np.float32, N) for (_, N, _, _), y in zip(runs, ys)]
    finally:
        for y in ys:
            y.free()
    for i, (a, b) in enumerate(zip(out, refs)):
        assert np.array_equal(a, b), i


@pytest.mark.parametrize("streams", [2, 4])
def test_join_orders_later_work(ctx, mats, streams):
    """An overlapped run, then a multi-GEMV that reads the run's outputs as its
    activation, then another overlapped run reading the multi's output: each
    step sees the previous one's results (the multi joins the second stream
    back; the next run forks after it)."""
    ws, xs = mats
    t, N, K, w = ws[0]  # Q4_0 4096 x 4096
    ya, yb, yc, yd = (ctx.alloc(4 * N) for _ in range(4))
    try:
        x0 = xs[K]

        def chain():
            mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, x0.ptr, ya.ptr))
            mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, x0.ptr, yb.ptr))
            jobs = (mi355x.GemvJob * 1)(mi355x.GemvJob(w.ptr, N, yc.ptr))
            mi355x.check(ctx.lib.mi355x_gemv_multi(ctx.h, t, K, yb.ptr, 1, jobs))
            mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, yc.ptr, yd.ptr))
            mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, ya.ptr, yb.ptr))
            ctx.sync()
            return [b.download(np.float32, N) for b in (ya, yb, yc, yd)]

        ref = chain()
        for b in (ya, yb, yc, yd):
            mi355x.check(ctx.lib.mi355x_fill(ctx.h, b.ptr, 0, b.nbytes))
        with overlap(ctx, streams):
            got = chain()
    finally:
        for b in (ya, yb, yc, yd):
            b.free()
    for i, (a, b) in enumerate(zip(got, ref)):
        assert np.array_equal(a, b), i


def test_ctx_stream_and_copies_after_overlap(ctx, mats):
    hip = ctypes.CDLL("libamdhip64.so")
    ws, xs = mats
    t, N, K, w = ws[1]  # Q4_0 8192 x 8192
    ys = [ctx.alloc(4 * N) for _ in range(6)]
    host = np.zeros(N, np.float32)
    try:
        mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, ys[0].ptr))
        ref = ys[0].download(np.float32, N)
        with overlap(ctx, 3):
            for y in ys:
                mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, y.ptr))
            # a copy the caller queues on the context's stream comes after the run
            s = ctx.lib.mi355x_ctx_stream(ctx.h)
            assert hip.hipMemcpyAsync(host.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ys[-1].ptr),
                                      ctypes.c_size_t(4 * N), 2, ctypes.c_void_p(s)) == 0
            assert hip.hipStreamSynchronize(ctypes.c_void_p(s)) == 0
            assert np.array_equal(host, ref)
            # the library's own synchronous copies join first too
            for y in ys:
                mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, y.ptr))
            outs = [y.download(np.float32, N) for y in ys]
    finally:
        for y in ys:
            y.free()
    for o in outs:
        assert np.array_equal(o, ref)


@pytest.mark.parametrize("streams", [2, 4])
def test_time_gemv_overlap_rotates_outputs(ctx, mats, streams):
    ws, xs = mats
    t, N, K, w = ws[1]
    y = ctx.alloc(4 * streams * N)
    ref_b = ctx.alloc(4 * N)
    try:
        mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xs[K].ptr, ref_b.ptr))
        ref = ref_b.download(np.float32, N)
        with overlap(ctx, streams):
            ms = ctx.time_gemv(t, [w.ptr], N, K, xs[K].ptr, y.ptr, 3, 20)
            outs = y.download(np.float32, streams * N).reshape(streams, N)
    finally:
        y.free()
        ref_b.free()
    assert ms > 0
    for o in outs:
        assert np.array_equal(o, ref)


def test_overlap_option_values(ctx):
    for bad in (1, 5, -1):
        assert ctx.lib.mi355x_ctx_set_option(ctx.h, mi355x.OPT_OVERLAP, bad) == mi355x.EINVAL
    for v in (2, 4, 3, 0):
        ctx.set_option(mi355x.OPT_OVERLAP, v)
