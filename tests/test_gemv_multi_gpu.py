"""mi355x_gemv_multi (several matrices sharing the activation row) on the
GPU: against single mi355x_gemv calls and the CPU oracle, the one-launch
pipelined form for Q4_0 rows of whole 64-block columns (the decode's q|k|v
and gate|up groups), and the per-matrix fallback elsewhere (other row
lengths, unaligned activations, the K/IQ types, the ggml-cpu numerics
variant), which must equal single calls bit for bit."""
import numpy as np
import pytest

import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu


def run_multi(ctx, t, K, raws, Ns, x, x_offset=0):
    ws = [ctx.resident(t, r, n, K) for r, n in zip(raws, Ns)]
    xp = np.zeros(K + 4, np.float32)
    xp[x_offset:x_offset + K] = x
    xb = ctx.to_device(xp)
    ys = [ctx.alloc(4 * n) for n in Ns]
    try:
        xptr = xb.ptr + 4 * x_offset
        mi355x.check(ctx.gemv_multi_ptr(t, K, xptr, [(w.ptr, n, y.ptr) for w, n, y in zip(ws, Ns, ys)]))
        ctx.sync()
        multi = [y.download(np.float32, n) for y, n in zip(ys, Ns)]
        single = []
        for w, n, y in zip(ws, Ns, ys):
            mi355x.check(ctx.gemv_ptr(t, w.ptr, n, K, xptr, y.ptr))
            ctx.sync()
            single.append(y.download(np.float32, n))
        return multi, single
    finally:
        for w in ws:
            w.free()
        for y in ys:
            y.free()
        xb.free()


@pytest.mark.parametrize("K,Ns", [(2048, [2048, 256, 256]), (2048, [11008, 11008]), (4096, [4096, 1024, 1024]),
                                  (8192, [64, 8192, 33]), (2048, [1, 2, 3, 4, 5, 6, 7, 8])])
def test_q4_0_one_launch_matches_single_calls_and_oracle(ctx, oracle, K, Ns):
    raws = [synth.random_q4_0(n, K, seed=n + i) for i, n in enumerate(Ns)]
    x = synth.activations(K, seed=K)
    multi, single = run_multi(ctx, mi355x.Q4_0, K, raws, Ns, x)
    for raw, n, ym, ys in zip(raws, Ns, multi, single):
        norms = oracle.row_norms(mi355x.Q4_0, raw, n, K)
        check_gemv(ym, oracle.gemv(mi355x.Q4_0, raw, n, K, x), norms, x, f"multi {n}x{K}")
        # the same per-row arithmetic; only the order of the 64 lane partials
        # may follow another rows-per-wavefront count
        assert np.abs(ym - ys).max() <= 1e-6 * np.abs(ys).max() + 1e-30


@pytest.mark.parametrize("K,Ns", [(2048, [2048, 256, 256]), (2048, [11008, 11008]), (11008, [2048, 5]),
                                  (4096, [1, 2, 3, 4, 5, 6, 7, 8])])
def test_ggml_q8_one_launch_is_bit_identical_to_single_calls(ctx, K, Ns):
    """The ggml-cpu numerics variant's multi-job launch: every row summed by
    one lane in block order, so bit-identical to one call per matrix."""
    raws = [synth.random_q4_0(n, K, seed=3 * n + i) for i, n in enumerate(Ns)]
    x = synth.activations(K, seed=K + 1)
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    try:
        multi, single = run_multi(ctx, mi355x.Q4_0, K, raws, Ns, x)
    finally:
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
    for ym, ys in zip(multi, single):
        assert np.array_equal(ym.view(np.uint32), ys.view(np.uint32))


@pytest.mark.parametrize("case", ["row_length", "unaligned_x", "q4_k", "ggml_q8_unaligned"])
def test_fallback_equals_single_calls(ctx, case):
    t, K, Ns, off = mi355x.Q4_0, 11008, [512, 512], 0
    if case == "unaligned_x":
        K, off = 2048, 1
    if case == "q4_k":
        t, K, Ns = mi355x.Q4_K, 2048, [300, 64, 64]
    if case == "ggml_q8_unaligned":
        K, off = 2048, 1
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    try:
        raws = [synth.random_blocks(t, n, K, seed=n) if t != mi355x.Q4_0 else synth.random_q4_0(n, K, seed=n)
                for n in Ns]
        x = synth.activations(K, seed=5)
        multi, single = run_multi(ctx, t, K, raws, Ns, x, off)
    finally:
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
    for ym, ys in zip(multi, single):
        assert np.array_equal(ym.view(np.uint32), ys.view(np.uint32))


def test_rejects_bad_job_lists(ctx):
    K = 2048
    w = ctx.resident(mi355x.Q4_0, synth.random_q4_0(64, K, 1), 64, K)
    xb = ctx.alloc(4 * K)
    yb = ctx.alloc(4 * 64)
    try:
        job = (w.ptr, 64, yb.ptr)
        for jobs in ([], [job] * (mi355x.MULTI_MAX_JOBS + 1), [(0, 64, yb.ptr)], [(w.ptr, 64, 0)]):
            assert ctx.gemv_multi_ptr(mi355x.Q4_0, K, xb.ptr, jobs) == mi355x.EINVAL
        assert ctx.gemv_multi_ptr(mi355x.Q4_0, K + 16, xb.ptr, [job]) == mi355x.EINVAL  # K % 32
        assert ctx.gemv_multi_ptr(mi355x.Q4_0, K, 0, [job]) == mi355x.EINVAL
    finally:
        w.free()
        xb.free()
        yb.free()
