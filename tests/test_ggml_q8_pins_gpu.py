"""ggml-cpu's Q4_0 x Q8_0 rounding and sum order on the GPU (context variant
MI355X_VARIANT_GGML_Q8): the launch kernel (single matrix and the
multi-matrix job form) and the persistent server's Q8_0 job form against
hand-written known answers (tests/ggml_q8_cases.py):
- Q8_0 codes of exact halves round away from zero (ggml's roundf), at
  d_x = 1 and d_x = 0.5;
- each block adds (sumi * d_w) * d_x, and the blocks of a row are summed in
  block order;
and bit for bit against the oracle's restatement on the same inputs."""
import numpy as np
import pytest

import ggml_q8_cases as gq
import mi355x

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0


@pytest.fixture(scope="module")
def cases():
    return gq.weights(), gq.activation(), gq.expected_y()


def same_bits(y, want, what):
    bad = np.nonzero(y.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, (what, bad[:8], y[bad[:8]], want[bad[:8]])


class ggml_q8:
    def __init__(self, ctx):
        self.ctx = ctx

    def __enter__(self):
        self.ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)

    def __exit__(self, *exc):
        self.ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


def test_oracle_gives_the_known_answers(oracle, cases):
    raw, x, want = cases
    same_bits(oracle.gemv_q4_0_q8_0(raw, gq.N, gq.K, x), want, "oracle")


def test_launch_kernel_ties_and_order(ctx, oracle, cases):
    raw, x, want = cases
    w = ctx.resident(Q4_0, raw, gq.N, gq.K)
    try:
        with ggml_q8(ctx):
            y = ctx.gemv(w, x)
    finally:
        w.free()
    same_bits(y, want, "mi355x_gemv GGML_Q8")
    same_bits(y, oracle.gemv_q4_0_q8_0(raw, gq.N, gq.K, x), "mi355x_gemv GGML_Q8 vs oracle")


def test_multi_job_kernel_ties_and_order(ctx, cases):
    # the same matrix as two jobs (rows 0..31 and 32..67) in one launch
    raw, x, want = cases
    rb = mi355x.row_bytes(Q4_0, gq.K)
    parts = [(0, 32), (32, gq.N)]
    ws = [ctx.resident(Q4_0, np.ascontiguousarray(raw[a:b]), b - a, gq.K) for a, b in parts]
    ys = [ctx.alloc(4 * (b - a)) for a, b in parts]
    xb = ctx.to_device(x)
    try:
        with ggml_q8(ctx):
            mi355x.check(ctx.gemv_multi_ptr(Q4_0, gq.K, xb.ptr,
                                            [(w.ptr, b - a, y.ptr) for w, y, (a, b) in zip(ws, ys, parts)]))
            ctx.sync()
        y = np.concatenate([yy.download(np.float32, b - a) for yy, (a, b) in zip(ys, parts)])
    finally:
        for w in ws:
            w.free()
        for yy in ys:
            yy.free()
        xb.free()
    assert rb * gq.N == raw.size
    same_bits(y, want, "mi355x_gemv_multi GGML_Q8")


def test_server_q8_0_job_ties_and_order(ctx, cases):
    raw, x, want = cases
    w = ctx.resident(Q4_0, raw, gq.N, gq.K)
    yd = ctx.alloc(4 * gq.N)
    try:
        with ggml_q8(ctx):
            with mi355x.Server(ctx, 4096) as srv:
                srv.gemv(x, [(w.ptr, gq.N, yd.ptr)])
                y = yd.download(np.float32, gq.N)
    finally:
        yd.free()
        w.free()
    same_bits(y, want, "server Q8_0 job")
