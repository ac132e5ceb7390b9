"""Persistent Q4_0 GEMV server (mi355x_server_*): a resident kernel that takes
GEMV commands through pinned host memory, for decode loops.  Every output is
bit-identical to the launch path's arithmetic of the context's variant (the
row form MI355X_FORM_ROWS for the digit planes, mi355x_gemv for GGML_Q8) and
within the GEMV tolerance of the oracle.

Any free on the device stops the resident kernel (a hipFree waits for it), so
the tests that run several commands on one launch make their references and
buffers first and free nothing until the end; mi355x_server_running tells
whether the resident kernel is still there."""
import ctypes
import time

import numpy as np
import pytest

import decode
import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0


@pytest.fixture(scope="module")
def server(ctx):
    s = mi355x.Server(ctx, 16384)
    yield s
    s.close()


def rows_form(ctx, w, x):
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_ROWS)
    try:
        return ctx.gemv(w, x)
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)


def ggml_q8(ctx, w, x):
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    try:
        return ctx.gemv(w, x)
    finally:
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


class variant:
    def __init__(self, ctx, v):
        self.ctx, self.v = ctx, v

    def __enter__(self):
        self.ctx.set_option(mi355x.OPT_VARIANT, self.v)

    def __exit__(self, *exc):
        self.ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


def run_server(ctx, server, ws, x):
    """One command with one job per resident tensor in ws; device outputs."""
    ys = [ctx.alloc(4 * w.N) for w in ws]
    try:
        server.gemv(x, [(w.ptr, w.N, y.ptr) for w, y in zip(ws, ys)])
        return [y.download(np.float32, w.N) for w, y in zip(ws, ys)]
    finally:
        for y in ys:
            y.free()


# decode shapes (q|k|v, o, gate|up, down, vocabulary) and others: 1-8 block
# columns per lane, with and without a partial last column (8 with one:
# 448 < K / 32 < 512), tiny N
SHAPES = [(2560, 2048), (2048, 2048), (22016, 2048), (2048, 11008), (151936, 2048), (300, 4096), (777, 5120),
          (513, 8192), (64, 14336), (129, 15616), (200, 16384), (3, 2048), (255, 256)]


@pytest.mark.parametrize("N,K", SHAPES)
def test_server_matches_row_form_and_oracle(ctx, server, oracle, N, K):
    raw = synth.random_q4_0(N, K, seed=N ^ K)
    x = synth.activations(K, seed=K + 1)
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        (y,) = run_server(ctx, server, [w], x)
        ref = rows_form(ctx, w, x)
    finally:
        w.free()
    assert np.array_equal(y, ref), (N, K, np.abs(y - ref).max())
    if N * K <= 50_000_000:
        check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), oracle.row_norms(Q4_0, raw, N, K), x, f"server {N}x{K}")


@pytest.mark.parametrize("N,K", SHAPES)
def test_server_ggml_q8_bit_identical(ctx, server, oracle, N, K):
    """The Q8_0 job form (context variant GGML_Q8): bit-identical to
    mi355x_gemv in that variant and to the oracle's restatement of ggml-cpu's
    Q4_0 x Q8_0 arithmetic (blocks summed in order per row)."""
    raw = synth.random_q4_0(N, K, seed=N ^ K ^ 5)
    x = synth.activations(K, seed=K + 2)
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        with variant(ctx, mi355x.VARIANT_GGML_Q8):
            (y,) = run_server(ctx, server, [w], x)
        ref = ggml_q8(ctx, w, x)
    finally:
        w.free()
    assert np.array_equal(y, ref), (N, K, np.abs(y - ref).max())
    if N * K <= 50_000_000:
        assert np.array_equal(y, oracle.gemv_q4_0_q8_0(raw, N, K, x)), (N, K)


def test_server_many_commands_per_launch(ctx, server):
    """24 commands on one resident kernel, 1-4 jobs each, alternating the
    digit and Q8_0 job forms: every output equals its launch-path reference
    and the kernel stays resident throughout."""
    K = 2048
    shapes = [700, 64, 3000, 129]
    raws = [synth.random_q4_0(N, K, seed=10 + i) for i, N in enumerate(shapes)]
    ws = [ctx.resident(Q4_0, r, N, K) for r, N in zip(raws, shapes)]
    xs = [synth.activations(K, seed=500 + it) for it in range(24)]
    modes = [mi355x.VARIANT_AUTO if it % 3 else mi355x.VARIANT_GGML_Q8 for it in range(24)]
    refs = [[(rows_form if m == mi355x.VARIANT_AUTO else ggml_q8)(ctx, w, x) for w in ws]
            for x, m in zip(xs, modes)]
    ys = [ctx.alloc(4 * w.N) for w in ws]
    try:
        server.stop()
        assert not server.running()
        for it, (x, m) in enumerate(zip(xs, modes)):
            sel = [(it + j) % 4 for j in range(1 + it % 4)]
            with variant(ctx, m):
                server.gemv(x, [(ws[i].ptr, ws[i].N, ys[i].ptr) for i in sel])
            assert server.running(), it
            for i in sel:
                assert np.array_equal(ys[i].download(np.float32, ws[i].N), refs[it][i]), (it, i)
    finally:
        for b in ys + ws:
            b.free()
    assert not server.running()  # the frees stopped it


def test_server_pinned_outputs(ctx, server):
    hip = ctypes.CDLL("libamdhip64.so")
    N, K = 4096, 2048
    raw = synth.random_q4_0(N, K, seed=77)
    w = ctx.resident(Q4_0, raw, N, K)
    xs = [synth.activations(K, seed=900 + it) for it in range(30)]
    refs = [rows_form(ctx, w, x) for x in xs]
    hptr = ctypes.c_void_p()
    mi355x.check(ctx.lib.mi355x_host_malloc(4 * N, ctypes.byref(hptr)))
    dptr = ctypes.c_void_p()
    try:
        assert hip.hipHostGetDevicePointer(ctypes.byref(dptr), hptr, 0) == 0
        host_y = np.ctypeslib.as_array(ctypes.cast(hptr, ctypes.POINTER(ctypes.c_float)), shape=(N,))
        for it, x in enumerate(xs):
            host_y[:] = np.nan
            server.gemv(x, [(w.ptr, N, dptr.value)])
            assert np.array_equal(host_y, refs[it]), it
    finally:
        mi355x.check(ctx.lib.mi355x_host_free(hptr))
        w.free()


def test_server_stop_and_idle_relaunch(ctx, server):
    """The host's relaunch after 0.5 s idle (inside the next call) and the
    kernel's own exit after 1 s without a command."""
    N, K = 1000, 4096
    raw = synth.random_q4_0(N, K, seed=3)
    w = ctx.resident(Q4_0, raw, N, K)
    x = synth.activations(K, seed=4)
    ref = rows_form(ctx, w, x)
    y = ctx.alloc(4 * N)
    out = []
    try:
        job = [(w.ptr, N, y.ptr)]
        server.gemv(x, job)
        t0 = time.perf_counter()
        out.append(y.download(np.float32, N))
        # the copy ran beside the resident kernel (room for it on the CUs)
        assert time.perf_counter() - t0 < 0.2
        assert server.running()
        server.stop()
        assert not server.running()
        server.gemv(x, job)  # relaunch after a stop
        out.append(y.download(np.float32, N))
        assert server.running()
        time.sleep(0.7)  # past the host's idle limit, before the kernel's
        assert server.running()
        server.gemv(x, job)  # the call stops and relaunches the kernel
        out.append(y.download(np.float32, N))
        assert server.running()
        time.sleep(2.5)  # past the kernel's own idle exit
        assert not server.running()
        server.gemv(x, job)  # relaunch after the kernel left by itself
        out.append(y.download(np.float32, N))
    finally:
        y.free()
        w.free()
    for i, o in enumerate(out):
        assert np.array_equal(o, ref), i


def test_free_on_another_context_stops_the_server(ctx, server):
    """A free through a second context on the same device stops this
    server's resident kernel first (hipFree would otherwise wait for it)."""
    N, K = 512, 2048
    w = ctx.resident(Q4_0, synth.random_q4_0(N, K, seed=21), N, K)
    y = ctx.alloc(4 * N)
    try:
        x = synth.activations(K, seed=22)
        server.gemv(x, [(w.ptr, N, y.ptr)])
        assert server.running()
        with mi355x.Context(0) as other:
            b = other.alloc(1 << 20)
            t0 = time.perf_counter()
            b.free()
            assert time.perf_counter() - t0 < 0.5  # no wait for the idle exit
        assert not server.running()
    finally:
        y.free()
        w.free()


# (K, F, N): the decode FFN, tiny, ragged N, F = max_k, N above the grid
SWIGLU_SHAPES = [(2048, 11008, 2048), (256, 256, 3), (4096, 1024, 777), (512, 16384, 100), (1024, 768, 4099)]


def swiglu_weights(ctx, K, F, N, seed):
    raws = [synth.random_q4_0(F, K, seed=seed), synth.random_q4_0(F, K, seed=seed + 1),
            synth.random_q4_0(N, F, seed=seed + 2)]
    ws = [ctx.resident(Q4_0, raws[0], F, K), ctx.resident(Q4_0, raws[1], F, K), ctx.resident(Q4_0, raws[2], N, F)]
    return raws, ws


def swiglu_separate(ctx, server, ws, x):
    """gate and up as one command, the host's SwiGLU step, down as another."""
    g, u = run_server(ctx, server, ws[:2], x)
    (y,) = run_server(ctx, server, ws[2:], decode.silu_mul(g, u))
    return y, g, u


def swiglu_fused(ctx, server, ws, x):
    F, N = ws[0].N, ws[2].N
    y = ctx.alloc(4 * N)
    try:
        server.swiglu(x, ws[0].ptr, ws[1].ptr, F, ws[2].ptr, N, y.ptr)
        return y.download(np.float32, N)
    finally:
        y.free()


@pytest.mark.parametrize("v", [mi355x.VARIANT_AUTO, mi355x.VARIANT_GGML_Q8])
@pytest.mark.parametrize("K,F,N", SWIGLU_SHAPES)
def test_server_swiglu_matches_separate_commands(ctx, server, oracle, K, F, N, v):
    """mi355x_server_swiglu (gate|up, SiLU on the device, grid barrier, down)
    equals three separate steps -- server GEMVs around the host's SwiGLU
    step -- bit for bit, in the digit and the ggml Q8_0 arithmetic; in the
    latter also the oracle's ggml-cpu chain."""
    raws, ws = swiglu_weights(ctx, K, F, N, seed=K ^ F ^ N)
    x = synth.activations(K, seed=F + 3)
    try:
        with variant(ctx, v):
            want, g, u = swiglu_separate(ctx, server, ws, x)
            got = swiglu_fused(ctx, server, ws, x)
    finally:
        for w in ws:
            w.free()
    assert np.array_equal(got, want), (K, F, N, np.abs(got - want).max())
    if v == mi355x.VARIANT_GGML_Q8 and F * K <= 30_000_000:
        go = oracle.gemv_q4_0_q8_0(raws[0], F, K, x)
        uo = oracle.gemv_q4_0_q8_0(raws[1], F, K, x)
        assert np.array_equal(g, go) and np.array_equal(u, uo)
        assert np.array_equal(got, oracle.gemv_q4_0_q8_0(raws[2], N, F, decode.silu_mul(go, uo)))


def test_server_swiglu_between_plain_commands(ctx, server):
    """SwiGLU and plain commands alternating on one resident kernel (the grid
    barrier's count carries across commands): every output equals its
    reference and the kernel stays resident."""
    K, F, N = 2048, 2816, 2048
    _, ws = swiglu_weights(ctx, K, F, N, seed=40)
    xs = [synth.activations(K, seed=600 + it) for it in range(12)]
    want = [swiglu_separate(ctx, server, ws, x)[0] for x in xs]
    plain = [rows_form(ctx, ws[0], x) for x in xs]
    y = ctx.alloc(4 * N)
    yp = ctx.alloc(4 * F)
    try:
        server.stop()
        for it, x in enumerate(xs):
            server.swiglu(x, ws[0].ptr, ws[1].ptr, F, ws[2].ptr, N, y.ptr)
            assert server.running(), it
            assert np.array_equal(y.download(np.float32, N), want[it]), it
            server.gemv(x, [(ws[0].ptr, F, yp.ptr)])
            assert np.array_equal(yp.download(np.float32, F), plain[it]), it
    finally:
        for b in [y, yp] + ws:
            b.free()


def test_server_swiglu_rejects_bad_arguments(ctx, server):
    K, F, N = 512, 512, 64
    _, ws = swiglu_weights(ctx, K, F, N, seed=50)
    y = ctx.alloc(4 * N)
    try:
        x = np.ones(K, np.float32)
        g, u, d = ws[0].ptr, ws[1].ptr, ws[2].ptr
        assert server.swiglu_ptr(x[:500], g, u, F, d, N, y.ptr) == mi355x.EINVAL  # K % 256
        assert server.swiglu_ptr(x, g, u, 500, d, N, y.ptr) == mi355x.EINVAL  # F % 256
        assert server.swiglu_ptr(x, g, u, 16640, d, N, y.ptr) == mi355x.EINVAL  # F > max_k
        assert server.swiglu_ptr(x, g, u, F, d, 0, y.ptr) == mi355x.EINVAL
        assert server.swiglu_ptr(x, g + 2, u, F, d, N, y.ptr) == mi355x.EINVAL  # alignment
        assert server.swiglu_ptr(x, g, u, F, d + 8, N, y.ptr) == mi355x.EINVAL
        assert server.swiglu_ptr(x, g, u, F, d, N, 0) == mi355x.EINVAL
        with variant(ctx, mi355x.VARIANT_EXACT_F32):
            assert server.swiglu_ptr(x, g, u, F, d, N, y.ptr) == mi355x.EUNSUPPORTED
        server.swiglu(x, g, u, F, d, N, y.ptr)  # still serves
    finally:
        for b in [y] + ws:
            b.free()


# (K, H, F): the 3B decode layer, tiny, H at its 4096 limit, F = max_k, K != H
BLOCK_SHAPES = [(2048, 2048, 11008), (256, 256, 512), (4096, 4096, 1024), (512, 1024, 16384 - 1024),
                (1024, 2048, 768)]
EPS = 1e-6


def block_weights(ctx, K, H, F, seed):
    shapes = [(H, K), (F, H), (F, H), (H, F)]
    raws = [synth.random_q4_0(n, k, seed=seed + i) for i, (n, k) in enumerate(shapes)]
    return raws, [ctx.resident(Q4_0, r, n, k) for r, (n, k) in zip(raws, shapes)]


def block_separate(ctx, server, ws, x, resid, norm_w):
    """o, the residual add, the host's RMSNorm, gate|up, the host's SwiGLU
    step, down and the second residual add as separate steps."""
    (o,) = run_server(ctx, server, ws[:1], x)
    r = resid + o
    g, u = run_server(ctx, server, ws[1:3], decode.rmsnorm(r, norm_w, EPS))
    (dn,) = run_server(ctx, server, ws[3:], decode.silu_mul(g, u))
    return r + dn


def block_fused(ctx, server, ws, x, resid, nw, nxt=None):
    """nxt: (next norm weights on the device, resident W_next) or None;
    returns y and, with nxt, y_next."""
    H, F = ws[0].N, ws[1].N
    y = ctx.alloc(4 * H)
    yn = ctx.alloc(4 * nxt[1].N) if nxt else None
    try:
        extra = (nxt[0].ptr, nxt[1].ptr, nxt[1].N, yn.ptr) if nxt else ()
        server.block(x, ws[0].ptr, resid, nw.ptr, EPS, ws[1].ptr, ws[2].ptr, F, ws[3].ptr, y.ptr, *extra)
        out = y.download(np.float32, H)
        return (out, yn.download(np.float32, nxt[1].N)) if nxt else out
    finally:
        y.free()
        if yn:
            yn.free()


@pytest.mark.parametrize("v", [mi355x.VARIANT_AUTO, mi355x.VARIANT_GGML_Q8])
@pytest.mark.parametrize("K,H,F", BLOCK_SHAPES)
def test_server_block_matches_separate_steps(ctx, server, K, H, F, v):
    """mi355x_server_block (o, residual, RMSNorm on the device, gate|up, SiLU,
    down, residual, with grid barriers) equals the separate steps around the
    host's RMSNorm and SwiGLU step, bit for bit, in both arithmetics; with
    the next stage (RMSNorm of y, then the next layer's q|k|v), y is the same
    and y_next equals a server GEMV over the host's RMSNorm of y."""
    _, ws = block_weights(ctx, K, H, F, seed=K ^ H ^ F)
    rng = np.random.default_rng(H + F)
    x = synth.activations(K, seed=K + 9)
    resid = (rng.standard_normal(H) * 0.5).astype(np.float32)
    norm_w = rng.uniform(0.5, 1.5, H).astype(np.float32)
    nw = ctx.to_device(norm_w)
    next_norm = rng.uniform(0.5, 1.5, H).astype(np.float32)
    nn = ctx.to_device(next_norm)
    n_next = 2560 if H == 2048 else 3 * H // 2 + 17
    w_next = ctx.resident(Q4_0, synth.random_q4_0(n_next, H, seed=H + 5), n_next, H)
    try:
        with variant(ctx, v):
            want = block_separate(ctx, server, ws, x, resid, norm_w)
            (want_next,) = run_server(ctx, server, [w_next], decode.rmsnorm(want, next_norm, EPS))
            got = block_fused(ctx, server, ws, x, resid, nw)
            again = block_fused(ctx, server, ws, x, resid, nw)
            got2, got_next = block_fused(ctx, server, ws, x, resid, nw, (nn, w_next))
    finally:
        for b in ws + [nw, nn, w_next]:
            b.free()
    assert np.array_equal(got, want), (K, H, F, np.abs(got - want).max())
    assert np.array_equal(again, got)
    assert np.array_equal(got2, want)
    assert np.array_equal(got_next, want_next), (K, H, F, np.abs(got_next - want_next).max())


@pytest.mark.parametrize("v", [mi355x.VARIANT_AUTO, mi355x.VARIANT_GGML_Q8])
def test_server_block_residual_kept_in_the_server(ctx, server, v):
    """A chain of block commands that pass the residual only to the first and
    read y back only after the last (the server keeps it in between, with
    plain and SwiGLU commands in the way): the same bits as the separate
    steps with the residual on the host."""
    K, H, F = 2048, 2048, 2816
    _, ws = block_weights(ctx, K, H, F, seed=90)
    rng = np.random.default_rng(91)
    norm_w = rng.uniform(0.5, 1.5, H).astype(np.float32)
    nw = ctx.to_device(norm_w)
    xs = [synth.activations(K, seed=900 + it) for it in range(4)]
    r0 = (rng.standard_normal(H) * 0.5).astype(np.float32)
    y = ctx.alloc(4 * H)
    yp = ctx.alloc(4 * F)
    try:
        with variant(ctx, v):
            want = r0
            for x in xs:
                want = block_separate(ctx, server, ws, x, want, norm_w)
            for it, x in enumerate(xs):
                last = it == len(xs) - 1
                server.block(x, ws[0].ptr, r0 if it == 0 else H, nw.ptr, EPS, ws[1].ptr, ws[2].ptr, F, ws[3].ptr,
                             y.ptr if last else 0)
                if not last:  # other commands between the blocks leave the kept residual alone
                    server.gemv(x, [(ws[0].ptr, H, yp.ptr)])
                    server.swiglu(x, ws[1].ptr, ws[2].ptr, F, ws[3].ptr, H, yp.ptr)
            got = y.download(np.float32, H)
    finally:
        for b in [y, yp, nw] + ws:
            b.free()
    assert np.array_equal(got, want), np.abs(got - want).max()


def test_server_block_between_other_commands(ctx, server):
    """Block, SwiGLU and plain commands in turn on one resident kernel (the
    barrier count carries across commands of both kinds)."""
    K, H, F = 2048, 2048, 2816
    _, ws = block_weights(ctx, K, H, F, seed=70)
    rng = np.random.default_rng(71)
    norm_w = rng.uniform(0.5, 1.5, H).astype(np.float32)
    nw = ctx.to_device(norm_w)
    xs = [synth.activations(K, seed=700 + it) for it in range(8)]
    rs = [(rng.standard_normal(H) * 0.5).astype(np.float32) for _ in xs]
    want = [block_separate(ctx, server, ws, x, r, norm_w) for x, r in zip(xs, rs)]
    want_sw = [swiglu_separate(ctx, server, ws[1:], x)[0] for x in xs]
    plain = [rows_form(ctx, ws[0], x) for x in xs]
    y = ctx.alloc(4 * H)
    try:
        server.stop()
        for it, (x, r) in enumerate(zip(xs, rs)):
            server.block(x, ws[0].ptr, r, nw.ptr, EPS, ws[1].ptr, ws[2].ptr, F, ws[3].ptr, y.ptr)
            assert np.array_equal(y.download(np.float32, H), want[it]), it
            server.swiglu(x, ws[1].ptr, ws[2].ptr, F, ws[3].ptr, H, y.ptr)
            assert np.array_equal(y.download(np.float32, H), want_sw[it]), it
            server.gemv(x, [(ws[0].ptr, H, y.ptr)])
            assert np.array_equal(y.download(np.float32, H), plain[it]), it
            assert server.running(), it
    finally:
        for b in [y, nw] + ws:
            b.free()


def test_server_block_rejects_bad_arguments(ctx, server):
    K, H, F = 512, 512, 512
    _, ws = block_weights(ctx, K, H, F, seed=80)
    nw = ctx.to_device(np.ones(H, np.float32))
    y = ctx.alloc(4 * H)
    try:
        x, r = np.ones(K, np.float32), np.ones(H, np.float32)
        o, g, u, d = (w.ptr for w in ws)
        args = lambda **kw: dict(dict(x=x, w_o=o, resid=r, norm_w=nw.ptr, eps=EPS, w_gate=g, w_up=u, F=F,  # noqa: E731
                                      w_down=d, y=y.ptr), **kw)
        call = lambda **kw: server.block_ptr(**args(**kw))  # noqa: E731
        assert call(x=x[:500]) == mi355x.EINVAL  # K % 256
        assert call(resid=r[:500]) == mi355x.EINVAL  # H % 256
        assert call(F=500) == mi355x.EINVAL
        assert call(resid=np.ones(4352, np.float32)) == mi355x.EINVAL  # H > 4096
        assert call(x=np.ones(16384, np.float32)) == mi355x.EINVAL  # K + H > max_k
        assert call(w_o=o + 2) == mi355x.EINVAL
        assert call(w_down=d + 8) == mi355x.EINVAL
        assert call(norm_w=0) == mi355x.EINVAL
        assert call(w_next=g, next_norm_w=nw.ptr, N_next=0, y_next=y.ptr) == mi355x.EINVAL
        assert call(w_next=g, next_norm_w=0, N_next=64, y_next=y.ptr) == mi355x.EINVAL
        assert call(w_next=g + 4, next_norm_w=nw.ptr, N_next=64, y_next=y.ptr) == mi355x.EINVAL
        with variant(ctx, mi355x.VARIANT_EXACT_F32):
            assert call() == mi355x.EUNSUPPORTED
        assert call() == mi355x.OK  # still serves
        assert call(resid=H) == mi355x.OK  # the residual that call left
        assert call(resid=2 * H) == mi355x.EINVAL  # none of that length kept
    finally:
        for b in [y, nw] + ws:
            b.free()


def test_server_rejects_bad_arguments(ctx, server):
    N, K = 64, 2048
    w = ctx.resident(Q4_0, synth.random_q4_0(N, K, seed=1), N, K)
    y = ctx.alloc(4 * N)
    try:
        x = np.ones(K, np.float32)
        assert server.gemv_ptr(x[:2016], [(w.ptr, N, y.ptr)]) == mi355x.EINVAL  # K % 256
        assert server.gemv_ptr(np.ones(16640, np.float32), [(w.ptr, N, y.ptr)]) == mi355x.EINVAL  # > max_k
        assert server.gemv_ptr(x, []) == mi355x.EINVAL
        assert server.gemv_ptr(x, [(w.ptr, N, y.ptr)] * 5) == mi355x.EINVAL
        assert server.gemv_ptr(x, [(w.ptr + 2, N, y.ptr)]) == mi355x.EINVAL  # alignment
        assert server.gemv_ptr(x, [(w.ptr, 0, y.ptr)]) == mi355x.EINVAL
        with variant(ctx, mi355x.VARIANT_EXACT_F32):
            assert server.gemv_ptr(x, [(w.ptr, N, y.ptr)]) == mi355x.EUNSUPPORTED
        server.gemv(x, [(w.ptr, N, y.ptr)])  # still serves
    finally:
        y.free()
        w.free()
