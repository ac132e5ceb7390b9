"""Persistent Q4_0 GEMV server (mi355x_server_*): a resident kernel that takes
GEMV commands through pinned host memory, for decode loops.  Every output is
bit-identical to the row form (MI355X_FORM_ROWS) on the same inputs and within
the GEMV tolerance of the oracle; commands run back to back, with several
jobs per command, outputs in device or pinned host memory, across stops,
idle relaunches and rejected arguments."""
import ctypes
import time

import numpy as np
import pytest

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
# columns per lane, with and without a partial last column, tiny N
SHAPES = [(2560, 2048), (2048, 2048), (22016, 2048), (2048, 11008), (151936, 2048), (300, 4096), (777, 5120),
          (513, 8192), (64, 14336), (200, 16384), (3, 2048), (255, 256)]


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


def test_server_several_jobs_and_back_to_back_commands(ctx, server):
    K = 2048
    shapes = [700, 64, 3000, 129]
    raws = [synth.random_q4_0(N, K, seed=10 + i) for i, N in enumerate(shapes)]
    ws = [ctx.resident(Q4_0, r, N, K) for r, N in zip(raws, shapes)]
    try:
        for it in range(60):
            x = synth.activations(K, seed=500 + it)
            sel = ws[it % 4:] + ws[:it % 4]
            sel = sel[:1 + it % 4]
            ys = run_server(ctx, server, sel, x)
            for w, y in zip(sel, ys):
                assert np.array_equal(y, rows_form(ctx, w, x)), (it, w.N)
    finally:
        for w in ws:
            w.free()


def test_server_pinned_outputs(ctx, server):
    hip = ctypes.CDLL("libamdhip64.so")
    N, K = 4096, 2048
    raw = synth.random_q4_0(N, K, seed=77)
    w = ctx.resident(Q4_0, raw, N, K)
    hptr = ctypes.c_void_p()
    mi355x.check(ctx.lib.mi355x_host_malloc(4 * N, ctypes.byref(hptr)))
    dptr = ctypes.c_void_p()
    try:
        assert hip.hipHostGetDevicePointer(ctypes.byref(dptr), hptr, 0) == 0
        host_y = np.ctypeslib.as_array(ctypes.cast(hptr, ctypes.POINTER(ctypes.c_float)), shape=(N,))
        for it in range(30):
            x = synth.activations(K, seed=900 + it)
            host_y[:] = np.nan
            server.gemv(x, [(w.ptr, N, dptr.value)])
            assert np.array_equal(host_y, rows_form(ctx, w, x)), it
    finally:
        mi355x.check(ctx.lib.mi355x_host_free(hptr))
        w.free()


def test_server_stop_and_idle_relaunch(ctx, server):
    N, K = 1000, 4096
    raw = synth.random_q4_0(N, K, seed=3)
    w = ctx.resident(Q4_0, raw, N, K)
    try:
        x = synth.activations(K, seed=4)
        ref = rows_form(ctx, w, x)
        (a,) = run_server(ctx, server, [w], x)
        server.stop()
        (b,) = run_server(ctx, server, [w], x)  # relaunch after a stop
        time.sleep(0.7)  # past the host's idle limit: stop and relaunch inside the call
        (c,) = run_server(ctx, server, [w], x)
        time.sleep(2.5)  # past the kernel's own idle exit
        (d,) = run_server(ctx, server, [w], x)
        for y in (a, b, c, d):
            assert np.array_equal(y, ref)
    finally:
        w.free()


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
        server.gemv(x, [(w.ptr, N, y.ptr)])  # still serves
    finally:
        y.free()
        w.free()
