"""The ggml plugin on the GPU, driven through its vtables the way
ggml-backend drives a dynamically loaded backend, and through the
compatibility API the reference's own tests use.

Reference cases mirrored: tests/test-backend.cpp:58-105 (compat graph,
128.0), tests/test-gemv-accuracy.cpp:529-621 (4 concurrent callers, no
cross-talk), and the claim/dispatch semantics of src/ggml-xdna.cpp:81-308.
"""
import ctypes as C
import threading
from types import SimpleNamespace

import numpy as np
import pytest

import ggml_host as gh
import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0
RB = lambda K: (K // 32) * 18  # noqa: E731  Q4_0 row bytes


@pytest.fixture(scope="module")
def plugin():
    lib = gh.bind_compat(mi355x.load())
    assert lib.ggml_backend_mi355x_set_op_mul_mat(gh.HOST_OP_MUL_MAT)
    reg = gh.Reg(lib.ggml_backend_init())
    assert reg.call("get_device_count") >= 1
    dev = reg.device(0)
    be = dev.backend()
    assert be is not None
    p = SimpleNamespace(lib=lib, reg=reg, dev=dev, backend=be, buft=dev.buffer_type())
    yield p
    be.free()


def weight_tensor(buf, raw, N, K, name=b"w"):
    w = gh.tensor(Q4_0, [K, N], [18, RB(K), RB(K) * N, RB(K) * N], name)
    buf.place(w, N * RB(K))
    buf.set(w, raw)
    return w


def f32_tensor(buf, arr, ne, name=b"x"):
    ne = list(ne) + [1] * (4 - len(ne))
    t = gh.tensor(gh.TYPE_F32, ne, gh.contiguous_nb(4, 1, ne), name)
    buf.place(t, 4 * int(np.prod(ne)))
    if arr is not None:
        buf.set(t, np.ascontiguousarray(arr, dtype=np.float32))
    return t


def read_f32(buf, t, n):
    return np.frombuffer(buf.get(t, 4 * n), dtype=np.float32).copy()


def test_device_props_and_buffer_types(plugin):
    dev = plugin.dev
    assert dev.call("get_name") == b"MI355X0"
    assert dev.call("get_type") == 1  # GPU
    p = dev.props()
    assert p.type == 1 and p.memory_total > 100 * 2**30 and 0 < p.memory_free <= p.memory_total
    assert p.caps.async_ and p.caps.host_buffer and not p.caps.buffer_from_host_ptr
    assert p.device_id  # PCI bus id
    buft, host = plugin.buft, dev.host_buffer_type()
    assert buft.name() == "MI355X" and not buft.call("is_host")
    assert buft.call("get_alignment") == 256
    assert host.name() == "MI355X_Host" and host.call("is_host")
    assert dev.call("supports_buft", buft.addr) and not dev.call("supports_buft", host.addr)
    w = gh.tensor(Q4_0, [4096, 96], [18, RB(4096), RB(4096) * 96, RB(4096) * 96])
    assert buft.call("get_alloc_size", C.addressof(w)) == 96 * RB(4096)
    assert plugin.lib.ggml_backend_is_mi355x(plugin.backend.addr)
    assert plugin.backend.call("get_name") == b"MI355X0"
    assert plugin.lib.ggml_backend_mi355x_buffer_type(0) == buft.addr


def test_host_buffer_is_pinned_host_memory(plugin):
    buf = plugin.dev.host_buffer_type().alloc(1 << 20)
    try:
        t = f32_tensor(buf, np.arange(256, dtype=np.float32), [256])
        # host memory: readable directly through the data pointer
        direct = np.ctypeslib.as_array((C.c_float * 256).from_address(t.data))
        assert np.array_equal(direct, np.arange(256, dtype=np.float32))
    finally:
        buf.free()


@pytest.mark.parametrize("N,K", [(96, 320), (64, 4160), (40, 32)])
def test_weight_bytes_round_trip(plugin, ctx, N, K):
    """set_tensor prepacks, get_tensor returns the original ggml bytes, for
    whole tensors and arbitrary byte ranges."""
    raw = synth.random_q4_0(N, K, seed=N + K)
    buf = plugin.buft.alloc(N * RB(K) + 4096)
    try:
        w = weight_tensor(buf, raw, N, K)
        assert buf.get(w, raw.nbytes) == raw.tobytes()
        resident = np.empty_like(raw)
        mi355x.check(ctx.lib.mi355x_memcpy_d2h(ctx.h, resident.ctypes.data, w.data, raw.nbytes))
        assert not np.array_equal(resident, raw)  # the device holds the resident layout
        rng = np.random.default_rng(7)
        for _ in range(12):
            off = int(rng.integers(0, raw.nbytes))
            n = int(rng.integers(1, raw.nbytes - off + 1))
            assert buf.get(w, n, off) == raw.tobytes()[off:off + n], (off, n)
        # piecewise upload of a second tensor's bytes in ragged chunks
        raw2 = synth.random_q4_0(N, K, seed=1 + N)
        buf.call("clear", 0)
        off = 0
        while off < raw2.nbytes:
            n = int(rng.integers(1, 97))
            buf.set(w, raw2.tobytes()[off:off + n], off)
            off += n
        assert buf.get(w, raw2.nbytes) == raw2.tobytes()
    finally:
        buf.free()


@pytest.mark.parametrize("N,K", [(36, 256), (4096, 4096), (17408, 5120), (1024, 8192)])
def test_graph_compute_matches_oracle(plugin, oracle, N, K):
    raw = synth.random_q4_0(N, K, seed=11)
    x = synth.activations(K, seed=12)
    buf = plugin.buft.alloc(N * RB(K) + 4 * (K + N) + 3 * 256)
    try:
        w = weight_tensor(buf, raw, N, K)
        xt = f32_tensor(buf, x, [K, 1])
        d = gh.mul_mat(w, xt, [N, 1])
        buf.place(d, 4 * N)
        assert plugin.dev.supports_op(d)
        assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(buf, d, N)
        check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), oracle.row_norms(Q4_0, raw, N, K), x, f"{N}x{K}")
    finally:
        buf.free()


def test_graph_compute_groups_mul_mats_sharing_an_activation(plugin, oracle):
    """Consecutive MUL_MAT nodes that read one activation row (a q|k|v and a
    gate|up group, as a decoder layer's graph has them) go to one
    mi355x_gemv_multi call; a node reading another activation ends a group.
    Every output matches the oracle."""
    K = 2048
    Ns = [2048, 256, 256, 512, 1024]
    raws = [synth.random_q4_0(n, K, seed=40 + i) for i, n in enumerate(Ns)]
    x = synth.activations(K, seed=41)
    x2 = synth.activations(K, seed=42)
    buf = plugin.buft.alloc(sum(n * RB(K) for n in Ns) + 8 * 4 * K + 4 * 8192 + 16 * 256)
    try:
        ws = [weight_tensor(buf, raw, n, K, b"w%d" % i) for i, (raw, n) in enumerate(zip(raws, Ns))]
        xt = f32_tensor(buf, x, [K, 1])
        x2t = f32_tensor(buf, x2, [K, 1], b"x2")
        plan = [(0, xt, x), (1, xt, x), (2, xt, x), (3, x2t, x2), (4, x2t, x2), (0, x2t, x2)]
        nodes = []
        for wi, at, _ in plan:
            d = gh.mul_mat(ws[wi], at, [Ns[wi], 1])
            buf.place(d, 4 * Ns[wi])
            nodes.append(d)
        assert plugin.backend.compute(nodes) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        for (wi, _, a), d in zip(plan, nodes):
            n = Ns[wi]
            check_gemv(read_f32(buf, d, n), oracle.gemv(Q4_0, raws[wi], n, K, a),
                       oracle.row_norms(Q4_0, raws[wi], n, K), a, f"node w{wi}")
    finally:
        buf.free()


def test_supports_op_through_device(plugin):
    N, K = 64, 512
    raw = synth.random_q4_0(N, K, seed=3)
    buf = plugin.buft.alloc(N * RB(K) + 4 * K * 8 + 4 * N * 8 + 1024)
    try:
        w = weight_tensor(buf, raw, N, K)
        x8 = f32_tensor(buf, None, [K, 8])
        d8 = gh.mul_mat(w, x8, [N, 8])
        assert plugin.dev.supports_op(d8)  # weights resident here: M > 1 allowed
        assert not plugin.dev.call("offload_op", C.addressof(d8))
        # weights in a host (CPU) buffer: single-row only
        wh = gh.tensor(Q4_0, [K, N], [18, RB(K), RB(K) * N, RB(K) * N])
        d8h = gh.mul_mat(wh, x8, [N, 8])
        assert not plugin.dev.supports_op(d8h)
        x1 = gh.tensor(gh.TYPE_F32, [K, 1], gh.contiguous_nb(4, 1, [K, 1, 1, 1]))
        assert plugin.dev.supports_op(gh.mul_mat(wh, x1, [N, 1]))
        # the loader's zero-size probe buffer lifts the M == 1 rule (src/ggml-xdna.cpp:81-89)
        probe = (C.c_uint8 * 160)()
        wh.buffer = C.addressof(probe)
        assert plugin.dev.supports_op(gh.mul_mat(wh, x8, [N, 8]))
        # other ops and non-F32 activations are not claimed
        d = gh.mul_mat(w, x8, [N, 8])
        d.op = gh.HOST_OP_RMS_NORM
        assert not plugin.dev.supports_op(d)
        xh = gh.tensor(1, [K, 1], [2, 2 * K, 2 * K, 2 * K])
        assert not plugin.dev.supports_op(gh.mul_mat(w, xh, [N, 1]))
        # size cutoff and alignment
        w30 = gh.tensor(Q4_0, [K, 30], [18, RB(K), RB(K) * 30, RB(K) * 30])
        assert not plugin.dev.supports_op(gh.mul_mat(w30, x1, [30, 1]))
    finally:
        buf.free()


def test_graph_compute_batched_rows_and_broadcast(plugin, oracle):
    N, K, M = 128, 1024, 3
    raw = synth.random_q4_0(N, K, seed=21)
    xs = np.stack([synth.activations(K, seed=30 + m) for m in range(M)])
    buf = plugin.buft.alloc(N * RB(K) + 4 * K * M * 2 + 4 * N * M * 2 + 8 * 256)
    try:
        w = weight_tensor(buf, raw, N, K)
        xt = f32_tensor(buf, xs, [K, M])
        d = gh.mul_mat(w, xt, [N, M])
        buf.place(d, 4 * N * M)
        # ne2 = 2 activation batches against the same weights (src0 broadcast)
        xb = f32_tensor(buf, xs[:2], [K, 1, 2])
        db = gh.mul_mat(w, xb, [N, 1, 2])
        buf.place(db, 4 * N * 2)
        assert plugin.backend.compute([d, db]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(buf, d, N * M).reshape(M, N)
        yb = read_f32(buf, db, N * 2).reshape(2, N)
        norms = oracle.row_norms(Q4_0, raw, N, K)
        for m in range(M):
            check_gemv(y[m], oracle.gemv(Q4_0, raw, N, K, xs[m]), norms, xs[m], f"row {m}")
        for m in range(2):
            check_gemv(yb[m], oracle.gemv(Q4_0, raw, N, K, xs[m]), norms, xs[m], f"batch {m}")
    finally:
        buf.free()


def test_graph_compute_skips_other_ops_and_reports_failures(plugin):
    N, K = 64, 256
    raw = synth.random_q4_0(N, K, seed=2)
    buf = plugin.buft.alloc(N * RB(K) + 4 * K + 4 * N + 1024)
    try:
        w = weight_tensor(buf, raw, N, K)
        xt = f32_tensor(buf, np.ones(K, np.float32), [K, 1])
        other = gh.mul_mat(w, xt, [N, 1])
        other.op = gh.HOST_OP_RMS_NORM  # not ours: skipped
        assert plugin.backend.compute([other]) == gh.STATUS_SUCCESS
        bad = gh.mul_mat(w, xt, [N, 1])
        buf.place(bad, 4 * N)
        bad_x = gh.tensor(1, [K, 1], [2, 2 * K, 2 * K, 2 * K])  # F16 activations
        bad_x.data = xt.data
        bad.src[1] = C.addressof(bad_x)
        assert plugin.backend.compute([bad]) == gh.STATUS_FAILED
        nodata = gh.mul_mat(w, xt, [N, 1])  # dst without memory
        assert plugin.backend.compute([nodata]) == gh.STATUS_FAILED
    finally:
        buf.free()


def test_weight_view_rows(plugin, oracle):
    """A view of rows [64, 128) of a Q4_0 tensor: byte-range set_tensor through
    the view lands in the right resident rows, and the view computes."""
    N, K, r0 = 128, 2112, 64
    raw = synth.random_q4_0(N, K, seed=41)
    new_rows = synth.random_q4_0(N - r0, K, seed=42)
    x = synth.activations(K, seed=43)
    buf = plugin.buft.alloc(N * RB(K) + 4 * K + 4 * N + 1024)
    try:
        w = weight_tensor(buf, raw, N, K)
        v = gh.tensor(Q4_0, [K, N - r0], [18, RB(K), RB(K) * (N - r0), RB(K) * (N - r0)])
        v.buffer, v.view_src, v.view_offs = w.buffer, C.addressof(w), r0 * RB(K)
        v.data = w.data + r0 * RB(K)
        buf.set(v, new_rows)
        want = raw.copy().reshape(N, -1)
        want[r0:] = new_rows.reshape(N - r0, -1)
        assert buf.get(w, raw.nbytes) == want.tobytes()
        assert buf.get(v, 100, 37) == new_rows.tobytes()[37:137]
        xt = f32_tensor(buf, x, [K, 1])
        d = gh.mul_mat(v, xt, [N - r0, 1])
        buf.place(d, 4 * (N - r0))
        assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(buf, d, N - r0)
        check_gemv(y, oracle.gemv(Q4_0, new_rows, N - r0, K, x), oracle.row_norms(Q4_0, new_rows, N - r0, K), x)
    finally:
        buf.free()


def test_memset_clear_and_copy(plugin):
    N, K = 40, 320
    raw = synth.random_q4_0(N, K, seed=5)
    buf = plugin.buft.alloc(3 * N * RB(K) + 8192)
    try:
        a = weight_tensor(buf, raw, N, K, b"a")
        b = weight_tensor(buf, np.zeros_like(raw), N, K, b"b")
        assert buf.call("cpy_tensor", C.addressof(a), C.addressof(b))
        assert buf.get(b, raw.nbytes) == raw.tobytes()
        buf.call("memset_tensor", C.addressof(a), 0x11, 50, 300)
        want = bytearray(raw.tobytes())
        want[50:350] = b"\x11" * 300
        assert buf.get(a, raw.nbytes) == bytes(want)
        f = f32_tensor(buf, np.arange(100, dtype=np.float32), [100])
        g = f32_tensor(buf, None, [100])
        assert buf.call("cpy_tensor", C.addressof(f), C.addressof(g))
        assert np.array_equal(read_f32(buf, g, 100), np.arange(100, dtype=np.float32))
        buf.call("memset_tensor", C.addressof(g), 0, 0, 400)
        assert not read_f32(buf, g, 100).any()
        buf.call("clear", 0)
        assert not read_f32(buf, f, 100).any()
        # clear() zeroes device bytes without tensor knowledge; a cleared Q4_0
        # weight tensor reads back as d = 0 with codes 8 (0x88): all-zero weights
        blocks = np.frombuffer(buf.get(a, raw.nbytes), dtype=np.uint8).reshape(-1, 18)
        assert not blocks[:, :2].any() and (blocks[:, 2:] == 0x88).all()
    finally:
        buf.free()


def test_async_uploads_are_ordered_after_compute(plugin, oracle):
    """Per-token pattern: set x (async), compute, next x, compute, ... with a
    single synchronize at the end; each token's output must use its own x.
    The caller's activation buffers are overwritten right after each
    set_tensor_async (the backend must have taken its own copy), and the
    get_tensor_async destinations are read after synchronize, as ggml's
    contract has it."""
    N, K, T = 4096, 4096, 6
    raw = synth.random_q4_0(N, K, seed=8)
    xs = [synth.activations(K, seed=100 + t) for t in range(T)]
    buf = plugin.buft.alloc(N * RB(K) + 4 * K + T * 4 * N + 16 * 256)
    be = plugin.backend
    try:
        w = weight_tensor(buf, raw, N, K)
        xt = f32_tensor(buf, None, [K, 1])
        outs = []
        src = (C.c_float * K)()
        for t in range(T):
            C.memmove(src, xs[t].ctypes.data, 4 * K)
            be.call("set_tensor_async", C.addressof(xt), C.addressof(src), 0, 4 * K)
            C.memset(src, 0xFF, 4 * K)  # the backend holds its own copy
            d = gh.mul_mat(w, xt, [N, 1])
            buf.place(d, 4 * N)
            assert be.compute([d]) == gh.STATUS_SUCCESS
            outs.append(d)
        dsts = []
        for d in outs:
            dst = (C.c_float * N)()
            be.call("get_tensor_async", C.addressof(d), C.addressof(dst), 0, 4 * N)
            dsts.append(dst)
        be.call("synchronize")
        got = [np.ctypeslib.as_array(dst).copy() for dst in dsts]
        norms = oracle.row_norms(Q4_0, raw, N, K)
        for t in range(T):
            check_gemv(got[t], oracle.gemv(Q4_0, raw, N, K, xs[t]), norms, xs[t], f"token {t}")
    finally:
        buf.free()


# ---- compatibility API (host pointers) ------------------------------------

def compat_mul_mat(raw, N, K, x, out):
    w = gh.CompatTensor(type=Q4_0, data=raw.ctypes.data)
    w.ne[:] = [K, N, 1, 1]
    a = gh.CompatTensor(type=0, data=x.ctypes.data)
    a.ne[:] = [K, 1, 1, 1]
    o = gh.CompatTensor(type=0, op=gh.COMPAT_OP_MUL_MAT, data=out.ctypes.data)
    o.ne[:] = [N, 1, 1, 1]
    o.src[0] = C.addressof(w)
    o.src[1] = C.addressof(a)
    return o, (w, a)


def test_compat_compute_graph_known_answer(plugin):
    # tests/test-backend.cpp:58-100: 128 x 256, qs 0x99, d = 1.0, x = 0.5 -> 128.0
    lib = plugin.lib
    be = lib.ggml_backend_mi355x_init(0)
    assert be and lib.ggml_backend_is_mi355x(be)
    try:
        N, K = 128, 256
        blk = np.array([0x00, 0x3C] + [0x99] * 16, dtype=np.uint8)
        raw = np.tile(blk, N * K // 32)
        x = np.full(K, 0.5, dtype=np.float32)
        out = np.zeros(N, dtype=np.float32)
        o, keep = compat_mul_mat(raw, N, K, x, out)
        assert lib.ggml_backend_mi355x_supports_op(be, C.byref(o))
        nodes = (C.POINTER(gh.CompatTensor) * 1)(C.pointer(o))
        assert lib.ggml_backend_mi355x_compute_graph(be, nodes, 1)
        assert np.array_equal(out, np.full(N, 128.0, dtype=np.float32))
    finally:
        lib.ggml_backend_mi355x_free(be)


def test_compat_four_concurrent_callers(plugin, oracle):
    # tests/test-gemv-accuracy.cpp:529-621: one backend shared by 4 threads,
    # activations t+1, 50 iterations; no errors and no cross-contamination
    lib = plugin.lib
    be = lib.ggml_backend_mi355x_init(0)
    assert be
    N, K, threads, iters = 512, 256, 4, 50
    raw = synth.random_q4_0(N, K, seed=9999)
    expected = [oracle.gemv(Q4_0, raw, N, K, np.full(K, t + 1.0, np.float32)) for t in range(threads)]
    norms = oracle.row_norms(Q4_0, raw, N, K)
    errors, contamination = [], []
    start = threading.Barrier(threads)

    def work(t):
        x = np.full(K, t + 1.0, dtype=np.float32)
        out = np.zeros(N, dtype=np.float32)
        o, keep = compat_mul_mat(raw, N, K, x, out)
        nodes = (C.POINTER(gh.CompatTensor) * 1)(C.pointer(o))
        start.wait()
        for _ in range(iters):
            out[:] = 0
            if not lib.ggml_backend_mi355x_compute_graph(be, nodes, 1):
                errors.append((t, "call failed"))
                continue
            try:
                check_gemv(out, expected[t], norms, x)
            except AssertionError as e:
                errors.append((t, str(e)))
            for other in range(threads):
                if other != t and np.max(np.abs(out - expected[other])) < 1e-3:
                    contamination.append((t, other))

    try:
        ts = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
        for th in ts:
            th.start()
        for th in ts:
            th.join()
    finally:
        lib.ggml_backend_mi355x_free(be)
    assert not errors, errors[:3]
    assert not contamination, contamination[:3]


def test_four_backends_share_resident_weights(plugin, oracle):
    """One stream per backend: 4 backends on 4 threads read one resident
    weight tensor with their own activations and outputs."""
    N, K, threads, iters = 2048, 2048, 4, 20
    raw = synth.random_q4_0(N, K, seed=77)
    xs = [synth.activations(K, seed=200 + t) for t in range(threads)]
    buf = plugin.buft.alloc(N * RB(K) + threads * (4 * K + 4 * N) + 16 * 256)
    backends = [plugin.dev.backend() for _ in range(threads)]
    errors = []
    try:
        w = weight_tensor(buf, raw, N, K)
        xts = [f32_tensor(buf, xs[t], [K, 1]) for t in range(threads)]
        ds = []
        for t in range(threads):
            d = gh.mul_mat(w, xts[t], [N, 1])
            buf.place(d, 4 * N)
            ds.append(d)
        expected = [oracle.gemv(Q4_0, raw, N, K, xs[t]) for t in range(threads)]
        norms = oracle.row_norms(Q4_0, raw, N, K)

        def work(t):
            be = backends[t]
            for _ in range(iters):
                if be.compute([ds[t]]) != gh.STATUS_SUCCESS:
                    errors.append((t, "compute failed"))
                    return
                dst = (C.c_float * N)()
                be.call("get_tensor_async", C.addressof(ds[t]), C.addressof(dst), 0, 4 * N)
                be.call("synchronize")
                try:
                    check_gemv(np.ctypeslib.as_array(dst), expected[t], norms, xs[t])
                except AssertionError as e:
                    errors.append((t, str(e)))

        ts = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
        for th in ts:
            th.start()
        for th in ts:
            th.join()
    finally:
        for be in backends:
            be.free()
        buf.free()
    assert not errors, errors[:3]


# ---- K-quant / IQ weights through the plugin --------------------------------
# The reference claims and dispatches all eight 256-value types through the
# same process_mul_mat_node (src/ggml-xdna.cpp:185-254;
# tests/test-kquants-gemv.cpp:351-414).  Rows of an odd number of superblocks
# of the 2-mod-4 block sizes (Q3_K, Q6_K, IQ3_S, IQ3_XXS, IQ2_S) start 2 mod 4
# on odd rows, where the resident layout moves the fp16 plane to the front.

KQ = {"Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23, "IQ3_S": 21, "IQ3_XXS": 18, "IQ2_S": 22}


def iq_grid(t):
    # the synthetic grids the other K/IQ GPU tests install (process-wide)
    rng = np.random.default_rng(t)
    n, w = (256, 4) if t == 18 else (1024, 8)
    g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


def kq_weight(buf, t, raw, N, K, name=b"wk"):
    bb = mi355x.BLOCK_BYTES[t]
    rb = mi355x.row_bytes(t, K)
    w = gh.tensor(t, [K, N], [bb, rb, rb * N, rb * N], name)
    buf.place(w, N * rb)
    return w


@pytest.mark.parametrize("name", list(KQ))
def test_kq_weights_set_get_compute_and_views(plugin, oracle, name):
    t = KQ[name]
    grid = iq_grid(t) if t in (18, 22) else None
    if grid is not None:
        mi355x.set_iq_grid(t, grid)
    N, K, r0 = 64, 256 * 3, 9  # odd superblock count; a view from an odd row
    rb = mi355x.row_bytes(t, K)
    raw = synth.random_blocks(t, N, K, seed=t)
    new_rows = synth.random_blocks(t, N - r0, K, seed=t + 100)
    x = synth.activations(K, seed=t + 1)
    buf = plugin.buft.alloc(N * rb + 8 * K + 8 * N + 8 * 256)
    try:
        w = kq_weight(buf, t, raw, N, K)
        # ragged byte-range uploads, then whole and partial read-backs
        rng = np.random.default_rng(t)
        off = 0
        while off < raw.nbytes:
            n = int(rng.integers(1, 300))
            buf.set(w, raw.tobytes()[off:off + n], off)
            off += n
        assert buf.get(w, raw.nbytes) == raw.tobytes()
        for _ in range(6):
            o = int(rng.integers(0, raw.nbytes))
            n = int(rng.integers(1, raw.nbytes - o + 1))
            assert buf.get(w, n, o) == raw.tobytes()[o:o + n], (o, n)
        assert plugin.dev.supports_op(gh.mul_mat(w, f32_tensor(buf, None, [K, 1], b"probe"), [N, 1]))
        xt = f32_tensor(buf, x, [K, 1])
        d = gh.mul_mat(w, xt, [N, 1])
        buf.place(d, 4 * N)
        assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(buf, d, N)
        check_gemv(y, oracle.gemv(t, raw, N, K, x, grid=grid), oracle.row_norms(t, raw, N, K, grid=grid), x,
                   f"{name} plugin")
        # a row view from odd row r0: set_tensor through the view lands in
        # the right resident rows, get_tensor through it reads them back, and
        # the view computes
        v = gh.tensor(t, [K, N - r0], [mi355x.BLOCK_BYTES[t], rb, rb * (N - r0), rb * (N - r0)])
        v.buffer, v.view_src, v.view_offs = w.buffer, C.addressof(w), r0 * rb
        v.data = w.data + r0 * rb
        buf.set(v, new_rows)
        want = raw.copy().reshape(N, -1)
        want[r0:] = new_rows.reshape(N - r0, -1)
        assert buf.get(w, raw.nbytes) == want.tobytes()
        assert buf.get(v, 77, 13) == new_rows.tobytes()[13:90]
        dv = gh.mul_mat(v, xt, [N - r0, 1])
        buf.place(dv, 4 * (N - r0))
        assert plugin.backend.compute([dv]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        yv = read_f32(buf, dv, N - r0)
        check_gemv(yv, oracle.gemv(t, new_rows, N - r0, K, x, grid=grid),
                   oracle.row_norms(t, new_rows, N - r0, K, grid=grid), x, f"{name} view")
    finally:
        buf.free()


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "IQ4_XS"])
def test_kq_batched_rows_through_plugin(plugin, oracle, name):
    """M = 3 activation rows against K/IQ weights in this buffer (M sequential
    GEMVs, as the reference's loop)."""
    t = KQ[name]
    N, K, M = 128, 1024, 3
    rb = mi355x.row_bytes(t, K)
    raw = synth.random_blocks(t, N, K, seed=5)
    xs = np.stack([synth.activations(K, seed=60 + m) for m in range(M)])
    buf = plugin.buft.alloc(N * rb + 4 * K * M + 4 * N * M + 4 * 256)
    try:
        w = kq_weight(buf, t, raw, N, K)
        buf.set(w, raw)
        xt = f32_tensor(buf, xs, [K, M])
        d = gh.mul_mat(w, xt, [N, M])
        buf.place(d, 4 * N * M)
        assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(buf, d, N * M).reshape(M, N)
        norms = oracle.row_norms(t, raw, N, K)
        for m in range(M):
            check_gemv(y[m], oracle.gemv(t, raw, N, K, xs[m]), norms, xs[m], f"{name} row {m}")
    finally:
        buf.free()


@pytest.mark.parametrize("group_mode,entry,nodes", [(gh.GROUPS_LAUNCH, "mi355x_gemv", 1),
                                                    (gh.GROUPS_LAUNCH, "mi355x_gemv_multi", 2),
                                                    (gh.GROUPS_SERVER, "mi355x_server_gemv", 2)])
def test_injected_device_error_fails_the_graph_then_recovers(plugin, oracle, group_mode, entry, nodes):
    """A HIP error on the real device (injected at the C-ABI before any
    device work, so no GPU fault) makes graph_compute return
    GGML_STATUS_FAILED (src/ggml-xdna.cpp:299-305, 803-807); the next graph
    on the same backend computes the right answer."""
    N, K = 256, 2048
    raw = synth.random_q4_0(N, K, seed=5)
    x = synth.activations(K, seed=6)
    buf = plugin.buft.alloc(N * RB(K) + 4 * (K + 2 * N) + 4 * 256)
    try:
        w = weight_tensor(buf, raw, N, K)
        xt = f32_tensor(buf, x, [K, 1])
        ds = [gh.mul_mat(w, xt, [N, 1], name=f"d{i}".encode()) for i in range(nodes)]
        for d in ds:
            buf.place(d, 4 * N)
        assert plugin.lib.ggml_backend_mi355x_set_group_mode(plugin.backend.addr, group_mode)
        mi355x.inject_fault(entry, mi355x.HIP_ERROR_LAUNCH_FAILURE)
        assert plugin.backend.compute(ds) == gh.STATUS_FAILED
        assert plugin.backend.compute(ds) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        ref = oracle.gemv(Q4_0, raw, N, K, x)
        for d in ds:
            check_gemv(read_f32(buf, d, N), ref, oracle.row_norms(Q4_0, raw, N, K), x, "after the injected error")
    finally:
        mi355x.inject_fault(None)
        plugin.lib.ggml_backend_mi355x_set_group_mode(plugin.backend.addr, gh.GROUPS_LAUNCH)
        buf.free()
