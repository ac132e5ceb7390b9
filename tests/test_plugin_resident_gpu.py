"""Host-resident small tensors of the plugin's non-weight buffers on the
GPU: an activation row and a group's outputs live in the buffer's
page-locked shadow, graph_compute reads and writes them there (as a command
to the device's persistent GEMV server, or as one launch), and every other
access sees the same bytes.  Results are checked against the oracle (ggml-cpu
numerics: bit for bit), in both group modes."""
import ctypes as C
from types import SimpleNamespace

import numpy as np
import pytest

import ggml_host as gh
import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0
RB = lambda K: (K // 32) * 18  # noqa: E731


@pytest.fixture(scope="module")
def plugin():
    lib = gh.bind_compat(mi355x.load())
    assert lib.ggml_backend_mi355x_set_op_mul_mat(gh.HOST_OP_MUL_MAT)
    reg = gh.Reg(lib.ggml_backend_init())
    dev = reg.device(0)
    be = dev.backend()
    p = SimpleNamespace(lib=lib, dev=dev, backend=be, buft=dev.buffer_type())
    yield p
    be.free()


def mode(plugin, m, variant=mi355x.VARIANT_AUTO):
    assert plugin.lib.ggml_backend_mi355x_set_group_mode(plugin.backend.addr, m)
    assert plugin.lib.ggml_backend_mi355x_set_kernel_variant(plugin.backend.addr, variant)


def weights_buffer(plugin, raws_and_shapes):
    """A WEIGHTS buffer holding Q4_0 matrices (as llama.cpp keeps them)."""
    total = sum(n * RB(k) + 256 for _, n, k in raws_and_shapes)
    buf = plugin.buft.alloc(total)
    buf.set_usage(gh.USAGE_WEIGHTS)
    ws = []
    for i, (raw, n, k) in enumerate(raws_and_shapes):
        w = gh.tensor(Q4_0, [k, n], [18, RB(k), RB(k) * n, RB(k) * n], b"w%d" % i)
        buf.place(w, n * RB(k))
        buf.set(w, raw)
        ws.append(w)
    return buf, ws


def f32_tensor(buf, arr, ne, name=b"t"):
    ne = list(ne) + [1] * (4 - len(ne))
    t = gh.tensor(gh.TYPE_F32, ne, gh.contiguous_nb(4, 1, ne), name)
    buf.place(t, 4 * int(np.prod(ne)))
    if arr is not None:
        buf.set(t, np.ascontiguousarray(arr, dtype=np.float32))
    return t


def device_bytes(ctx, t, n):
    out = np.empty(n, np.uint8)
    mi355x.check(ctx.lib.mi355x_memcpy_d2h(ctx.h, out.ctypes.data, t.data, n))
    return out


def read_f32(buf, t, n):
    return np.frombuffer(buf.get(t, 4 * n), dtype=np.float32).copy()


def test_small_tensor_lives_in_the_shadow_until_the_device_needs_it(plugin, ctx):
    cbuf = plugin.buft.alloc(1 << 16)
    try:
        cbuf.set_usage(gh.USAGE_COMPUTE)
        cbuf.call("clear", 0)
        a = f32_tensor(cbuf, None, [1000], b"a")
        b = f32_tensor(cbuf, None, [1000], b"b")
        v = np.arange(1000, dtype=np.float32) + 0.5
        cbuf.set(a, v)
        assert np.array_equal(read_f32(cbuf, a, 1000), v)
        assert not device_bytes(ctx, a, 4000).any()          # the device copy is stale (cleared)
        # a partial write lands in the shadow too
        cbuf.set(a, np.full(10, -1.0, np.float32), offset=40)
        v[10:20] = -1.0
        assert np.array_equal(read_f32(cbuf, a, 1000), v)
        # a device-to-device copy needs the device bytes: a is copied down first
        assert cbuf.call("cpy_tensor", C.addressof(a), C.addressof(b))
        assert np.array_equal(device_bytes(ctx, a, 4000).view(np.float32), v)
        assert np.array_equal(read_f32(cbuf, b, 1000), v)
        # memset of a small tensor: shadow again
        cbuf.call("memset_tensor", C.addressof(b), 0, 400, 400)
        v2 = v.copy()
        v2[100:200] = 0.0
        assert np.array_equal(read_f32(cbuf, b, 1000), v2)
        # clear: device fill, nothing host-resident any more
        cbuf.call("clear", 0)
        assert not read_f32(cbuf, a, 1000).any() and not read_f32(cbuf, b, 1000).any()
    finally:
        cbuf.free()


def test_weight_buffers_have_no_shadow(plugin, ctx):
    buf = plugin.buft.alloc(1 << 16)
    try:
        buf.set_usage(gh.USAGE_WEIGHTS)
        t = f32_tensor(buf, np.arange(256, dtype=np.float32), [256])
        assert np.array_equal(device_bytes(ctx, t, 1024).view(np.float32), np.arange(256, dtype=np.float32))
    finally:
        buf.free()


@pytest.mark.parametrize("group_mode", [gh.GROUPS_SERVER, gh.GROUPS_LAUNCH])
@pytest.mark.parametrize("variant", [mi355x.VARIANT_AUTO, mi355x.VARIANT_GGML_Q8])
def test_decode_layer_groups(plugin, oracle, group_mode, variant):
    """A decoder layer's MUL_MATs as ggml-backend hands them over: q|k|v
    (one activation, three nodes), o, gate|up, down, and a chained pair
    (the second node reads the first one's host-resident output) -- every
    output against the oracle, in both group modes."""
    H, F, KV = 2048, 5632, 256
    shapes = [(H, H), (KV, H), (KV, H), (H, H), (F, H), (F, H), (H, F), (1024, H)]
    raws = [synth.random_q4_0(n, k, seed=300 + i) for i, (n, k) in enumerate(shapes)]
    wbuf, ws = weights_buffer(plugin, [(r, n, k) for r, (n, k) in zip(raws, shapes)])
    cbuf = plugin.buft.alloc(1 << 22)
    cbuf.set_usage(gh.USAGE_COMPUTE)
    be = plugin.backend
    try:
        mode(plugin, group_mode, variant)
        x = synth.activations(H, seed=7)
        x2 = synth.activations(H, seed=8)
        x3 = synth.activations(F, seed=9)
        xt, x2t, x3t = f32_tensor(cbuf, None, [H, 1], b"x"), f32_tensor(cbuf, None, [H, 1], b"x2"), \
            f32_tensor(cbuf, None, [F, 1], b"x3")
        def node(i, src, name):
            d = gh.mul_mat(ws[i], src, [shapes[i][0], 1], name=name)
            cbuf.place(d, 4 * shapes[i][0])
            return d
        q, k, v = node(0, xt, b"q"), node(1, xt, b"k"), node(2, xt, b"v")
        o = node(3, x2t, b"o")
        g, u = node(4, xt, b"g"), node(5, xt, b"u")
        dn = node(6, x3t, b"down")
        chain = node(7, q, b"chain")  # reads q's output
        graphs = [([q, k, v], xt, x), ([o], x2t, x2), ([g, u], xt, x), ([dn], x3t, x3)]
        got = {}
        for nodes, at, a in graphs:
            be.call("set_tensor_async", C.addressof(at), a.ctypes.data, 0, a.nbytes)
            assert be.compute(nodes) == gh.STATUS_SUCCESS
            for d in nodes:
                dst = np.empty(d.ne[0], np.float32)
                be.call("get_tensor_async", C.addressof(d), dst.ctypes.data, 0, dst.nbytes)
                got[d.name] = dst
            be.call("synchronize")
        be.call("set_tensor_async", C.addressof(xt), x.ctypes.data, 0, x.nbytes)
        assert be.compute([q, chain]) == gh.STATUS_SUCCESS
        be.call("synchronize")
        yq = read_f32(cbuf, q, H)
        ych = read_f32(cbuf, chain, 1024)
        inputs = {b"q": x, b"k": x, b"v": x, b"o": x2, b"g": x, b"u": x, b"down": x3}
        idx = {b"q": 0, b"k": 1, b"v": 2, b"o": 3, b"g": 4, b"u": 5, b"down": 6}
        ggml = variant == mi355x.VARIANT_GGML_Q8
        for name, y in list(got.items()) + [(b"q", yq)]:
            i = idx[name]
            n, kk = shapes[i]
            if ggml:
                assert np.array_equal(y, oracle.gemv_q4_0_q8_0(raws[i], n, kk, inputs[name])), name
            else:
                check_gemv(y, oracle.gemv(Q4_0, raws[i], n, kk, inputs[name]), oracle.row_norms(Q4_0, raws[i], n, kk),
                           inputs[name], name.decode())
        if ggml:
            assert np.array_equal(ych, oracle.gemv_q4_0_q8_0(raws[7], 1024, H, yq))
        else:
            check_gemv(ych, oracle.gemv(Q4_0, raws[7], 1024, H, yq), oracle.row_norms(Q4_0, raws[7], 1024, H), yq,
                       "chain")
    finally:
        mode(plugin, gh.GROUPS_LAUNCH)
        cbuf.free()
        wbuf.free()


def test_modes_are_bit_identical_in_ggml_numerics(plugin):
    """GGML_Q8 rows are summed in block order by one lane: the server and the
    launch give the same bits."""
    N, K = 4096, 2048
    raw = synth.random_q4_0(N, K, seed=12)
    wbuf, (w,) = weights_buffer(plugin, [(raw, N, K)])
    cbuf = plugin.buft.alloc(1 << 20)
    cbuf.set_usage(gh.USAGE_COMPUTE)
    try:
        x = synth.activations(K, seed=13)
        xt = f32_tensor(cbuf, x, [K, 1])
        d = gh.mul_mat(w, xt, [N, 1])
        cbuf.place(d, 4 * N)
        outs = []
        for m in (gh.GROUPS_SERVER, gh.GROUPS_LAUNCH, gh.GROUPS_SERVER):
            mode(plugin, m, mi355x.VARIANT_GGML_Q8)
            assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
            outs.append(read_f32(cbuf, d, N))
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    finally:
        mode(plugin, gh.GROUPS_LAUNCH)
        cbuf.free()
        wbuf.free()


def test_large_outputs_and_batched_nodes_use_device_memory(plugin, ctx, oracle):
    """An output above the host-resident size (1 MiB) is written to the
    device; an M = 2 node reading a host-resident activation gets it copied
    down first."""
    N, K = 300000, 256
    raw = synth.random_q4_0(N, K, seed=21)
    raw2 = synth.random_q4_0(64, 512, seed=22)
    wbuf, (w, w2) = weights_buffer(plugin, [(raw, N, K), (raw2, 64, 512)])
    cbuf = plugin.buft.alloc(8 << 20)
    cbuf.set_usage(gh.USAGE_COMPUTE)
    try:
        mode(plugin, gh.GROUPS_SERVER)
        x = synth.activations(K, seed=23)
        xt = f32_tensor(cbuf, x, [K, 1])
        d = gh.mul_mat(w, xt, [N, 1])
        cbuf.place(d, 4 * N)
        assert plugin.backend.compute([d]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y = read_f32(cbuf, d, N)
        assert np.array_equal(device_bytes(ctx, d, 4 * N).view(np.float32), y)
        check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), oracle.row_norms(Q4_0, raw, N, K), x, "large output")
        # M = 2 reading a host-resident [512, 2] activation
        xs = np.stack([synth.activations(512, seed=24), synth.activations(512, seed=25)])
        x2t = f32_tensor(cbuf, xs, [512, 2], b"x2")
        d2 = gh.mul_mat(w2, x2t, [64, 2], name=b"m2")
        cbuf.place(d2, 4 * 128)
        assert plugin.backend.compute([d2]) == gh.STATUS_SUCCESS
        plugin.backend.call("synchronize")
        y2 = read_f32(cbuf, d2, 128).reshape(2, 64)
        norms = oracle.row_norms(Q4_0, raw2, 64, 512)
        for m in range(2):
            check_gemv(y2[m], oracle.gemv(Q4_0, raw2, 64, 512, xs[m]), norms, xs[m], f"M=2 row {m}")
    finally:
        mode(plugin, gh.GROUPS_LAUNCH)
        cbuf.free()
        wbuf.free()


def test_server_and_launched_kernels_alternate(plugin, oracle):
    """Q4_0 groups go to the server, a Q4_K node is launched (the server
    leaves the CUs first), then Q4_0 again: all correct, in one graph and
    across graphs."""
    H = 2048
    raw = synth.random_q4_0(H, H, seed=31)
    rawk = synth.random_blocks(12, 512, H, seed=32)
    wbuf = plugin.buft.alloc(H * RB(H) + 512 * mi355x.row_bytes(12, H) + 1024)
    wbuf.set_usage(gh.USAGE_WEIGHTS)
    cbuf = plugin.buft.alloc(1 << 20)
    cbuf.set_usage(gh.USAGE_COMPUTE)
    try:
        mode(plugin, gh.GROUPS_SERVER)
        w = gh.tensor(Q4_0, [H, H], [18, RB(H), RB(H) * H, RB(H) * H], b"w")
        wbuf.place(w, H * RB(H))
        wbuf.set(w, raw)
        rbk = mi355x.row_bytes(12, H)
        wk = gh.tensor(12, [H, 512], [144, rbk, rbk * 512, rbk * 512], b"wk")
        wbuf.place(wk, 512 * rbk)
        wbuf.set(wk, rawk)
        x = synth.activations(H, seed=33)
        xt = f32_tensor(cbuf, x, [H, 1])
        d1 = gh.mul_mat(w, xt, [H, 1], name=b"d1")
        cbuf.place(d1, 4 * H)
        dk = gh.mul_mat(wk, xt, [512, 1], name=b"dk")
        cbuf.place(dk, 4 * 512)
        d2 = gh.mul_mat(w, d1, [H, 1], name=b"d2")
        cbuf.place(d2, 4 * H)
        for _ in range(3):
            assert plugin.backend.compute([d1, dk, d2]) == gh.STATUS_SUCCESS
            plugin.backend.call("synchronize")
        y1, yk, y2 = read_f32(cbuf, d1, H), read_f32(cbuf, dk, 512), read_f32(cbuf, d2, H)
        n0 = oracle.row_norms(Q4_0, raw, H, H)
        check_gemv(y1, oracle.gemv(Q4_0, raw, H, H, x), n0, x, "q4_0 first")
        check_gemv(yk, oracle.gemv(12, rawk, 512, H, x), oracle.row_norms(12, rawk, 512, H), x, "q4_k")
        check_gemv(y2, oracle.gemv(Q4_0, raw, H, H, y1), n0, y1, "q4_0 chained")
    finally:
        mode(plugin, gh.GROUPS_LAUNCH)
        cbuf.free()
        wbuf.free()


def test_views_partial_overlaps_and_large_fills(plugin, ctx):
    """Writes through views (parts of a tensor become host-resident), a
    device-side copy into another part, and fills larger than the
    host-resident size: every read returns the last write, byte for byte."""
    cbuf = plugin.buft.alloc(8 << 20)
    try:
        cbuf.set_usage(gh.USAGE_COMPUTE)
        cbuf.call("clear", 0)
        n = 4096
        base = f32_tensor(cbuf, None, [n], b"base")
        want = np.zeros(n, np.float32)
        # views of 256 floats at a few offsets, written through set_tensor
        for i, off in enumerate((0, 1000, 3840)):
            v = gh.tensor(gh.TYPE_F32, [256], gh.contiguous_nb(4, 1, [256, 1, 1, 1]), b"view")
            v.buffer, v.data, v.view_src = base.buffer, base.data + 4 * off, C.addressof(base)
            vals = np.arange(256, dtype=np.float32) + 1000 * (i + 1)
            cbuf.call("set_tensor", C.addressof(v), vals.ctypes.data, 0, vals.nbytes)
            want[off:off + 256] = vals
        assert np.array_equal(read_f32(cbuf, base, n), want)
        # a device-to-device copy into [2000, 2256) from a host-resident tensor
        src = f32_tensor(cbuf, -np.ones(256, np.float32), [256], b"src")
        dv = gh.tensor(gh.TYPE_F32, [256], gh.contiguous_nb(4, 1, [256, 1, 1, 1]), b"dview")
        dv.buffer, dv.data, dv.view_src = base.buffer, base.data + 4 * 2000, C.addressof(base)
        assert cbuf.call("cpy_tensor", C.addressof(src), C.addressof(dv))
        want[2000:2256] = -1.0
        assert np.array_equal(read_f32(cbuf, base, n), want)
        # odd-sized byte ranges straddling host-resident and device parts
        raw = np.frombuffer(cbuf.get(base, 4 * n), np.uint8)
        for off, size in ((3, 5), (990 * 4 + 1, 40 * 4), (3839 * 4, 8), (0, 4 * n)):
            assert cbuf.get(base, size, off) == raw[off:off + size].tobytes(), (off, size)
        # a fill of a tensor above 1 MiB goes to the device and covers the
        # host-resident ranges inside it
        big = f32_tensor(cbuf, None, [300000], b"big")
        small = gh.tensor(gh.TYPE_F32, [100], gh.contiguous_nb(4, 1, [100, 1, 1, 1]), b"in_big")
        small.buffer, small.data, small.view_src = big.buffer, big.data + 4 * 5000, C.addressof(big)
        cbuf.call("set_tensor", C.addressof(small), np.full(100, 7.0, np.float32).ctypes.data, 0, 400)
        cbuf.call("memset_tensor", C.addressof(big), 0, 0, 4 * 300000)
        assert not read_f32(cbuf, small, 100).any()
        assert not device_bytes(ctx, big, 4 * 300000).any()
    finally:
        cbuf.free()


def test_usage_set_after_allocation(plugin, ctx):
    """ggml allocates a buffer, then marks it WEIGHTS: a buffer marked before
    its first write never gets a shadow (its small tensors are device bytes
    from the first write on)."""
    buf = plugin.buft.alloc(1 << 16)
    try:
        buf.set_usage(gh.USAGE_WEIGHTS)
        t = f32_tensor(buf, np.full(64, 3.0, np.float32), [64], b"bias")
        assert np.array_equal(device_bytes(ctx, t, 256).view(np.float32), np.full(64, 3.0, np.float32))
    finally:
        buf.free()
