"""The end-to-end decode harness on the CPU (callback backend): its weight
quantizer against the Q4_0 recipe pinned elsewhere, its forward pass against
an independent float64 numpy Qwen2 decoder, and its error paths."""
from fractions import Fraction

import numpy as np
import pytest

import decode
import oracle as orc
import synth
from qwen2_numpy import Qwen2Numpy, dequantized

TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000,
            rope_theta=1e6, norm_eps=1e-6, seed=7)
# a second shape: one KV head for four query heads, other theta/eps
TINY_MQA = dict(n_layers=3, hidden=128, n_heads=4, n_kv_heads=1, head_dim=32, ffn=320, vocab=500,
                rope_theta=1e4, norm_eps=1e-5, seed=11)


def test_quantizer_matches_q4_0_recipe():
    w = synth.normal_weights(64, 1024, seed=3)
    w[5, :32] = 0.0          # all-zero block: d = 0
    w[6, 40] = 1.0           # positive absmax: d < 0
    w[7, 64:96] *= 1e-3      # tiny block: d is a subnormal half
    assert np.array_equal(decode.quantize_q4_0(w).reshape(-1), synth.quantize_q4_0(w).reshape(-1))


@pytest.mark.parametrize("cfg", [TINY, TINY_MQA], ids=["gqa2", "mqa"])
def test_forward_matches_numpy_qwen2(oracle, cfg):
    with decode.Model(threads=4, **cfg) as m:
        ref = Qwen2Numpy(m, oracle)
        p = decode.prompt_tokens(10, cfg["vocab"], 3)
        f, _ = orc.decode_gemv("oracle")
        toks, t = m.generate(p, 6, f)
        rt, rl = ref.generate(p, 6)
        assert np.array_equal(toks, rt)
        lg = m.last_logits()
        assert np.abs(lg - rl).max() <= 1e-5 * np.abs(rl).max()
        assert t["gen_passes"] == 5 and t["gen_s"] > 0


# long enough for the threaded attention (>= 64 positions: two 64-position
# score blocks, the second partial), 12 query heads on one KV head (blocks of
# 8 and 4 heads) and a head dimension of 5 eight-wide slices
LONG = dict(n_layers=2, hidden=480, n_heads=12, n_kv_heads=1, head_dim=40, ffn=256, vocab=300,
            rope_theta=1e4, norm_eps=1e-6, seed=5)


def test_long_context_matches_numpy_and_thread_count(oracle):
    p = decode.prompt_tokens(70, LONG["vocab"], 4)
    f, _ = orc.decode_gemv("oracle")
    runs = []
    for threads in (1, 5):
        with decode.Model(threads=threads, **LONG) as m:
            runs.append((m.generate(p, 5, f)[0], m.last_logits()))
            if threads == 1:
                rt, rl = Qwen2Numpy(m, oracle).generate(p, 5)
    assert np.array_equal(runs[0][0], rt)
    assert np.abs(runs[0][1] - rl).max() <= 1e-5 * np.abs(rl).max()
    # the attention's split of the work does not depend on the team size
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1])


def test_model_shapes_and_vectors():
    with decode.Model(threads=2, **TINY) as m:
        assert m.n_matrices() == 7 * 2 + 1
        H, Q, KV, F = 256, 4 * 64, 2 * 64, 512
        want = [(Q, H), (KV, H), (KV, H), (H, Q), (F, H), (F, H), (H, F)] * 2 + [(1000, H)]
        assert [m.matrix(i)[1:] for i in range(m.n_matrices())] == want
        assert np.all(m.vector(0) == 1.0) and np.all(m.vector(5 * 2) == 1.0)
        b = m.vector(2)
        assert b.shape == (Q,) and 0.01 < b.std() < 0.04
        with pytest.raises(IndexError):
            m.vector(5 * 2 + 1)


def test_weights_are_normal_0_02(oracle):
    with decode.Model(threads=4, **TINY) as m:
        w = dequantized(m, oracle, 4).reshape(-1)  # gate, 512 x 256
        assert abs(w.mean()) < 5e-4 and 0.0195 < w.std() < 0.0205
        # fourth moment of a normal: 3 sigma^4 (a uniform or clipped generator fails this)
        assert 2.8 < np.mean(w ** 4) / w.var() ** 2 < 3.2


def test_reference_engine_callback_agrees(reflib, oracle):
    with decode.Model(threads=4, **TINY) as m:
        p = decode.prompt_tokens(12, 1000, 9)
        out = {}
        for kind in ("oracle", "reference"):
            f, _ = orc.decode_gemv(kind)
            out[kind] = (m.generate(p, 8, f)[0], m.last_logits())
        assert np.array_equal(out["oracle"][0], out["reference"][0])
        a, b = (v[1].astype(np.float64) for v in out.values())
        assert np.dot(a, b) / np.linalg.norm(a) / np.linalg.norm(b) >= 0.999999


def test_seeded_weights_are_reproducible():
    with decode.Model(threads=3, **TINY) as a, decode.Model(threads=1, **TINY) as b:
        for i in (0, 6, 14):
            pa, N, K = a.matrix(i)
            pb, _, _ = b.matrix(i)
            n = N * (K // 32) * 18
            assert bytes((decode.C.c_uint8 * n).from_address(pa)) == bytes((decode.C.c_uint8 * n).from_address(pb))


def test_errors():
    with pytest.raises(RuntimeError, match="invalid configuration"):
        decode.Model(**dict(TINY, hidden=250))
    with decode.Model(threads=1, **TINY) as m:
        with pytest.raises(RuntimeError, match="qd_attach_gpu first"):
            m.generate(np.array([1, 2], dtype=np.int32), 2)

        def bad(*a):
            raise ValueError("boom")
        with pytest.raises(RuntimeError, match="GEMV failed"):
            m.generate(np.array([1, 2], dtype=np.int32), 2, bad)


# ---- the SwiGLU step shared by the host and mi355x_server_swiglu ------------
def _round_f32(q: Fraction) -> np.float32:
    """q rounded to the nearest f32, ties to even (exact, no double rounding)."""
    f = np.float32(float(q))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - q)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return best[1]


def _q(v) -> Fraction:
    return Fraction(float(v))


def _silu_mul_steps(g: np.float32, u: np.float32) -> np.float32:
    """The stated f32 steps (mi355x-gemv.h, mi355x_server_swiglu), each
    rounded exactly once."""
    fma = lambda a, b, c: _round_f32(_q(a) * _q(b) + _q(c))  # noqa: E731
    lit = lambda s: _round_f32(Fraction(s))  # noqa: E731  an f32 literal
    t = -g
    c = min(max(t, lit("-87.3")), lit("88"))
    n = _round_f32(_q(fma(c, lit("1.44269504088896341"), lit("12582912"))) - 12582912)
    r = fma(-n, lit("0.693145751953125"), c)
    r = fma(-n, lit("1.42860682030941723e-6"), r)
    p = _round_f32(Fraction(1, 5040))
    for k in (Fraction(1, 720), Fraction(1, 120), Fraction(1, 24), Fraction(1, 6), Fraction(1, 2), 1, 1):
        p = fma(p, r, _round_f32(Fraction(k)))
    e = np.float32(0) if t < lit("-87.3") else _round_f32(_q(p) * Fraction(2) ** int(n))
    d = _round_f32(1 + _q(e))
    if g == 0 or u == 0:
        return np.float32(g / d * u)  # an exact zero: IEEE's sign rules
    return _round_f32(_q(_round_f32(_q(g) / _q(d))) * _q(u))


def _silu_inputs():
    rng = np.random.default_rng(31)
    g = np.concatenate([rng.normal(0, 2, 1200), rng.uniform(-95, 95, 200),
                        [0.0, -0.0, 1e-30, -1e-30, 87.29, 87.3, 87.31, -88.0, -88.5, 100.0, -100.0, 0.5, -0.5,
                         np.log(2) / 2, -np.log(2) / 2]]).astype(np.float32)
    u = rng.normal(0, 1, g.size).astype(np.float32)
    return g, u


def test_host_silu_mul_is_the_stated_steps():
    """qd_silu_mul (the decoder's host SwiGLU step) equals an exact-rational
    evaluation of the f32 steps mi355x_server_swiglu states, bit for bit:
    a contraction the steps do not name, or a step left out, changes bits."""
    g, u = _silu_inputs()
    h = decode.silu_mul(g, u)
    want = np.array([_silu_mul_steps(a, b) for a, b in zip(g, u)], dtype=np.float32)
    bad = np.flatnonzero(h.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (g[bad[:5]], h[bad[:5]], want[bad[:5]])


def test_host_silu_mul_accuracy():
    """Against silu in float64 (the steps approximate e^t with relative error
    below 5e-9, then add a few f32 roundings): within 4 ulp of the result
    where e^-g is in range; below g = -88 (e^-g clamped to e^88) the result
    stays below 1e-35 in magnitude."""
    g, u = _silu_inputs()
    h = decode.silu_mul(g, u).astype(np.float64)
    low = g < -88
    assert low.sum() >= 5 and np.abs(h[low]).max() < 1e-35
    g, u, h = g[~low], u[~low], h[~low]
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    with np.errstate(over="ignore"):
        ref = g64 / (1.0 + np.exp(-g64)) * u64
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    ok = np.abs(h - ref) <= 4 * ulp + 1e-37
    assert ok.all(), (g[~ok][:5], h[~ok][:5], ref[~ok][:5])


def _rmsnorm_steps(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The stated RMSNorm steps (mi355x-gemv.h, mi355x_server_block) with
    Python floats (IEEE double, each add rounded once, squares exact)."""
    H = x.size
    xd = [float(v) for v in x]
    p = []
    for k in range(16):
        acc = 0.0
        for i0 in range(0, H, 16):
            acc = acc + xd[i0 + k] * xd[i0 + k]
        p.append(acc)
    lanes = [(p[k] + p[4 + k]) + (p[8 + k] + p[12 + k]) for k in range(4)]
    ss = (lanes[0] + lanes[1]) + (lanes[2] + lanes[3])
    s = np.float32(1.0) / np.sqrt(np.float32(ss / H) + np.float32(eps))
    return (x * s) * w


@pytest.mark.parametrize("H", [256, 2048, 4096])
def test_host_rmsnorm_is_the_stated_steps(H):
    """qd_rmsnorm equals the stated steps bit for bit and is within 2 ulp of
    the float64 formula."""
    rng = np.random.default_rng(H)
    x = (rng.standard_normal(H) * np.exp(rng.uniform(-3, 3, H))).astype(np.float32)
    w = rng.uniform(0.5, 1.5, H).astype(np.float32)
    got = decode.rmsnorm(x, w, 1e-6)
    assert np.array_equal(got.view(np.uint32), _rmsnorm_steps(x, w, 1e-6).view(np.uint32))
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2 * np.spacing(np.abs(ref).astype(np.float32)))


def test_host_rmsnorm_order_is_pinned():
    """Over 300 short vectors the stated steps hold every time, while a
    float32 sum of squares (a plausible slip) changes the output of some: the
    bit-exact check above can tell the two apart."""
    rng = np.random.default_rng(5)
    differ = 0
    for _ in range(300):
        x = (rng.standard_normal(256) * np.exp(rng.uniform(-4, 4, 256))).astype(np.float32)
        w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
        want = _rmsnorm_steps(x, w, 1e-6)
        assert np.array_equal(decode.rmsnorm(x, w, 1e-6).view(np.uint32), want.view(np.uint32))
        ss32 = np.float32(0)
        for v in x:
            ss32 = np.float32(ss32 + np.float32(v * v))
        alt = (x * (np.float32(1) / np.sqrt(np.float32(ss32 / np.float32(256)) + np.float32(1e-6)))) * w
        differ += not np.array_equal(alt, want)
    assert differ > 0
