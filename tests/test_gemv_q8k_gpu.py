"""K-quant and IQ GEMVs in ggml-cpu numerics (MI355X_VARIANT_GGML_Q8): the
activation row quantized to Q8_K and ggml's generic vec_dot_<type>_q8_K
sums, the reference's live path whenever ggml-cpu is loaded
(src/xdna-gemv-engine.cpp:1382-1399, 1430-1453).  Every output must be
bit-identical to the oracle's restatement (oracle.c, orc_gemv_q8_K) -- at
the BASELINE config-3 and config-4 shapes, at small and odd shapes, with
activation blocks of zeros, ties and extreme magnitudes, and with BF16
activations.  IQ3_XXS / IQ2_S use synthetic grids (ggml's are not in this
build)."""
import numpy as np
import pytest

import mi355x
import synth

pytestmark = pytest.mark.gpu

TYPES = {"Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23, "IQ3_S": 21, "IQ3_XXS": 18, "IQ2_S": 22}


def synthetic_grid(t, seed=0):
    # the same grids as the other K/IQ GPU tests install (process-wide table)
    rng = np.random.default_rng(seed)
    n, w = (256, 4) if t == 18 else (1024, 8)
    g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


GRIDS = {t: synthetic_grid(t, seed=t) for t in (18, 22)}


@pytest.fixture(scope="module", autouse=True)
def q8k_variant(ctx):
    for t, g in GRIDS.items():
        mi355x.set_iq_grid(t, g)
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    yield
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


def blocks(t, N, K, seed):
    # random blocks with d (and dmin) spread over several binades
    raw = synth.random_blocks(t, N, K, seed).reshape(N, K // 256, -1)
    rng = np.random.default_rng(seed + 7)
    for off in synth.HALF_FIELDS[t]:
        h = rng.choice(np.array([0x2E66, 0x3266, 0x2A00, 0x1C00, 0x3800, 0xAE66], dtype=np.uint16),
                       size=raw.shape[:2])
        raw[..., off] = (h & 0xFF).astype(np.uint8)
        raw[..., off + 1] = (h >> 8).astype(np.uint8)
    return raw.reshape(N, -1)


def check_bits(ctx, oracle, t, N, K, seed, x=None):
    raw = blocks(t, N, K, seed)
    if x is None:
        x = synth.activations(K, seed=seed + 1)
    w = ctx.resident(t, raw, N, K)
    try:
        y = ctx.gemv(w, x)
    finally:
        w.free()
    xf = x if x.dtype != np.uint16 else (x.astype(np.uint32) << 16).view(np.float32)
    ref = oracle.gemv_q8_K(t, raw, N, K, xf, grid=GRIDS.get(t))
    bad = np.nonzero(y.view(np.uint32) != ref.view(np.uint32))[0]
    assert bad.size == 0, (t, N, K, bad[:5], y[bad[:5]], ref[bad[:5]])


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("N,K", [(1, 256), (64, 256), (37, 768), (128, 4096), (96, 5120), (64, 11008),
                                 (40, 61 * 256), (33, 16384)])
def test_q8k_bit_identical(ctx, oracle, name, N, K):
    check_bits(ctx, oracle, TYPES[name], N, K, seed=N + K)


@pytest.mark.parametrize("name", ["Q3_K", "Q4_K", "Q5_K", "Q6_K"])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_q8k_config3_shapes(ctx, oracle, name, N, K):
    # BASELINE config 3 at full size
    check_bits(ctx, oracle, TYPES[name], N, K, seed=3)


@pytest.mark.parametrize("name", ["IQ2_S", "IQ3_S", "IQ3_XXS", "IQ4_XS"])
def test_q8k_config4_shapes(ctx, oracle, name):
    # BASELINE config 4 at full size
    check_bits(ctx, oracle, TYPES[name], 8192, 8192, seed=4)


@pytest.mark.parametrize("name", list(TYPES))
def test_q8k_activation_edge_blocks(ctx, oracle, name):
    """Superblocks of x that are all zero, hold a tie of the largest |x| with
    both signs (the first one sets the sign of d), span 1e-30..1e30, or are
    small integers (exact halves round to even)."""
    K = 256 * 6
    rng = np.random.default_rng(9)
    x = synth.activations(K, seed=10)
    x[0:256] = 0.0
    x[256:512] = rng.uniform(-1, 1, 256).astype(np.float32)
    x[256 + 17], x[256 + 200] = -3.0, 3.0
    x[512:768] = (rng.standard_normal(256) * 1e-30).astype(np.float32)
    x[768:1024] = (rng.standard_normal(256) * 1e30).astype(np.float32)
    x[1024:1280] = rng.integers(-127, 128, 256).astype(np.float32) / 2
    check_bits(ctx, oracle, TYPES[name], 72, K, seed=11, x=x)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "IQ4_XS", "IQ2_S"])
def test_q8k_bf16_and_unaligned_activations(ctx, oracle, name):
    t, N, K = TYPES[name], 48, 2048
    xb = synth.activations(K, seed=21).view(np.uint32)
    x16 = (xb >> 16).astype(np.uint16)  # bf16 bits
    check_bits(ctx, oracle, t, N, K, seed=22, x=x16)
    raw = blocks(t, N, K, seed=23)
    x = synth.activations(K, seed=24)
    w = ctx.resident(t, raw, N, K)
    xd = ctx.alloc(4 * K + 16)
    yd = ctx.alloc(4 * N)
    try:
        xd.upload(x, offset=4)  # activation row 4 bytes past 16-byte alignment
        mi355x.check(ctx.gemv_ptr(t, w.ptr, N, K, xd.ptr + 4, yd.ptr))
        ctx.sync()
        y = yd.download(np.float32, N)
    finally:
        yd.free()
        xd.free()
        w.free()
    ref = oracle.gemv_q8_K(t, raw, N, K, x, grid=GRIDS.get(t))
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_q8k_rows_longer_than_supported(ctx):
    N, K = 8, 256 * 65
    w = ctx.resident(12, synth.random_blocks(12, N, K, 1), N, K)
    xd = ctx.to_device(synth.activations(K, seed=2))
    yd = ctx.alloc(4 * N)
    try:
        assert ctx.gemv_ptr(12, w.ptr, N, K, xd.ptr, yd.ptr) == mi355x.EUNSUPPORTED
        assert "16384" in mi355x.last_error()
    finally:
        yd.free()
        xd.free()
        w.free()
