"""K-quant and IQ GEMVs on the GPU vs the CPU oracle (through the C-ABI).

Mirrors tests/test-kquants-gemv.cpp of the reference: accuracy against the
scalar refs on random blocks (218-270), zero-activation invariance (258-270),
BF16 activations (272-330); plus the BASELINE K-quant shapes at full size,
odd superblock counts (rows whose planes flip), K beyond one LDS chunk, and
the prepack round trip.  IQ3_XXS / IQ2_S run with a synthetic grid installed
through mi355x_set_iq_grid (their ggml grids are not available here), so
their parity is against the oracle's restatement only.
"""
import functools

import numpy as np
import pytest

import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

REF_TYPES = {"Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23, "IQ3_S": 21}
GRID_TYPES = {"IQ3_XXS": 18, "IQ2_S": 22}
ALL = {**REF_TYPES, **GRID_TYPES}


def synthetic_grid(t, seed=0):
    # magnitudes in the range of ggml's grids (odd values up to 62)
    rng = np.random.default_rng(seed)
    n, w = (256, 4) if t == 18 else (1024, 8)
    g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
    return g.view(np.uint32 if w == 4 else np.uint64).reshape(n)


GRIDS = {t: synthetic_grid(t, seed=t) for t in GRID_TYPES.values()}


@pytest.fixture(scope="module", autouse=True)
def install_grids():
    for t, g in GRIDS.items():
        mi355x.set_iq_grid(t, g)
    yield


@pytest.fixture(params=["digits", "exact_f32", "pipelined", "digits_prefetch", "f32_prefetch", "digits_two_rows",
                        "auto"], autouse=True)
def variant(request, ctx):
    """Every test runs on each kernel family: activations as 16-bit digit
    planes with integer dot products (several workgroups per CU; each
    step's registers refilled with the next row group's step after its
    decode), f32 activations as given, the pipelined form (digit arithmetic,
    one workgroup per CU, each lane's digit slices kept in registers), the
    row form with prefetch (each wavefront's next row group requested before
    the current one's decode) in both arithmetics, the digit row form with
    two rows per wavefront step, and the defaults."""
    p = request.param
    if p != "auto":
        v = mi355x.VARIANT_EXACT_F32 if p.startswith(("exact", "f32")) else mi355x.VARIANT_DIGITS
        ctx.set_option(mi355x.OPT_VARIANT, v)
    if p == "pipelined":
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_PIPE)
    if p.endswith("prefetch"):
        ctx.set_option(mi355x.OPT_PREFETCH, 1)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 1)
    if p.endswith("two_rows"):
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 2)
    yield p
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
    ctx.set_option(mi355x.OPT_PREFETCH, 0)
    ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)


def blocks(t, N, K, seed):
    # spread d (and dmin) over several binades, per block
    raw = synth.random_blocks(t, N, K, seed).reshape(N, K // 256, -1)
    rng = np.random.default_rng(seed + 7)
    for i, off in enumerate(synth.HALF_FIELDS[t]):
        h = rng.choice(np.array([0x2E66, 0x3266, 0x2A00, 0x1C00, 0x3800, 0xAE66], dtype=np.uint16),
                       size=raw.shape[:2])
        raw[..., off] = (h & 0xFF).astype(np.uint8)
        raw[..., off + 1] = (h >> 8).astype(np.uint8)
    return raw.reshape(N, -1)


def run(ctx, t, raw, N, K, x):
    w = ctx.resident(t, raw, N, K)
    try:
        return ctx.gemv(w, x)
    finally:
        w.free()


@functools.lru_cache(maxsize=16)
def quantized(t, N, K, seed):
    """The BASELINE recipe: f32 N(0, 0.02) weights quantized to type t (IQ
    types: with 1% of the weights scaled by 8), on the installed grids."""
    if t in (18, 21, 22, 23):
        w = synth.heavy_tail_weights(N, K, seed)
    else:
        w = synth.normal_weights(N, K, seed)
    grid = synth.iq3s_grid() if t == 21 else GRIDS.get(t)
    return synth.quantize_kq(t, w, grid)


def parity(ctx, oracle, t, N, K, seed, x=None, what="", raw=None):
    if raw is None:
        raw = blocks(t, N, K, seed)
    if x is None:
        x = np.random.default_rng(seed + 1).uniform(-0.5, 0.5, K).astype(np.float32)
    y = run(ctx, t, raw, N, K, x)
    grid = GRIDS.get(t)
    xr = x if x.dtype != np.uint16 else x
    ref = oracle.gemv(t, raw, N, K, xr, grid=grid)
    norms = oracle.row_norms(t, raw, N, K, grid=grid)
    xf = x if x.dtype != np.uint16 else (x.astype(np.uint32) << 16).view(np.float32)
    return check_gemv(y, ref, norms, xf, what or f"type {t} {N}x{K}")


@pytest.mark.parametrize("name", list(ALL))
@pytest.mark.parametrize("N,K", [(1, 256), (64, 256), (37, 768), (128, 4096), (96, 5120), (64, 11008)])
def test_parity_random_blocks(ctx, oracle, name, N, K):
    parity(ctx, oracle, ALL[name], N, K, seed=N + K)


@pytest.mark.parametrize("name", list(ALL))
def test_parity_two_lds_chunks(ctx, oracle, name):
    # K = 61 superblocks > one 60-superblock activation chunk
    parity(ctx, oracle, ALL[name], 40, 61 * 256, seed=5)


@pytest.mark.parametrize("name", ["Q3_K", "Q4_K", "Q5_K", "Q6_K"])
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_parity_baseline_kquant_shapes(ctx, oracle, name, N, K):
    # BASELINE config 3 at full size: random blocks, then the config's own
    # recipe (quantized N(0, 0.02) weights, N(0, 1) activations)
    t = REF_TYPES[name]
    parity(ctx, oracle, t, N, K, seed=3)
    parity(ctx, oracle, t, N, K, seed=3, x=synth.activations(K, seed=43), raw=quantized(t, N, K, 3),
           what=f"{name} {N}x{K} quantized")


@pytest.mark.parametrize("name", ["IQ2_S", "IQ3_S", "IQ3_XXS", "IQ4_XS"])
def test_parity_baseline_iq_shape(ctx, oracle, name):
    # BASELINE config 4 at full size (8192 x 8192), random blocks and the
    # config's recipe (N(0, 0.02) weights with 1% x8 outliers, quantized)
    t = ALL[name]
    parity(ctx, oracle, t, 8192, 8192, seed=4)
    parity(ctx, oracle, t, 8192, 8192, seed=4, x=synth.activations(8192, seed=43), raw=quantized(t, 8192, 8192, 4),
           what=f"{name} 8192x8192 quantized")


@pytest.mark.parametrize("name", list(ALL))
def test_zero_activations_give_exact_zero(ctx, name):
    t = ALL[name]
    raw = blocks(t, 64, 1024, 9)
    y = run(ctx, t, raw, 64, 1024, np.zeros(1024, np.float32))
    assert np.all(y == 0.0)


@pytest.mark.parametrize("name", list(ALL))
def test_bf16_activations(ctx, oracle, name):
    # tests/test-kquants-gemv.cpp:272-330: x = (i % 32) / 32 in BF16
    K = 512
    xf = ((np.arange(K) % 32) * 0.03125).astype(np.float32)
    xb = (xf.view(np.uint32) >> 16).astype(np.uint16)
    parity(ctx, oracle, ALL[name], 128, K, seed=8, x=xb)


@pytest.mark.parametrize("name", list(ALL))
def test_activation_scales(ctx, oracle, name):
    t = ALL[name]
    for i, scale in enumerate((1e-20, 1e-3, 1.0, 1e4, 1e15)):
        x = (np.random.default_rng(i).standard_normal(2048) * scale).astype(np.float32)
        parity(ctx, oracle, t, 48, 2048, seed=20 + i, x=x, what=f"{name} scale {scale}")


@pytest.mark.parametrize("name", list(ALL))
def test_prepack_round_trip(ctx, name):
    t = ALL[name]
    for N, K in ((5, 768), (8, 2048), (3, 256)):
        raw = blocks(t, N, K, N * K).reshape(-1)
        w = ctx.resident(t, raw, N, K, chunk=97)
        try:
            assert np.array_equal(w.raw_bytes(), raw)
            rng = np.random.default_rng(1)
            for _ in range(10):
                off = int(rng.integers(0, raw.size))
                n = int(rng.integers(1, raw.size - off + 1))
                assert np.array_equal(w.raw_bytes(off, n), raw[off:off + n])
        finally:
            w.free()


def test_rows_per_wave_option_keeps_results(ctx, oracle):
    t = REF_TYPES["Q4_K"]
    for r in (1, 2):
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, r)
        try:
            parity(ctx, oracle, t, 300, 2048, seed=r)
        finally:
            ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)


def test_grid_types_refuse_without_grid_or_bad_table(ctx):
    bad = np.zeros(7, dtype=np.uint8)
    with pytest.raises(mi355x.Mi355xError):
        mi355x.set_iq_grid(18, bad)


@pytest.mark.parametrize("form", ["pipelined", "ksplit"])
@pytest.mark.parametrize("name", list(ALL))
@pytest.mark.parametrize("N,K", [(1, 256), (5, 2048), (1023, 4096), (4096, 8192), (14336, 4096), (300, 14336),
                                 (2000, 16384), (777, 11008), (4096, 14336), (8192, 8192)])
def test_form_matches_digit_kernel(ctx, name, variant, form, N, K):
    """The pipelined and activation-stationary (K-split) forms share the digit
    row kernel's per-row arithmetic (same slices, step order and
    expressions), so they agree with it bit for bit: every step count 1..8,
    rows that leave the last wavefronts or tiles partly or wholly empty, K
    beyond one LDS chunk (16384), the BASELINE shapes."""
    if variant != "digits":
        pytest.skip("one run per shape is enough")
    t = ALL[name]
    raw = blocks(t, N, K, N + K)
    x = np.random.default_rng(K).uniform(-0.5, 0.5, K).astype(np.float32)
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_ROWS)
    try:
        y_dg = run(ctx, t, raw, N, K, x)
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_PIPE if form == "pipelined" else mi355x.FORM_KSPLIT)
        y_f = run(ctx, t, raw, N, K, x)
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
    bad = np.nonzero(y_f.view(np.uint32) != y_dg.view(np.uint32))[0]
    assert bad.size == 0, f"{name} {N}x{K}: {bad.size} rows differ, first {bad[:5]} {y_f[bad[:3]]} {y_dg[bad[:3]]}"


@pytest.mark.parametrize("name", ["Q5_K", "IQ2_S"])
def test_ksplit_tile_rows_option(ctx, variant, name):
    """2 and 4 rows per group and tile (OPT_ROWS_PER_WAVE) give the same bits."""
    if variant != "digits":
        pytest.skip("one run per case is enough")
    t = ALL[name]
    N, K = 999, 6144
    raw = blocks(t, N, K, 11)
    x = np.random.default_rng(3).uniform(-0.5, 0.5, K).astype(np.float32)
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_KSPLIT)
    try:
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 4)
        y4 = run(ctx, t, raw, N, K, x)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 2)
        yr = run(ctx, t, raw, N, K, x)
    finally:
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
    assert np.array_equal(y4.view(np.uint32), yr.view(np.uint32))


@pytest.mark.parametrize("name", list(ALL))
@pytest.mark.parametrize("N,K", [(1023, 4096), (515, 8192), (257, 14336)])
def test_many_row_groups_per_wavefront(ctx, name, variant, N, K):
    """With the grid capped at 1 or 3 workgroups each wavefront walks dozens
    of row groups: every refill (or prefetch) of the next group's registers
    lands, the last group's reads nothing, and the rows come out bit for bit
    as with the full grid (the arithmetic of a row does not depend on which
    wavefront computes it)."""
    if variant not in ("digits", "digits_two_rows", "digits_prefetch"):
        pytest.skip("row-form options only")
    t = ALL[name]
    raw = blocks(t, N, K, 5 * N + K)
    x = np.random.default_rng(N).uniform(-0.5, 0.5, K).astype(np.float32)
    y_full = run(ctx, t, raw, N, K, x)
    for cap in (1, 3):
        ctx.set_option(mi355x.OPT_GRID, cap)
        try:
            y_cap = run(ctx, t, raw, N, K, x)
        finally:
            ctx.set_option(mi355x.OPT_GRID, 0)
        bad = np.nonzero(y_cap.view(np.uint32) != y_full.view(np.uint32))[0]
        assert bad.size == 0, f"{name} {N}x{K} grid {cap}: {bad.size} rows differ, first {bad[:5]}"


def test_iq3s_every_grid_index_in_every_position(ctx, oracle, variant):
    """IQ3_S blocks whose 9-bit grid indices (low 8 bits from qs, the high
    bit from qh: bit j % 8 of qh[j / 8] for index j of a superblock) take
    all 512 values in each of the 64 index positions across the matrix's
    512 superblocks, with random signs, scales and d: every index pair the
    digit decode assembles in one word, and every lookup of the f32 decode,
    reads the entry the oracle reads.  Rows of 32 superblocks: in order, the
    default takes the twelve-wavefront kernel."""
    t = ALL["IQ3_S"]
    N, K = 16, 8192
    nb = K // 256
    raw = blocks(t, N, K, 5).reshape(N * nb, 110)
    b = np.arange(N * nb)[:, None]
    j = np.arange(64)[None, :]
    idx = (b + 7 * j) % 512
    raw[:, 2:66] = (idx & 255).astype(np.uint8)
    hi = (idx >> 8).astype(np.uint8).reshape(N * nb, 8, 8)
    raw[:, 66:74] = (hi << np.arange(8, dtype=np.uint8)).sum(axis=2).astype(np.uint8)
    raw = raw.reshape(N, -1)
    x = synth.activations(K, seed=19)
    y = run(ctx, t, raw, N, K, x)
    ref = oracle.gemv(t, raw, N, K, x)
    norms = oracle.row_norms(t, raw, N, K)
    check_gemv(y, ref, norms, x, "IQ3_S every grid index")


def test_iq2s_extreme_grid_and_scales(ctx, oracle, variant):
    """IQ2_S at the edge of the digit arithmetic: every grid magnitude 127
    (the largest a grid may hold), every sign positive, every 4-bit scale
    15, and a constant activation whose digits all sit at the top of their
    range (Z = 32638, high digit 127): the scale-mixed plane sums of a slice
    then come near 2^24 and their combine exceeds int32, which the decode
    must not wrap."""
    t = ALL["IQ2_S"]
    N, K = 64, 2048
    grid = np.full(1024, 0x7F7F7F7F7F7F7F7F, dtype=np.uint64)
    raw = blocks(t, N, K, 3).reshape(N, K // 256, 82)
    raw[..., 0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    raw[..., 34:66] = 0  # signs
    raw[..., 74:82] = 0xFF  # scales
    raw = raw.reshape(N, -1)
    x = np.full(K, 1.015625, dtype=np.float32)
    mi355x.set_iq_grid(t, grid)
    try:
        y = run(ctx, t, raw, N, K, x)
    finally:
        mi355x.set_iq_grid(t, GRIDS[t])
    ref = oracle.gemv(t, raw, N, K, x, grid=grid)
    norms = oracle.row_norms(t, raw, N, K, grid=grid)
    check_gemv(y, ref, norms, x, "IQ2_S extreme grid")
