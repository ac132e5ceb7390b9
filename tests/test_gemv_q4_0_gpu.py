"""Q4_0 GEMV on the GPU vs the CPU oracle (through the C-ABI).

Mirrors the reference's Q4_0 checks: known answers of
tests/test-q4-0-reference.cpp:157-210 and tests/test-backend.cpp:58-98,
the accuracy/zero/sweep cases of tests/test-gemv-accuracy.cpp:103-409, and
the BASELINE shapes at full size.
"""
import numpy as np
import pytest

import mi355x
import synth
from tolerance import check_gemv

pytestmark = pytest.mark.gpu

Q4_0 = mi355x.Q4_0


@pytest.fixture(params=["digits", "exact_f32"], autouse=True)
def variant(request, ctx):
    """Every test runs on both Q4_0 kernel families."""
    v = mi355x.VARIANT_AUTO if request.param == "digits" else mi355x.VARIANT_EXACT_F32
    ctx.set_option(mi355x.OPT_VARIANT, v)
    yield request.param
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


def run_gpu(ctx, raw, N, K, x, chunk=None):
    w = ctx.resident(Q4_0, raw, N, K, chunk=chunk)
    try:
        return ctx.gemv(w, x)
    finally:
        w.free()


def parity(ctx, oracle, raw, N, K, x, what):
    y = run_gpu(ctx, raw, N, K, x)
    ref = oracle.gemv(Q4_0, raw, N, K, x)
    norms = oracle.row_norms(Q4_0, raw, N, K)
    return check_gemv(y, ref, norms, x, what)


def test_known_answer_backend_128(ctx):
    # tests/test-backend.cpp:58-98: 128x256, qs 0x99 (+1,+1), d = 1.0, x = 0.5 -> 128.0
    N, K = 128, 256
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:] = 0x99
    raw = np.tile(blk, N * K // 32)
    y = run_gpu(ctx, raw, N, K, np.full(K, 0.5, dtype=np.float32))
    assert np.array_equal(y, np.full(N, 128.0, dtype=np.float32))


def test_known_answer_two_rows(ctx):
    # tests/test-q4-0-reference.cpp:128-143,193-210: rows give 528 and -264 for x = 1..32
    raw = np.zeros(36, dtype=np.uint8)
    raw[0:2] = [0x00, 0x3C]
    raw[2:18] = 0x99
    raw[18:20] = [0x00, 0x38]
    raw[20:36] = 0x77
    x = np.arange(1, 33, dtype=np.float32)
    y = run_gpu(ctx, raw, 2, 32, x)
    assert y.tolist() == [528.0, -264.0]


def test_known_answer_edge_block(ctx):
    # tests/test-q4-0-reference.cpp:49-54,186-191: low nibbles 0..15, high 15..0 -> dot = -264
    edge = np.array([0x00, 0x3c, 0xf0, 0xe1, 0xd2, 0xc3, 0xb4, 0xa5, 0x96,
                     0x87, 0x78, 0x69, 0x5a, 0x4b, 0x3c, 0x2d, 0x1e, 0x0f], dtype=np.uint8)
    x = np.arange(1, 33, dtype=np.float32)
    assert run_gpu(ctx, edge, 1, 32, x).tolist() == [-264.0]


def test_every_nibble_value(ctx, oracle):
    # all 16 codes in every position, scales spanning fp16 normal/subnormal range
    N, K = 64, 512
    rng = np.random.default_rng(3)
    raw = synth.random_q4_0(N, K, seed=5).reshape(N, K // 32, 18)
    scales = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xBC00, 0x8001, 0x2E66], dtype=np.uint16)
    raw[..., 0:2] = scales[rng.integers(0, len(scales), size=(N, K // 32))].view(np.uint8).reshape(N, K // 32, 2)
    raw = raw.reshape(-1)
    x = synth.activations(K, seed=6) * np.float32(1e-3)
    parity(ctx, oracle, raw, N, K, x, "edge scales")


def test_uniform_weights(ctx, oracle):
    # tests/test-gemv-accuracy.cpp:128-153: qs 0x99, d = 0.5, x = 0.25 -> 32.0 for all rows
    N, K = 256, 256
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = [0x00, 0x38]
    blk[2:] = 0x99
    raw = np.tile(blk, N * K // 32)
    y = run_gpu(ctx, raw, N, K, np.full(K, 0.25, dtype=np.float32))
    assert np.array_equal(y, np.full(N, 32.0, dtype=np.float32))


@pytest.mark.parametrize("N,K", [(16, 64), (128, 256), (256, 512), (512, 1024), (1024, 2048)])
def test_zero_activation_is_exact_zero(ctx, N, K):
    # tests/test-gemv-accuracy.cpp:184-217
    raw = synth.random_q4_0(N, K, seed=505)
    y = run_gpu(ctx, raw, N, K, np.zeros(K, dtype=np.float32))
    assert np.all(y == 0.0)


@pytest.mark.parametrize("N,K", [(512, 512), (256, 256), (1024, 1024), (4096, 4096), (1, 32), (1, 4096),
                                 (33, 64), (127, 128), (255, 64), (384, 128), (513, 64), (1536, 128),
                                 (11008, 4096), (100, 96), (64, 5120), (40, 14336), (24, 17408)])
def test_random_codes(ctx, oracle, N, K):
    # tests/test-gemv-accuracy.cpp:315-396 shapes, plus odd block counts and K beyond one LDS chunk
    raw = synth.random_q4_0(N, K, seed=810 + N + K)
    x = np.random.default_rng(811).uniform(-1, 1, K).astype(np.float32)
    parity(ctx, oracle, raw, N, K, x, f"random {N}x{K}")


@pytest.mark.parametrize("N,K", [(4096, 4096), (8192, 8192), (17408, 5120), (151936, 2048)])
def test_baseline_shapes(ctx, oracle, N, K):
    # f32 N(0,0.02) weights quantized to Q4_0, x ~ N(0,1)
    raw = synth.quantize_q4_0(synth.normal_weights(N, K, seed=1000 + K))
    x = synth.activations(K, seed=2000 + K)
    stats = parity(ctx, oracle, raw, N, K, x, f"baseline {N}x{K}")
    print(f"Q4_0 {N}x{K}: {stats}")


def test_bf16_activations(ctx, oracle):
    # tests/test-gemv-accuracy.cpp:156-178 (run_bf16 vs gemv_bf16)
    N, K = 512, 256
    raw = synth.random_q4_0(N, K, seed=303)
    xf = np.random.default_rng(404).uniform(-1, 1, K).astype(np.float32)
    xb = np.array([oracle.f32_to_bf16(float(v)) for v in xf], dtype=np.uint16)
    y = run_gpu(ctx, raw, N, K, xb)
    ref = oracle.gemv(Q4_0, raw, N, K, xb)
    xw = np.array([oracle.bf16_to_f32(int(b)) for b in xb], dtype=np.float32)
    check_gemv(y, ref, oracle.row_norms(Q4_0, raw, N, K), xw, "bf16")


def test_prepack_round_trip_and_chunks(ctx):
    N, K = 96, 2048
    raw = synth.random_q4_0(N, K, seed=11).reshape(-1)
    for chunk in (None, 7, 1000, 18 * 64 + 5):
        w = ctx.resident(Q4_0, raw, N, K, chunk=chunk)
        try:
            assert np.array_equal(w.raw_bytes(), raw), f"chunk={chunk}"
            assert np.array_equal(w.raw_bytes(1001, 333), raw[1001:1334])
        finally:
            w.free()


def test_chunked_upload_gives_same_gemv(ctx, oracle):
    N, K = 200, 4096
    raw = synth.random_q4_0(N, K, seed=12)
    x = synth.activations(K, seed=13)
    a = run_gpu(ctx, raw, N, K, x)
    b = run_gpu(ctx, raw, N, K, x, chunk=12345)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("prefetch", [1, 2])
@pytest.mark.parametrize("waves,rows", [(8, 1), (8, 2), (8, 4), (16, 1), (16, 2), (16, 4)])
@pytest.mark.parametrize("N,K", [(1000, 2048), (777, 8192), (300, 14336), (130, 5120), (64, 16384)])
def test_tuning_options_keep_results(ctx, oracle, variant, waves, rows, prefetch, N, K):
    # every launch shape the tuning options can select computes the same GEMV
    raw = synth.random_q4_0(N, K, seed=N * 7 + K)
    x = synth.activations(K, seed=99)
    ctx.set_option(mi355x.OPT_WAVES_PER_GROUP, waves)
    ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, rows)
    ctx.set_option(mi355x.OPT_PREFETCH, prefetch)
    try:
        parity(ctx, oracle, raw, N, K, x, f"{variant} waves={waves} rows={rows} pf={prefetch} {N}x{K}")
        ctx.set_option(mi355x.OPT_GRID, 7)
        parity(ctx, oracle, raw, N, K, x, f"{variant} grid=7 {N}x{K}")
    finally:
        ctx.set_option(mi355x.OPT_WAVES_PER_GROUP, 0)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)
        ctx.set_option(mi355x.OPT_PREFETCH, 0)
        ctx.set_option(mi355x.OPT_GRID, 0)


def test_activation_extremes(ctx, oracle):
    # large dynamic range inside a block, exact zeros, and a block that is all zero
    N, K = 128, 1024
    raw = synth.random_q4_0(N, K, seed=21)
    x = synth.activations(K, seed=22)
    x[0:32] = 0.0
    x[32:64] *= np.float32(1e-6)
    x[64] = np.float32(3e4)
    x[100:132] = np.float32(-7.5)
    parity(ctx, oracle, raw, N, K, x, "activation extremes")


def test_tiny_activation_blocks_stay_finite(ctx, oracle):
    """Blocks whose largest |x| is far below 2^-108 (down to subnormals) sit
    next to ordinary blocks: the digit staging keeps their scale finite, so
    the rows stay finite and within the bar (the tiny blocks' products are
    below the f32 resolution of the row sums)."""
    N, K = 256, 2048
    raw = synth.random_q4_0(N, K, seed=23)
    x = synth.activations(K, seed=24)
    x[0:32] *= np.float32(1e-36)
    x[96:128] = np.float32(3e-39)  # subnormal
    x[128:160] *= np.float32(1e-33)
    parity(ctx, oracle, raw, N, K, x, "tiny activation blocks")


def test_rejects_bad_shapes(ctx):
    buf = ctx.alloc(4096)
    try:
        rc = ctx.gemv_ptr(Q4_0, buf.ptr, 10, 33, buf.ptr, buf.ptr)
        assert rc == mi355x.EINVAL and "multiple of 32" in mi355x.last_error()
        rc = ctx.gemv_ptr(Q4_0, 0, 10, 64, buf.ptr, buf.ptr)
        assert rc == mi355x.EINVAL and "null pointer" in mi355x.last_error()
        rc = ctx.gemv_ptr(Q4_0, buf.ptr, -1, 64, buf.ptr, buf.ptr)
        assert rc == mi355x.EINVAL
        rc = ctx.gemv_ptr(Q4_0, buf.ptr, 1 << 62, 1 << 20, buf.ptr, buf.ptr)
        assert rc == mi355x.EINVAL and "overflow" in mi355x.last_error()
        assert ctx.gemv_ptr(Q4_0, buf.ptr, 0, 64, buf.ptr, buf.ptr) == mi355x.OK
    finally:
        buf.free()


@pytest.mark.parametrize("rows", [2, 4])
@pytest.mark.parametrize("N,K", [(8192, 8192), (4096, 4096), (17408, 5120), (1000, 2048), (37, 8192), (64, 256),
                                 (300, 16384)])
def test_ksplit_form(ctx, oracle, variant, rows, N, K):
    """The K-split work split (one 64-block column of R rows per wavefront)
    against the oracle, including partial last columns (K = 5120) and row
    counts that leave workgroups partly empty."""
    if variant != "digits":
        pytest.skip("the K-split form is a digit-plane kernel")
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_KSPLIT)
    ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, rows)
    try:
        raw = synth.random_q4_0(N, K, seed=N + K)
        x = synth.activations(K, seed=K)
        parity(ctx, oracle, raw, N, K, x, f"ksplit R{rows} {N}x{K}")
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)


@pytest.mark.parametrize("waves", [8, 16])
@pytest.mark.parametrize("rows", [0, 4, 8, 16])
@pytest.mark.parametrize("N,K", [(1, 32), (2, 32), (33, 64), (127, 128), (100, 96), (513, 64), (1000, 2048),
                                 (37, 8192), (4096, 4096), (8192, 8192), (2048, 11008), (17408, 5120),
                                 (300, 16384), (24, 4096)])
def test_stream_form(ctx, oracle, variant, waves, rows, N, K):
    """The stream work split (one workgroup per CU; a lane owns one block of
    every row of its team, digit planes in registers, batched butterfly
    reduction) against the oracle: single blocks, partial 64-block columns,
    row counts that leave teams and steps partly empty, every rows-per-step
    and wavefront setting."""
    if variant != "digits":
        pytest.skip("the stream form is a digit-plane kernel")
    if rows == 16 and waves == 16:
        pytest.skip("16 rows per step run with 8 wavefronts (register budget)")
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_STREAM)
    ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, rows)
    ctx.set_option(mi355x.OPT_WAVES_PER_GROUP, waves)
    try:
        raw = synth.random_q4_0(N, K, seed=N + K)
        x = synth.activations(K, seed=K)
        parity(ctx, oracle, raw, N, K, x, f"stream R{rows} W{waves} {N}x{K}")
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)
        ctx.set_option(mi355x.OPT_WAVES_PER_GROUP, 0)


def test_stream_form_edges(ctx, oracle):
    """Known answer, non-finite activations poisoning every row (as f32
    arithmetic does), and a misaligned activation row (the stream form needs
    16-byte alignment and hands such calls to the row form)."""
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_STREAM)
    try:
        N, K = 128, 256
        blk = np.zeros(18, dtype=np.uint8)
        blk[0:2] = [0x00, 0x3C]
        blk[2:] = 0x99
        y = run_gpu(ctx, np.tile(blk, N * K // 32), N, K, np.full(K, 0.5, dtype=np.float32))
        assert np.array_equal(y, np.full(N, 128.0, dtype=np.float32))

        N, K = 64, 512
        raw = synth.random_q4_0(N, K, seed=3)
        x = synth.activations(K, seed=4)
        x[40] = np.inf
        x[300] = np.nan
        assert np.all(np.isnan(run_gpu(ctx, raw, N, K, x)))

        N, K = 300, 2048
        raw = synth.random_q4_0(N, K, seed=5)
        x = synth.activations(K, seed=6)
        w = ctx.resident(Q4_0, raw, N, K)
        xb = ctx.alloc(4 * K + 16)
        yb = ctx.alloc(4 * N)
        try:
            xb.upload(x, offset=4)
            mi355x.check(ctx.gemv_ptr(Q4_0, w.ptr, N, K, xb.ptr + 4, yb.ptr))
            ctx.sync()
            y = yb.download(np.float32, N)
        finally:
            w.free()
            xb.free()
            yb.free()
        check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), oracle.row_norms(Q4_0, raw, N, K), x, "stream misaligned x")
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)


def check_q8(ctx, oracle, raw, N, K, x, what):
    """GGML_Q8 variant against the oracle's ggml-cpu restatement: the same
    quantization, the same per-block products ((sumi * d_w) * d_x, sumi
    exact) and the same sequential block sum -- bit-identical."""
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    try:
        y = run_gpu(ctx, raw, N, K, x)
    finally:
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
    ref = oracle.gemv_q4_0_q8_0(raw, N, K, x)
    bad = np.nonzero(y.view(np.uint32) != ref.view(np.uint32))[0]
    assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:5]} y={y[bad[:3]]} ref={ref[bad[:3]]}"
    return y, ref


def test_ggml_q8_single_block_rows(ctx, oracle, variant):
    if variant != "digits":
        pytest.skip("one run is enough")
    N, K = 1000, 32
    raw = synth.random_q4_0(N, K, seed=61)
    x = synth.activations(K, seed=62)
    check_q8(ctx, oracle, raw, N, K, x, "K=32")


@pytest.mark.parametrize("N,K", [(1, 64), (33, 96), (127, 128), (513, 2048), (4096, 4096), (300, 5120),
                                 (2048, 11008), (64, 16384), (8192, 8192), (151936, 2048)])
def test_ggml_q8_matches_oracle(ctx, oracle, variant, N, K):
    if variant != "digits":
        pytest.skip("one run is enough")
    raw = synth.quantize_q4_0(synth.normal_weights(N, K, seed=N + K))
    x = synth.activations(K, seed=K + 1)
    x[::97] *= np.float32(40.0)  # blocks with a dominant value
    x[5:37] = 0.0  # an all-zero block (d = 0, id = 0)
    check_q8(ctx, oracle, raw, N, K, x, f"{N}x{K}")


def test_ggml_q8_is_not_the_f32_path(ctx, oracle, variant):
    """Q8_0 activations are coarser than the f32 path: the variant must land
    on the ggml-cpu numbers, not on the f32 reference."""
    if variant != "digits":
        pytest.skip("one run is enough")
    N, K = 256, 4096
    raw = synth.random_q4_0(N, K, seed=71)
    x = synth.activations(K, seed=72)
    y, ref8 = check_q8(ctx, oracle, raw, N, K, x, "q8 vs f32")
    ref32 = oracle.gemv(Q4_0, raw, N, K, x)
    assert np.max(np.abs(y - ref8)) < 0.05 * np.max(np.abs(ref8 - ref32))


def test_ggml_q8_rejects_other_inputs(ctx):
    ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_GGML_Q8)
    buf = ctx.alloc(1 << 16)
    try:
        # BF16 activations for Q4_0 (the K/IQ types take them: test_gemv_q8k_gpu.py)
        assert ctx.gemv_ptr(Q4_0, buf.ptr, 4, 256, buf.ptr, buf.ptr + 4096, bf16=True) == mi355x.EUNSUPPORTED
    finally:
        buf.free()
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)


def gemv_with_form(ctx, raw, N, K, x, form, rows=0):
    ctx.set_option(mi355x.OPT_FORM, form)
    ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, rows)
    try:
        return run_gpu(ctx, raw, N, K, x)
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)
        ctx.set_option(mi355x.OPT_ROWS_PER_WAVE, 0)


@pytest.mark.parametrize("N,K", [(1, 2048), (5, 2048), (1023, 2048), (2560, 2048), (4097, 4096), (8192, 8192),
                                 (12288, 4096), (16384, 2048), (17, 6144), (1000, 10240), (999, 12288),
                                 (2048, 14336), (300, 16384), (3000, 8192), (17408, 4096), (151936, 2048),
                                 (12000, 14336), (9000, 16384)])
def test_pipelined_form(ctx, oracle, variant, N, K):
    """The pipelined work split (one workgroup of eight wavefronts per CU,
    runs of consecutive rows per wavefront, loads two rows ahead, digit
    planes in registers, one batched cross-lane reduction per wavefront)
    against the oracle, and against the row form with one row per wavefront,
    whose per-lane arithmetic it shares (only the order of the 64 lane
    partials differs): every block-column count 1..8, row counts that leave
    the last wavefronts partly or wholly empty, each compiled rows-per-
    wavefront count, the run-time count (17408 and 151936 rows), and the
    long-row cases the form hands to the other forms (12000x14336,
    9000x16384)."""
    if variant != "digits":
        pytest.skip("the pipelined form is a digit-plane kernel")
    raw = synth.random_q4_0(N, K, seed=N + 3 * K)
    x = synth.activations(K, seed=K + 7)
    y = gemv_with_form(ctx, raw, N, K, x, mi355x.FORM_PIPE)
    norms = oracle.row_norms(Q4_0, raw, N, K)
    check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), norms, x, f"pipelined {N}x{K}")
    y_rows = gemv_with_form(ctx, raw, N, K, x, mi355x.FORM_ROWS, rows=1)
    scale = norms * float(np.linalg.norm(x.astype(np.float64)))
    diff = np.abs(y.astype(np.float64) - y_rows)
    bad = np.nonzero(diff > 1e-6 * scale)[0]
    assert bad.size == 0, f"pipelined {N}x{K}: {bad.size} rows differ from the row form, first {bad[:5]}"


def test_pipelined_form_edges(ctx, oracle):
    """Known answer, non-finite activations poisoning every row, and the
    shapes the pipelined form does not take (K not a multiple of 2048, a
    misaligned activation row), which go to the other forms."""
    ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_PIPE)
    try:
        N, K = 128, 2048
        blk = np.zeros(18, dtype=np.uint8)
        blk[0:2] = [0x00, 0x3C]
        blk[2:] = 0x99
        y = run_gpu(ctx, np.tile(blk, N * K // 32), N, K, np.full(K, 0.5, dtype=np.float32))
        assert np.array_equal(y, np.full(N, 1024.0, dtype=np.float32))

        N, K = 64, 4096
        raw = synth.random_q4_0(N, K, seed=3)
        x = synth.activations(K, seed=4)
        x[40] = np.inf
        x[3000] = np.nan
        assert np.all(np.isnan(run_gpu(ctx, raw, N, K, x)))

        for N, K in ((300, 5120), (64, 256), (33, 11008)):
            raw = synth.random_q4_0(N, K, seed=N + K)
            x = synth.activations(K, seed=K)
            parity(ctx, oracle, raw, N, K, x, f"pipelined fallback {N}x{K}")

        N, K = 300, 2048
        raw = synth.random_q4_0(N, K, seed=5)
        x = synth.activations(K, seed=6)
        w = ctx.resident(Q4_0, raw, N, K)
        xb = ctx.alloc(4 * K + 16)
        yb = ctx.alloc(4 * N)
        try:
            xb.upload(x, offset=4)
            mi355x.check(ctx.gemv_ptr(Q4_0, w.ptr, N, K, xb.ptr + 4, yb.ptr))
            ctx.sync()
            y = yb.download(np.float32, N)
        finally:
            w.free()
            xb.free()
            yb.free()
        check_gemv(y, oracle.gemv(Q4_0, raw, N, K, x), oracle.row_norms(Q4_0, raw, N, K), x,
                   "pipelined misaligned x")
    finally:
        ctx.set_option(mi355x.OPT_FORM, mi355x.FORM_AUTO)


def test_fence_covers_pinned_outputs(ctx, oracle):
    """mi355x_ctx_fence: GEMVs write into pinned host memory and the host reads
    it right after the fence, 40 times in a row with changing activations and
    shapes; every result equals the same GEMV waited for with mi355x_ctx_sync."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    rng = np.random.default_rng(41)
    shapes = [(2560, 2048), (2048, 11008), (256, 4096)]
    ws = [(ctx.resident(Q4_0, synth.random_q4_0(N, K, 50 + i), N, K), N, K) for i, (N, K) in enumerate(shapes)]
    nmax = max(N for N, _ in shapes)
    hptr = ctypes.c_void_p()
    mi355x.check(ctx.lib.mi355x_host_malloc(4 * nmax, ctypes.byref(hptr)))
    dptr = ctypes.c_void_p()
    try:
        assert hip.hipHostGetDevicePointer(ctypes.byref(dptr), hptr, 0) == 0
        host_y = np.ctypeslib.as_array(ctypes.cast(hptr, ctypes.POINTER(ctypes.c_float)), shape=(nmax,))
        for it in range(40):
            w, N, K = ws[it % len(ws)]
            x = rng.standard_normal(K).astype(np.float32)
            want = ctx.gemv(w, x)
            host_y[:] = np.nan
            xb = ctx.to_device(x)
            try:
                mi355x.check(ctx.gemv_ptr(Q4_0, w.ptr, N, K, xb.ptr, dptr.value))
                ctx.fence()
                assert np.array_equal(host_y[:N], want), (it, N, K)
            finally:
                xb.free()
    finally:
        mi355x.check(ctx.lib.mi355x_host_free(hptr))
        for w, _, _ in ws:
            w.free()
