"""End-to-end greedy decode with every matrix-vector product on the MI355X
(weights prepacked into HBM) against the same decoder with the CPU oracle's
GEMV: the tokens must be identical and the last logits close.  The full
Qwen2.5-3B shape (512-token prompt, 128 tokens) is run by bench.py --decode;
here: tiny models and one 3B-shaped layer stack at reduced depth."""
import numpy as np
import pytest

import decode
import oracle as orc

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000,
            rope_theta=1e6, norm_eps=1e-6, seed=7)
# 3B layer shapes (hidden 2048, 16q/2kv x 128, FFN 11008, vocab 151936), 2 layers
SHAPE_3B_2L = dict(decode.QWEN25_3B, n_layers=2)


def run_both(cfg, n_prompt, n_gen, prompt_seed):
    with decode.Model(threads=8, **cfg) as m:
        p = decode.prompt_tokens(n_prompt, cfg["vocab"], prompt_seed)
        f, _ = orc.decode_gemv("oracle")
        cpu_toks, _ = m.generate(p, n_gen, f)
        cpu_logits = m.last_logits()
        m.attach_gpu(0)
        gpu_toks, t = m.generate(p, n_gen)
        gpu_logits = m.last_logits()
    return cpu_toks, cpu_logits, gpu_toks, gpu_logits, t


def check(cpu_toks, cpu_logits, gpu_toks, gpu_logits):
    assert np.array_equal(gpu_toks, cpu_toks), (gpu_toks, cpu_toks)
    a, b = gpu_logits.astype(np.float64), cpu_logits.astype(np.float64)
    assert np.dot(a, b) / np.linalg.norm(a) / np.linalg.norm(b) >= 0.99999
    assert np.abs(a - b).max() <= 1e-3 * np.abs(b).max()


@pytest.mark.parametrize("seed", [7, 8])
def test_tiny_decode_token_identical(seed):
    cfg = dict(TINY, seed=seed)
    cpu_toks, cpu_logits, gpu_toks, gpu_logits, t = run_both(cfg, 16, 12, seed)
    check(cpu_toks, cpu_logits, gpu_toks, gpu_logits)
    assert t["gen_passes"] == 11 and t["gen_gemv_s"] > 0


def test_3b_layer_shapes_token_identical():
    cpu_toks, cpu_logits, gpu_toks, gpu_logits, _ = run_both(SHAPE_3B_2L, 8, 6, 1)
    check(cpu_toks, cpu_logits, gpu_toks, gpu_logits)


def test_gpu_decode_repeatable():
    with decode.Model(threads=4, **TINY) as m:
        m.attach_gpu(0)
        m.attach_gpu(0)  # second attach keeps the resident weights
        p = decode.prompt_tokens(5, 1000, 2)
        a, _ = m.generate(p, 7)
        la = m.last_logits()
        b, _ = m.generate(p, 7)
        assert np.array_equal(a, b) and np.array_equal(la, m.last_logits())
        one, _ = m.generate(p, 1)
        assert one[0] == a[0]


@pytest.mark.parametrize("wait", ["fence", "server"])
def test_fused_launches_match_per_matrix_launches(wait):
    """q|k|v and gate|up as one launch (one server job) each, adjacent in
    HBM, against one per matrix: same tokens, logits equal to float rounding."""
    with decode.Model(threads=4, **TINY) as m:
        m.attach_gpu(0)
        m.set_wait(m.WAIT_FENCE if wait == "fence" else m.WAIT_SERVER)
        p = decode.prompt_tokens(9, 1000, 4)
        fused, _ = m.generate(p, 6)
        lf = m.last_logits()
        assert m.last_launches() == 5 * (4 * TINY["n_layers"] + 1)
        m.set_fuse(False)
        single, _ = m.generate(p, 6)
        ls = m.last_logits()
        assert m.last_launches() == 5 * (7 * TINY["n_layers"] + 1)
        assert np.array_equal(fused, single)
        assert np.abs(lf - ls).max() <= 1e-5 * np.abs(ls).max()
        assert m.last_wait() == (m.WAIT_FENCE if wait == "fence" else m.WAIT_SERVER)


def test_mapped_io_matches_staged_io():
    """Kernels reading the activation from / writing outputs to pinned host
    memory (mapped I/O, the default) against copies through HBM (staged
    I/O): the same kernels on the same numbers, so tokens and logits are
    bit-identical; the vocabulary projection (above the mapped-output limit)
    takes the copy path in both."""
    cfg = dict(TINY, vocab=70000)
    with decode.Model(threads=4, **cfg) as m:
        m.attach_gpu(0)
        m.set_wait(m.WAIT_FENCE)  # I/O modes are those of the launch path
        p = decode.prompt_tokens(7, cfg["vocab"], 5)
        mapped, _ = m.generate(p, 5)
        lm = m.last_logits()
        m.set_io(m.IO_STAGED)
        staged, _ = m.generate(p, 5)
        assert np.array_equal(mapped, staged)
        assert np.array_equal(lm, m.last_logits())
        with pytest.raises(RuntimeError, match="unknown mode"):
            m.set_io(7)


@pytest.mark.parametrize("cfg", [TINY, SHAPE_3B_2L], ids=["tiny", "3b_2layers"])
def test_ggml_numerics_decode_token_identical_to_cpu(cfg):
    """With the GGML_Q8 kernel variant (activations quantized to Q8_0 as
    ggml-cpu does) the GPU decode picks the tokens of the CPU decode that uses
    the oracle's restatement of ggml-cpu's Q4_0 x Q8_0 arithmetic."""
    import mi355x
    with decode.Model(threads=8, **cfg) as m:
        p = decode.prompt_tokens(9, cfg["vocab"], 3)
        f, _ = orc.decode_gemv("ggml_q8")
        cpu_toks, _ = m.generate(p, 8, f)
        cpu_logits = m.last_logits()
        m.attach_gpu(0)
        m.set_variant(mi355x.VARIANT_GGML_Q8)
        gpu_toks, _ = m.generate(p, 8)
        gpu_logits = m.last_logits()
        assert m.last_wait() == m.WAIT_SERVER  # the server's Q8_0 job form
        m.set_wait(m.WAIT_FENCE)
        launch_toks, _ = m.generate(p, 8)
        launch_logits = m.last_logits()
        assert m.last_wait() == m.WAIT_FENCE
        m.set_wait(m.WAIT_SERVER)
        m.set_variant(mi355x.VARIANT_AUTO)
    assert np.array_equal(launch_toks, cpu_toks) and np.array_equal(launch_logits, cpu_logits)
    # every GEMV is bit-identical to the restatement and the host ops are the
    # same code, so the whole decode is: tokens and logits alike.  (Q8_0
    # codes are discrete -- any upstream rounding difference could move an
    # activation across a code boundary and grow from layer to layer -- so
    # anything short of bit-identical GEMVs would not hold the tokens.)
    assert np.array_equal(gpu_toks, cpu_toks), (gpu_toks, cpu_toks)
    assert np.array_equal(gpu_logits, cpu_logits)


@pytest.mark.parametrize("cfg,n_prompt,n_gen", [(TINY, 16, 12), (SHAPE_3B_2L, 8, 6)], ids=["tiny", "3b_2layers"])
def test_server_decode_token_identical(cfg, n_prompt, n_gen):
    """Every GEMV group as a command to the persistent server kernel: same
    tokens as the CPU engine, and the same as launch-per-group decode."""
    with decode.Model(threads=8, **cfg) as m:
        p = decode.prompt_tokens(n_prompt, cfg["vocab"], 3)
        f, _ = orc.decode_gemv("oracle")
        cpu_toks, _ = m.generate(p, n_gen, f)
        cpu_logits = m.last_logits()
        m.attach_gpu(0)
        m.set_wait(m.WAIT_FENCE)
        launch_toks, _ = m.generate(p, n_gen)
        assert m.last_wait() == m.WAIT_FENCE
        m.set_wait(m.WAIT_SERVER)
        srv_toks, t = m.generate(p, n_gen)
        assert m.last_wait() == m.WAIT_SERVER
        srv_logits = m.last_logits()
        again, _ = m.generate(p, n_gen)  # a second decode relaunches the server
        m.set_wait(m.WAIT_FENCE)
    check(cpu_toks, cpu_logits, srv_toks, srv_logits)
    assert np.array_equal(srv_toks, launch_toks) and np.array_equal(again, srv_toks)
    assert t["gen_passes"] == n_gen - 1


@pytest.mark.parametrize("cfg", [TINY, SHAPE_3B_2L], ids=["tiny", "3b_2layers"])
def test_decode_through_the_plugin(cfg):
    """Every GEMV group through the ggml plugin (set_tensor'd weights,
    activation in, graph_compute over the group's MUL_MAT nodes -- one
    multi-job launch for q|k|v and gate|up -- outputs out, synchronize):
    the CPU engine's tokens; in the GGML_Q8 variant the restated ggml path's
    tokens and logits bit for bit."""
    import mi355x
    with decode.Model(threads=8, **cfg) as m:
        p = decode.prompt_tokens(9, cfg["vocab"], 6)
        f, _ = orc.decode_gemv("oracle")
        cpu_toks, _ = m.generate(p, 7, f)
        cpu_logits = m.last_logits()
        fq, _ = orc.decode_gemv("ggml_q8")
        q8_toks, _ = m.generate(p, 7, fq)
        q8_logits = m.last_logits()
        m.attach_gpu(0)
        m.set_wait(m.WAIT_PLUGIN)
        toks, t = m.generate(p, 7)
        logits = m.last_logits()
        assert m.last_wait() == m.WAIT_PLUGIN
        assert m.last_launches() == 6 * (7 * cfg["n_layers"] + 1)  # MUL_MAT nodes
        m.set_variant(mi355x.VARIANT_GGML_Q8)
        gq_toks, _ = m.generate(p, 7)
        gq_logits = m.last_logits()
        m.set_variant(mi355x.VARIANT_AUTO)
        m.set_wait(m.WAIT_SERVER)
    check(cpu_toks, cpu_logits, toks, logits)
    assert np.array_equal(gq_toks, q8_toks) and np.array_equal(gq_logits, q8_logits)


@pytest.mark.timeout(900)
def test_config5_full_decode_token_identical():
    """BASELINE config 5 at full size: the Qwen2.5-3B shape (36 layers), a
    512-token uniform-random prompt, then 128 greedy tokens.
      * default GPU decode (digit-plane GEMVs, persistent server) against the
        same decoder with every GEMV on the reference's own CPU engine
        (oracle/_ref, else the C oracle): the same 128 tokens;
      * GGML_Q8 GPU decode (server Q8_0 job form) against the CPU decode with
        the oracle's restatement of ggml-cpu's Q4_0 x Q8_0 arithmetic: the
        same 128 tokens and bit-identical last logits."""
    import mi355x
    cfg = decode.QWEN25_3B
    p = decode.prompt_tokens(512, cfg["vocab"], 1)
    with decode.Model(threads=16, **cfg) as m:
        kind = "reference" if orc.RefLib.available() else "oracle"
        f, _ = orc.decode_gemv(kind)
        cpu_toks, _ = m.generate(p, 128, f)
        cpu_logits = m.last_logits()
        fq, _ = orc.decode_gemv("ggml_q8")
        q8_toks, _ = m.generate(p, 128, fq)
        q8_logits = m.last_logits()
        m.attach_gpu(0)
        gpu_toks, t = m.generate(p, 128)
        gpu_logits = m.last_logits()
        assert m.last_wait() == m.WAIT_SERVER
        m.set_variant(mi355x.VARIANT_GGML_Q8)
        gq_toks, tq = m.generate(p, 128)
        gq_logits = m.last_logits()
        assert m.last_wait() == m.WAIT_SERVER
        m.set_variant(mi355x.VARIANT_AUTO)
    print(f"config 5: default {127 / t['gen_s']:.1f} tok/s, GGML_Q8 {127 / tq['gen_s']:.1f} tok/s "
          f"(CPU GEMVs: {kind})", flush=True)
    check(cpu_toks, cpu_logits, gpu_toks, gpu_logits)
    assert np.array_equal(gq_toks, q8_toks), (gq_toks, q8_toks)
    assert np.array_equal(gq_logits, q8_logits)
    assert t["gen_passes"] == 127 and tq["gen_passes"] == 127
