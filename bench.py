"""Decode-GEMV benchmark on one MI355X.

One step = LAUNCHES_PER_STEP (50) back-to-back Q4_0 GEMVs at N x K =
8192 x 8192 (the north-star shape, which is quoted "timed
over 1000 back-to-back launches") over one f32 activation row, with the
weights already resident in HBM; `--steps 20` is config 2's 1000 launches in
one timed window.  Launches rotate through enough resident weight copies
(>= 1 GiB) that the 256 MB Infinity Cache cannot serve them, so the figure is
HBM bandwidth.  Timing: HIP events around the `--steps` x 50 launches on the
library's own stream (mi355x_time_gemv), after `--warmup` x 50 launches;
before those, `--settle` seconds of the same launches, untimed, bring the
GPU's clocks out of idle.

Prints one JSON line (see README of the driver contract):
  value      = algorithmic GB/s of the whole job (one GPU)
  roofline   = the GEMV kernel against the 8 TB/s HBM3E peak
  cpu_baseline = the reference's own AVX2/OpenMP Q4GemvEngine
                 (oracle/_ref, 4 threads) on a bounded sample of the same
                 workload, timed on this host
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "xdna.cpp_amd"))

import mi355x  # noqa: E402
import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_0 GEMV HBM GB/s (% of roofline) at 8192x8192; decode tok/s, 3B shape"
ROTATE_BYTES = 1 << 30
# The reference's published Q4_0 8192x8192 GEMV throughput (README.md:98;
# weight bytes / time on its host CPU).
REFERENCE_GBS = 40.41
# GEMV launches per bench step: every timed window covers steps x 50
# launches, so a window's fixed cost (event records, the stream fork and join
# of overlapped launches) is spread as over config 2's 1000 launches
LAUNCHES_PER_STEP = 50
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_0_gemv_8192x8192_traffic.json")


def algorithmic_bytes(t: int, N: int, K: int) -> int:
    return N * mi355x.row_bytes(t, K) + 4 * K + 4 * N


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_rate(ctx, t, raw, N, K, x, steps, warmup, rotate_bytes, settle_s=0.0, overlap=0):
    """Returns (ms_per_launch, copies, y) for `steps` launches over resident
    copies.  With settle_s > 0 the same launches first run untimed for about
    that long, so the GPU's clocks have left their idle state before the
    warm-up and the timed launches (a cold GPU adds ~0.3 us per launch).
    With overlap = S (2-4) the context's MI355X_OPT_OVERLAP is S: up to S
    consecutive launches (independent: other weight copies, S outputs in
    turn) may run at once, each starting while the previous ones drain."""
    wbytes = N * mi355x.row_bytes(t, K)
    copies = max(1, -(-rotate_bytes // wbytes)) if rotate_bytes else 1
    first = ctx.resident(t, raw, N, K)
    bufs = [first.buf]
    for _ in range(copies - 1):
        b = ctx.alloc(wbytes)
        mi355x.check(ctx.lib.mi355x_memcpy_d2d(ctx.h, b.ptr, first.ptr, wbytes))
        bufs.append(b)
    xb = ctx.to_device(x)
    yb = ctx.alloc(4 * N * max(1, overlap))
    try:
        ctx.set_option(mi355x.OPT_OVERLAP, overlap)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < settle_s:
            ctx.time_gemv(t, [b.ptr for b in bufs], N, K, xb.ptr, yb.ptr, 0, 1000)
        ms = ctx.time_gemv(t, [b.ptr for b in bufs], N, K, xb.ptr, yb.ptr, warmup, steps)
        ctx.set_option(mi355x.OPT_OVERLAP, 0)
        y = yb.download(np.float32, N)
        if overlap and any(not np.array_equal(y, o)
                           for o in yb.download(np.float32, overlap * N).reshape(overlap, N)):
            raise RuntimeError("overlapped launches wrote different outputs")
    finally:
        ctx.set_option(mi355x.OPT_OVERLAP, 0)
        for b in bufs:
            b.free()
        xb.free()
        yb.free()
    return ms / steps, copies, y


def host_topology():
    """(logical CPUs this process may use, physical cores among them): the
    cores come from each allowed CPU's (package, core) id in sysfs, the same
    topology lscpu prints."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    return len(cpus), len(cores)


def timed(run, budget_s):
    run()
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            return n, dt


def cpu_baseline(raw, N, K, x, budget_s: float):
    """Time the reference's Q4GemvEngine (oracle/_ref) -- or the C oracle when
    the reference build is absent -- on the same bytes for ~budget_s seconds.
    The engine runs its rows on 4 OpenMP threads (num_threads(4) in
    src/cpu-q4-gemv-engine.cpp:166); to use every physical core of the host,
    cores / 4 host threads each run the engine on an equal slice of the rows
    (rows are independent, so the outputs are the engine's own)."""
    from concurrent.futures import ThreadPoolExecutor

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    logical, physical = host_topology()
    raw = np.ascontiguousarray(raw.reshape(-1))
    y = np.empty(N, dtype=np.float32)
    rb = mi355x.row_bytes(mi355x.Q4_0, K)
    if orc.RefLib.available():
        ref = orc.RefLib()
        teams = max(1, physical // orc.RefCpuEngine.THREADS)
        engines = [orc.RefCpuEngine(ref) for _ in range(teams)]
        bounds = [N * i // teams for i in range(teams + 1)]
        pool = ThreadPoolExecutor(max_workers=teams)

        def part(i):
            r0, r1 = bounds[i], bounds[i + 1]
            engines[i].run(raw[r0 * rb:r1 * rb], r1 - r0, K, x, y[r0:r1])

        run = lambda: list(pool.map(part, range(teams)))  # noqa: E731
        kind, cores = "reference", teams * orc.RefCpuEngine.THREADS
        what = (f"xdna::Q4GemvEngine::run (AVX2+OpenMP, 4 threads each) in {teams} concurrent row slices")
    else:
        o = orc.Oracle()
        run = lambda: o.gemv(2, raw, N, K, x)  # noqa: E731
        pool = None
        kind, cores, what = "port", physical, "C oracle (port of gemv_f32, OpenMP over rows)"
    try:
        n, dt = timed(run, budget_s)
    finally:
        if pool:
            pool.shutdown()
    sec = dt / n
    return {"value": round(algorithmic_bytes(mi355x.Q4_0, N, K) / sec / 1e9, 3), "unit": "GB/s",
            "cores": cores, "kind": kind,
            "sample": f"{n} GEMVs of Q4_0 {N}x{K} (same bytes and x) in {dt:.1f} s, {what}, "
                      f"{sec * 1e3:.3f} ms/GEMV; {cores} threads on a host share of {physical} physical cores "
                      f"({logical} logical CPUs)"}


KQ_TYPES = {"Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}
IQ_TYPES = {"IQ2_S": 22, "IQ3_S": 21, "IQ3_XXS": 18, "IQ4_XS": 23}


def synthetic_grids():
    """IQ3_XXS / IQ2_S codebooks of odd bytes 1..63 (seeded), installed; with
    IQ3_S's own codebook, the grids the quantizer encodes against."""
    rng = np.random.default_rng(0)
    grids = {21: synth.iq3s_grid()}
    for t, (n, w) in ((18, (256, 4)), (22, (1024, 8))):
        g = (2 * rng.integers(0, 32, (n, w)) + 1).astype(np.uint8)
        grids[t] = g.view(np.uint32 if w == 4 else np.uint64).reshape(n)
        mi355x.set_iq_grid(t, grids[t])
    return grids


def kq_weights(t, N, K, grids, seed=7):
    """BASELINE configs 3 and 4: f32 N(0, 0.02) weights (IQ types: 1% of them
    x8) quantized to type t."""
    heavy = t in IQ_TYPES.values()
    w = synth.heavy_tail_weights(N, K, seed) if heavy else synth.normal_weights(N, K, seed)
    return synth.quantize_kq(t, w, grids.get(t))


def kquant_sweep(ctx, steps, warmup, settle_s=0.0, overlap=0):
    """BASELINE configs 3 and 4: each K/IQ type at its shapes, HBM-resident
    (rotated) weights, built by the configs' recipe (kq_weights); IQ3_XXS /
    IQ2_S run with a synthetic grid, as ggml's grids are not part of this
    build."""
    grids = synthetic_grids()
    res = {}
    shapes = [(name, t, N, K) for name, t in KQ_TYPES.items() for (N, K) in ((14336, 4096), (4096, 14336))]
    shapes += [(name, t, 8192, 8192) for name, t in IQ_TYPES.items()]
    for name, t, N, K in shapes:
        raw = kq_weights(t, N, K, grids)
        x = synth.activations(K, seed=43)
        ms, copies, _ = gemv_rate(ctx, t, raw, N, K, x, steps, warmup, ROTATE_BYTES, settle_s)
        gbs = algorithmic_bytes(t, N, K) / (ms * 1e-3) / 1e9
        mso = gemv_rate(ctx, t, raw, N, K, x, steps, warmup, ROTATE_BYTES, settle_s, overlap=overlap)[0] if overlap else ms
        gbo = algorithmic_bytes(t, N, K) / (mso * 1e-3) / 1e9
        res[f"{name} {N}x{K}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                  "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies,
                                  "us_overlap": round(mso * 1e3, 3), "frac_overlap": round(gbo / HBM_PEAK_GBS, 4)}
        log(f"bench: {name} {N}x{K}: {ms * 1e3:.2f} us, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS:.1%}); "
            f"overlapped {mso * 1e3:.2f} us ({gbo / HBM_PEAK_GBS:.1%})")
    return res


def rows_sweep(ctx, steps, warmup, settle_s=0.0):
    """Duration against row count for two K/IQ types at a fixed K (rotated
    weights): t(N) = fixed + N * per_row by least squares over N >= 1024.
    The fixed part is what a launch costs before and after its rows
    (dispatch, activation and codebook staging, the last reduction); the
    per-row slope gives the marginal rate once many rows share that cost."""
    grids = synthetic_grids()
    res = {}
    for name, t, K in (("IQ2_S", IQ_TYPES["IQ2_S"], 8192), ("Q4_K", KQ_TYPES["Q4_K"], 4096)):
        pts = []
        rows = (256, 1024, 4096, 8192, 16384, 32768)
        full = kq_weights(t, max(rows), K, grids)
        for N in rows:
            raw = np.ascontiguousarray(full[:N])
            x = synth.activations(K, seed=43)
            ms, _, _ = gemv_rate(ctx, t, raw, N, K, x, steps, warmup, ROTATE_BYTES, settle_s)
            pts.append((N, ms * 1e3))
        fit = np.polyfit([n for n, _ in pts if n >= 1024], [u for n, u in pts if n >= 1024], 1)
        per_row_ns, fixed_us = fit[0] * 1e3, fit[1]
        row_b = algorithmic_bytes(t, 1, K) - 4 * K
        res[f"{name} K={K}"] = {"us": {str(n): round(u, 3) for n, u in pts}, "fixed_us": round(fixed_us, 3),
                                "per_row_ns": round(per_row_ns, 4),
                                "marginal_GB/s": round(row_b / per_row_ns, 1)}
        log(f"bench: rows sweep {name} K={K}: " + ", ".join(f"{n}: {u:.2f} us" for n, u in pts) +
            f"; fit {fixed_us:.2f} us + {per_row_ns:.3f} ns/row ({row_b / per_row_ns:.0f} GB/s marginal)")
    return res


DECODE_REPEATS = 3


def decode_leg(n_prompt: int, n_gen: int, cpu: bool):
    """greedy decode of the Qwen2.5-3B-shaped Q4_0 model,
    every matrix-vector product on the GPU (weights resident in HBM), the
    rest of the step on the host.  tok/s = generation-phase passes / their
    wall time.

    The headline runs in ggml-cpu's numerics (MI355X_VARIANT_GGML_Q8: the
    activation row quantized to Q8_0, integer block dots, blocks summed in
    order), the configuration whose tokens follow ggml's CPU path, with the
    config's split -- only the matrix-vector products on the GPU, every GEMV
    group a command to the persistent server kernel, RMSNorm, SiLU and the
    residual adds on the host.  Runs that move more than MUL_MATs to the GPU
    are reported as labelled extras (`beyond_split`).  The digit-plane
    f32-activation mode (the library's default arithmetic) is reported
    beside it.  With `cpu`, the same decode with the oracle's restatement of
    ggml-cpu's arithmetic is the baseline and the headline's token check, and
    the decode with the reference's own CPU engine checks the digit mode."""
    import decode

    cfg = decode.QWEN25_3B
    logical, physical = host_topology()
    threads = min(16, logical)
    t0 = time.perf_counter()
    model = decode.Model(threads=threads, **cfg)
    gemv_bytes = sum(algorithmic_bytes(mi355x.Q4_0, *model.matrix(i)[1:]) for i in range(model.n_matrices()))
    log(f"bench: decode: built the 3B-shape model ({model.weight_bytes() / 2**30:.2f} GiB Q4_0) "
        f"in {time.perf_counter() - t0:.1f} s with {threads} threads")
    prompt = decode.prompt_tokens(n_prompt, cfg["vocab"], seed=512)

    def run():
        # three decodes of the same prompt; the one with the median
        # generation time is reported (host-op time varies between runs on
        # one box by up to ~40%), and all three must pick the same tokens
        runs = [model.generate(prompt, n_gen) for _ in range(DECODE_REPEATS)]
        for toks_i, _ in runs[1:]:
            if not np.array_equal(toks_i, runs[0][0]):
                raise RuntimeError("decode: repeated runs picked different tokens")
        toks, t = sorted(runs, key=lambda r: r[1]["gen_s"])[len(runs) // 2]
        passes = t["gen_passes"]
        return toks, t, passes / t["gen_s"]

    def split(mul_mat_only: bool) -> None:
        # mul_mat_only: one server command per GEMV group, norms, SiLU and
        # residual adds on the host (config 5: only the MUL_MATs on the GPU);
        # else one block command per layer (o .. down and the next q|k|v)
        model.set_swiglu(not mul_mat_only)
        model.set_block(not mul_mat_only)

    def brief(tt, toks, ref, note):
        return {"tok_s": round(tt["gen_passes"] / tt["gen_s"], 2),
                "gemv_ms_per_token": round(tt["gen_gemv_s"] / tt["gen_passes"] * 1e3, 4),
                "host_ms_per_token": round(tt["gen_host_s"] / tt["gen_passes"] * 1e3, 4),
                "tokens_match": bool(np.array_equal(toks, ref)), "note": note}

    try:
        t0 = time.perf_counter()
        model.attach_gpu(0)
        log(f"bench: decode: weights prepacked into HBM in {time.perf_counter() - t0:.1f} s")
        model.set_variant(mi355x.VARIANT_GGML_Q8)
        split(True)
        model.generate(prompt[:8], 4)  # warm-up: first launches of each kernel form
        try:
            gq_toks, t, tok_s = run()
            mode = {0: "stream", 1: "fence", 2: "server"}.get(model.last_wait(), "?")
        except RuntimeError as e:
            log(f"bench: decode: server mode failed ({e}); one launch per group instead")
            model.set_wait(model.WAIT_FENCE)
            gq_toks, t, tok_s = run()
            mode = f"fence (server failed: {e})"
        passes = t["gen_passes"]
        launches = model.last_launches() / passes
        # the same numerics with one launch per group, the host spinning on a
        # completion word or waiting with hipStreamSynchronize
        model.set_wait(model.WAIT_FENCE)
        fence_toks, tf, _ = run()
        model.set_wait(model.WAIT_STREAM)
        sync_toks, tw, _ = run()
        # launch + fence with activations and outputs copied through HBM
        # (staged I/O)
        model.set_wait(model.WAIT_FENCE)
        model.set_io(model.IO_STAGED)
        staged_toks, ts, _ = run()
        model.set_io(model.IO_MAPPED)
        # through the ggml plugin, the drop-in boundary: weights set_tensor'd
        # into its buffer, per group activation in, graph_compute over the
        # group's MUL_MAT nodes, outputs out, synchronize
        model.set_wait(model.WAIT_PLUGIN)
        model.generate(prompt[:8], 4)  # places the weights in the plugin's buffer
        plugin_toks, tp, _ = run()
        plugin_nodes = model.last_launches() / passes
        model.set_plugin_groups(model.PLUGIN_GROUPS_SERVER)
        pl_toks, tpl, _ = run()
        model.set_plugin_groups(model.PLUGIN_GROUPS_LAUNCH)
        model.set_wait(model.WAIT_SERVER)
        # beyond config 5's split: the FFN (gate|up, SiLU, down) as one
        # server command, and whole-layer block commands
        model.set_swiglu(True)
        sw_toks, tsw, _ = run()
        split(False)
        blk_toks, tb, _ = run()
        split(True)
        # the digit-plane f32-activation arithmetic (library default)
        model.set_variant(mi355x.VARIANT_AUTO)
        dg_toks, td, dg_tok_s = run()
        log(f"bench: decode (ggml Q8_0 numerics): launch + fence {passes / tf['gen_s']:.1f} tok/s; "
            f"hipStreamSynchronize waits {passes / tw['gen_s']:.1f} tok/s; staged I/O {passes / ts['gen_s']:.1f} "
            f"tok/s; through the ggml plugin's graph_compute {passes / tp['gen_s']:.1f} tok/s (launches), "
            f"{passes / tpl['gen_s']:.1f} tok/s (server); beyond the "
            f"MUL_MAT split: SwiGLU commands {passes / tsw['gen_s']:.1f}, block commands "
            f"{passes / tb['gen_s']:.1f} tok/s")
        log(f"bench: decode: GPU {tok_s:.1f} tok/s in ggml Q8_0 numerics, MUL_MATs only on the GPU "
            f"({t['gen_s'] / passes * 1e3:.3f} ms/token, GEMV calls {t['gen_gemv_s'] / passes * 1e3:.3f} ms, "
            f"host ops {t['gen_host_s'] / passes * 1e3:.3f} ms); digit-plane mode {dg_tok_s:.1f} tok/s; prompt "
            f"{n_prompt / t['prompt_s']:.1f} tok/s token by token")
        res = {
            "tok_s": round(tok_s, 2), "unit": "tok/s",
            "numerics": "ggml-cpu Q4_0 x Q8_0 (MI355X_VARIANT_GGML_Q8): activations quantized to Q8_0 per "
                        "32-value block, exact integer block dots, (sumi * d_w) * d_x summed in block order per "
                        "row -- the arithmetic of ggml's generic CPU path",
            "workload": f"Qwen2.5-3B shape (36 layers, hidden 2048, 16q/2kv x 128, FFN 11008, vocab 151936, "
                        f"tied), Q4_0 of N(0,0.02), {n_prompt}-token uniform-random prompt then {n_gen} "
                        f"greedy tokens; tok/s over the {passes} generation-phase forward passes, the "
                        f"median-time run of {DECODE_REPEATS} (every mode below likewise)",
            "ms_per_token": round(t["gen_s"] / passes * 1e3, 4),
            "gemv_ms_per_token": round(t["gen_gemv_s"] / passes * 1e3, 4),
            "host_ms_per_token": round(t["gen_host_s"] / passes * 1e3, 4),
            "gemv_bytes_per_token": gemv_bytes,
            "gemv_GB_s": round(gemv_bytes / (t["gen_gemv_s"] / passes) / 1e9, 1),
            "prompt_tok_s": round(n_prompt / t["prompt_s"], 2),
            "gemv_commands_per_token": launches,
            "mode": mode,
            "split": "config 5's split: only the matrix-vector products run on the GPU -- the 253 weight GEMVs "
                     "per token as 145 groups (q|k|v and gate|up, adjacent in HBM, as one job each), one "
                     "command per group to a resident server kernel (mi355x_server_gemv) through pinned host "
                     "memory; RMSNorm, RoPE, the KV cache, attention, SiLU, the residual adds and argmax run "
                     "on the host",
            "fence": brief(tf, fence_toks, gq_toks, "one launch per GEMV group, the host spinning on a completion "
                                                    "word (mi355x_ctx_fence)"),
            "stream_wait": brief(tw, sync_toks, gq_toks, "one launch per GEMV group, then hipStreamSynchronize"),
            "staged_io": brief(ts, staged_toks, gq_toks, "launch + fence with the activation copied host->HBM "
                                                         "and outputs HBM->host around every GEMV group"),
            "plugin": {**brief(tp, plugin_toks, gq_toks,
                               "every GEMV group through the ggml plugin as ggml-backend drives a backend split: "
                               "weights are ggml tensors in the plugin's weight buffer (set_tensor prepacks them), "
                               "activation and outputs tensors of its compute buffer; per group the activation goes "
                               "in (set_tensor_async: into the buffer's page-locked shadow), one graph_compute runs "
                               "the group's MUL_MAT nodes as one launch that reads and writes the shadow and waits "
                               "for it, the outputs come out (get_tensor_async: memcpy), then synchronize"),
                       "mul_mat_nodes_per_token": plugin_nodes,
                       "server_groups": brief(tpl, pl_toks, gq_toks,
                                              "the same, graph_compute sending each group as one command to the "
                                              "device's persistent GEMV server (GGML_MI355X_GROUPS_SERVER)")},
            "beyond_split": {
                "note": "not config 5's split (non-MUL_MAT ops on the GPU); labelled extras",
                "swiglu_commands": brief(tsw, sw_toks, gq_toks, "server commands per GEMV group with gate|up, "
                                         "SiLU and down as one command (SiLU on the GPU)"),
                "block_commands": brief(tb, blk_toks, gq_toks, "one server command per layer: o, residual add, "
                                        "FFN RMSNorm, gate|up, SiLU, down, residual add, the next layer's "
                                        "RMSNorm and q|k|v (norms, SiLU and residual adds on the GPU)"),
            },
            "digit_mode": {"tok_s": round(dg_tok_s, 2),
                           "gemv_ms_per_token": round(td["gen_gemv_s"] / passes * 1e3, 4),
                           "host_ms_per_token": round(td["gen_host_s"] / passes * 1e3, 4),
                           "numerics": "the library's default arithmetic: f32 activations as 20-bit fixed point "
                                       "per 32-value block, int4 dot8 block dots, f32 row sums (within 1e-4 "
                                       "||w|| ||x|| of the reference's f32 GEMV)",
                           "mode": {0: "stream", 1: "fence", 2: "server"}.get(model.last_wait(), "?") +
                                   " (MUL_MATs only on the GPU)"},
        }
        if cpu:
            sys.path.insert(0, os.path.join(ROOT, "oracle"))
            import oracle as orc

            # the headline's check and baseline: every GEMV with ggml-cpu's
            # Q8_0 arithmetic, restated in the oracle (ggml itself is not in
            # this build), OpenMP over rows
            fq, _ = orc.decode_gemv("ggml_q8")
            log("bench: decode: CPU run with the restated ggml Q8_0 arithmetic (baseline, token check)")
            q8_toks, tq = model.generate(prompt, n_gen, fq)
            same = np.array_equal(q8_toks, gq_toks)
            diff = np.nonzero(q8_toks != gq_toks)[0]
            res["token_identical"] = bool(same)
            res["first_mismatch"] = None if same else int(diff[0])
            res["token_check"] = ("the same decode on the CPU with ggml-cpu's Q4_0 x Q8_0 arithmetic restated from "
                                  "ggml's generic C path (quantize_row_q8_0, ggml_vec_dot_q4_0_q8_0); identity "
                                  "with a real ggml build is not checked here (ggml is not in this build)")
            res["cpu_baseline"] = {
                "tok_s": round(passes / tq["gen_s"], 3), "unit": "tok/s", "cores": logical, "kind": "port",
                "sample": f"the same {n_prompt}+{n_gen}-token decode with every GEMV in the restated ggml-cpu "
                          f"Q4_0 x Q8_0 arithmetic (oracle/oracle.c, OpenMP over rows on {logical} threads of a "
                          f"host share of {physical} physical cores) and the same host ops",
                "ms_per_token": round(tq["gen_s"] / passes * 1e3, 3),
            }
            log(f"bench: decode: CPU {passes / tq['gen_s']:.2f} tok/s; GPU tokens identical: {same}")
            # the digit mode against the reference's own CPU GEMV engine
            kind = "reference" if orc.RefLib.available() else "oracle"
            f, cores = orc.decode_gemv(kind)
            ref_toks, tc = model.generate(prompt, n_gen, f)
            d_same = np.array_equal(ref_toks, dg_toks)
            d_diff = np.nonzero(ref_toks != dg_toks)[0]
            res["digit_mode"].update({
                "token_identical_vs_cpu_engine": bool(d_same),
                "first_mismatch": None if d_same else int(d_diff[0]),
                "cpu_engine": ("the reference's AVX2+OpenMP Q4GemvEngine (src/cpu-q4-gemv-engine.cpp)"
                               if kind == "reference" else "the C oracle"),
                "cpu_engine_tok_s": round(passes / tc["gen_s"], 3), "cpu_engine_cores": cores,
                "matching_tokens_vs_ggml_numerics": int(np.sum(q8_toks == dg_toks)),
            })
            log(f"bench: decode: digit mode vs the {kind} CPU engine: tokens identical {d_same}; CPU engine "
                f"{passes / tc['gen_s']:.2f} tok/s")
    finally:
        model.close()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help=f"timed steps of {LAUNCHES_PER_STEP} back-to-back launches each (20: config 2's 1000)")
    ap.add_argument("--warmup", type=int, default=2, help=f"untimed steps of {LAUNCHES_PER_STEP} launches")
    ap.add_argument("--N", type=int, default=8192)
    ap.add_argument("--K", type=int, default=8192)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed launches before the warm-up (GPU clocks out of idle)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep", action="store_true", help="also time the other BASELINE Q4_0 shapes")
    ap.add_argument("--kquants", action="store_true",
                    help="also time the K-quant (14336x4096, 4096x14336) and IQ (8192x8192) BASELINE configs")
    ap.add_argument("--overlap", type=int, default=4, choices=(2, 3, 4),
                    help="streams over which consecutive launches of the headline GEMV may overlap "
                         "(MI355X_OPT_OVERLAP); the --sweep and --kquants shapes use 2, which serves them "
                         "as well as more")
    ap.add_argument("--no-overlap", action="store_true",
                    help="time in-order launches only (one stream): a kernel trace then shows each kernel alone")
    ap.add_argument("--rows-sweep", action="store_true",
                    help="also time IQ2_S (K=8192) and Q4_K (K=4096) at N = 256..32768 rows: fixed cost + per row")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one device-to-device copy of 256 MiB (a plain copy kernel of known size, "
                         "the reference point for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--decode", type=int, default=1, help="1: also run the 3B-shape decode (config 5); 0: skip")
    ap.add_argument("--decode-prompt", type=int, default=512)
    ap.add_argument("--decode-tokens", type=int, default=128)
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "across GPUs the GEMV would shard by output rows (activation broadcast, outputs "
              "all-gathered), which is not built here", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: run without torch.distributed; one GPU only", file=sys.stderr)
        return 2

    N, K, t = args.N, args.K, mi355x.Q4_0
    launches, warm = args.steps * LAUNCHES_PER_STEP, args.warmup * LAUNCHES_PER_STEP
    log(f"bench: generating Q4_0 {N}x{K} (N(0,0.02) -> Q4_0) and x ~ N(0,1)")
    raw = synth.quantize_q4_0(synth.normal_weights(N, K, seed=42))
    x = synth.activations(K, seed=43)
    alg = algorithmic_bytes(t, N, K)

    with mi355x.Context(0) as ctx:
        if args.copy_calibration:
            nbytes = 256 << 20
            src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
            mi355x.check(ctx.lib.mi355x_fill(ctx.h, src.ptr, 1, nbytes))
            mi355x.check(ctx.lib.mi355x_memcpy_d2d(ctx.h, dst.ptr, src.ptr, nbytes))
            src.free()
            dst.free()
            log(f"bench: copy calibration: one {nbytes} B device-to-device copy done")
        name, pci = ctx.describe()
        log(f"bench: device {name} at {pci}; timing {args.steps} steps of {LAUNCHES_PER_STEP} launches "
            f"({launches} launches in one window) after {warm} warm-up launches")
        overlap = 0 if args.no_overlap else args.overlap
        ms_seq, copies, y_seq = gemv_rate(ctx, t, raw, N, K, x, launches, warm, ROTATE_BYTES, args.settle)
        log(f"bench: in order (one stream) {ms_seq * 1e3:.2f} us/launch over {copies} resident copies")
        ms, y = ms_seq, y_seq
        if overlap:
            ms, _, y = gemv_rate(ctx, t, raw, N, K, x, launches, warm, ROTATE_BYTES, args.settle,
                                 overlap=overlap)
            log(f"bench: {ms * 1e3:.2f} us/launch with consecutive launches overlapping")
            if not np.array_equal(y, y_seq):
                raise RuntimeError("overlapped and in-order launches disagree")
        ms_hot, _, _ = gemv_rate(ctx, t, raw, N, K, x, launches, warm, 0, args.settle)
        log(f"bench: cache-hot (one copy) {ms_hot * 1e3:.2f} us/launch")
        # the other arithmetic variants on the same workload
        variants = {}
        for vname, v in (("exact_f32", mi355x.VARIANT_EXACT_F32), ("ggml_q8", mi355x.VARIANT_GGML_Q8)):
            ctx.set_option(mi355x.OPT_VARIANT, v)
            try:
                msv, _, _ = gemv_rate(ctx, t, raw, N, K, x, launches, warm, ROTATE_BYTES, args.settle)
            finally:
                ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
            gv = alg / (msv * 1e-3) / 1e9
            variants[vname] = {"us_per_launch": round(msv * 1e3, 3), "GB/s": round(gv, 1),
                               "frac": round(gv / HBM_PEAK_GBS, 4)}
            log(f"bench: variant {vname}: {msv * 1e3:.2f} us/launch, {gv:.1f} GB/s")
        sweep = {}
        if args.sweep:
            for (n2, k2) in ((4096, 4096), (17408, 5120), (151936, 2048)):
                raw2 = synth.quantize_q4_0(synth.normal_weights(n2, k2, seed=42))
                x2 = synth.activations(k2, seed=43)
                ms2, c2, _ = gemv_rate(ctx, t, raw2, n2, k2, x2, launches, warm, ROTATE_BYTES, args.settle)
                gbs2 = algorithmic_bytes(t, n2, k2) / (ms2 * 1e-3) / 1e9
                mso = gemv_rate(ctx, t, raw2, n2, k2, x2, launches, warm, ROTATE_BYTES, args.settle,
                                overlap=overlap)[0] if overlap else ms2
                gbo = algorithmic_bytes(t, n2, k2) / (mso * 1e-3) / 1e9
                sweep[f"{n2}x{k2}"] = {"us": round(ms2 * 1e3, 3), "GB/s": round(gbs2, 1),
                                       "frac": round(gbs2 / HBM_PEAK_GBS, 4), "copies": c2,
                                       "us_overlap": round(mso * 1e3, 3), "frac_overlap": round(gbo / HBM_PEAK_GBS, 4),
                                       "overlap_streams": overlap}
                log(f"bench: Q4_0 {n2}x{k2}: {ms2 * 1e3:.2f} us, {gbs2:.1f} GB/s; overlapped {mso * 1e3:.2f} us "
                    f"({gbo / HBM_PEAK_GBS:.1%})")

        kq = {}
        if args.kquants:
            kq = kquant_sweep(ctx, launches, warm, args.settle, min(overlap, 2))
        rs = rows_sweep(ctx, launches, warm, args.settle) if args.rows_sweep else {}

    # the timed output must still be the right answer (checked, not measured)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle
    ref = Oracle().gemv(2, raw, N, K, x)
    cos = float(np.dot(y.astype(np.float64), ref) / (np.linalg.norm(y) * np.linalg.norm(ref)))

    gbs = alg / (ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms * LAUNCHES_PER_STEP, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(gbs / REFERENCE_GBS, 2),
        "baseline_note": f"value / {REFERENCE_GBS} GB/s, the reference's published Q4_0 8192x8192 GEMV rate "
                         "(README.md:98, host CPU, weight bytes only)",
        "dtype": "q4_0 x fx20 (int4 dot8)",
        "arithmetic": "Q4_0 weights (4-bit codes, fp16 block scales) times f32 activations: each 32-value "
                      "activation block as 20-bit fixed point (5 signed 4-bit digit planes, power-of-two block "
                      "scale), block dots exact in int32 with v_dot8_i32_i4, f32 scale-and-sum per row; inputs "
                      "and outputs f32",
        "data": "synthetic: f32 N(0,0.02) weights (seed 42) quantized to Q4_0, x ~ N(0,1) (seed 43)",
        "config": {"workload": f"Q4_0 GEMV {N}x{K} (N rows x K), 1 f32 activation row; one step = "
                               f"{LAUNCHES_PER_STEP} back-to-back launches, {launches} launches in the timed "
                               f"window; weights rotated over {copies} resident copies "
                               f"({copies * (alg - 4 * K - 4 * N) / 2**30:.2f} GiB) so HBM, not cache, serves them; "
                               + (f"back-to-back independent launches, up to {overlap} in flight ({overlap} streams)" if overlap
                                  else "back-to-back launches on one stream"),
                   "N": N, "K": K, "weight_type": "Q4_0", "rotate_copies": copies,
                   "launches_per_step": LAUNCHES_PER_STEP, "launches_timed": launches,
                   "launch_overlap": overlap, "parallelism": "single GPU"},
        # the roofline of the kernel: its own duration, which in-order
        # launches expose (each starts after the previous one ends, so the
        # HIP-event interval is the kernel plus the dispatch gap) and which a
        # rocprofv3 kernel trace of the same command reports; overlapped
        # launches sustain `value`, but a trace serialises them
        "roofline": {"bound": "hbm", "achieved": round(alg / (ms_seq * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(alg / (ms_seq * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "note": f"achieved = {alg} algorithmic bytes per launch / {ms_seq * 1e3:.3f} us, the mean "
                             f"interval of {launches} in-order launches on the library's stream (HIP events): the "
                             "kernel's duration plus the dispatch gap, the figure a rocprofv3 kernel trace of the "
                             "same command gives per dispatch; with up to "
                             f"{overlap or 1} launches in flight the same kernel sustains `value`"},
        "in_order": {"us_per_launch": round(ms_seq * 1e3, 3), "GB/s": round(alg / (ms_seq * 1e-3) / 1e9, 2),
                     "frac": round(alg / (ms_seq * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "note": "the same launches on one stream, each starting after the previous one ends "
                             "(includes the gap between kernels); this is the rate a caller whose GEMVs depend "
                             "on each other sees -- the decode and the plugin's graph_compute"},
        "overlapped": {"us_per_launch": round(ms * 1e3, 3), "GB/s": round(gbs, 2),
                       "frac": round(gbs / HBM_PEAK_GBS, 4), "streams": overlap,
                       "note": "`value`: consecutive independent launches, up to `streams` in flight "
                               "(MI355X_OPT_OVERLAP), HIP events on the library's stream after it has joined the "
                               "others; each launch's start overlaps the previous ones' drain"},
        "cache_hot": {"us_per_launch": round(ms_hot * 1e3, 3),
                      "GB/s": round(alg / (ms_hot * 1e-3) / 1e9, 2),
                      "note": "single resident copy, served partly from MALL/L2; not the HBM figure"},
        "parity": {"cosine_vs_oracle": cos},
        "variants": {**variants,
                     "note": "the same workload in the library's other arithmetic variants: exact_f32 (codes to "
                             "f32, fp32 FMA, activations exactly as given) and ggml_q8 (ggml-cpu's Q8_0 "
                             "activation numerics, blocks summed in order)"},
    }
    if sweep:
        out["sweep"] = sweep
    if kq:
        out["kquants"] = kq
        out["kquants_data"] = ("f32 N(0,0.02) weights (seed 7; IQ types with 1% of them x8) quantized per type by "
                               "synth.quantize_kq, x ~ N(0,1) (seed 43); IQ3_XXS/IQ2_S on synthetic grids")
    if rs:
        out["rows_sweep"] = rs
    if not args.no_cpu:
        log(f"bench: CPU baseline for ~{args.cpu_seconds:.0f} s")
        out["cpu_baseline"] = cpu_baseline(raw, N, K, x, args.cpu_seconds)
    if args.decode:
        try:
            out["decode"] = decode_leg(args.decode_prompt, args.decode_tokens, not args.no_cpu)
        except Exception as e:  # the GEMV line above stands on its own
            log(f"bench: decode leg failed: {e}")
            out["decode"] = {"error": str(e)}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
