"""Phase timeline of GEMV-server commands at the 3B decode shapes.

Needs the stamps build of the library (`make -C xdna.cpp_amd stamps`:
libggml-mi355x-stamps.so, the server kernel with MI355X_SRV_STAMPS), in
which thread 0 of every workgroup records s_memrealtime (100 MHz) at fixed
points of the last 64 commands.  For each command kind this prints, per
point, the median over 64 commands of the slowest workgroup's time from the
moment workgroup 0 saw the command, and the host's time per call.

    python3 xdna.cpp_amd/server_phases.py
"""
import ctypes
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import mi355x  # noqa: E402

SLOTS = 20
NAMES = {1: "record and x read", 2: "stage 0 staged", 3: "stage 0 rows done", 4: "stage 1 staged",
         5: "stage 1 rows done", 6: "stage 2 staged", 7: "stage 2 rows done", 8: "stage 3 staged",
         9: "stage 3 rows done", 10: "last stores done", 11: "arrived", 12: "completion stored",
         13: "stage 1 barrier passed", 14: "stage 2 barrier passed", 15: "stage 3 barrier passed",
         16: "last RMSNorm: r read", 17: "last RMSNorm: sums done", 18: "last RMSNorm: done"}
ORDER = [1, 2, 3, 13, 4, 5, 14, 6, 7, 15, 16, 17, 18, 8, 9, 10, 11, 12]


def random_q4_0(N, K, seed):
    """Random Q4_0 bytes: f16 scales of about 0.01, random nibbles."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(N, K // 32, 18), dtype=np.uint8)
    d = (rng.uniform(0.005, 0.015, size=(N, K // 32)).astype(np.float16)).view(np.uint8).reshape(N, K // 32, 2)
    b[:, :, :2] = d
    return b.reshape(-1)


def stamps(lib):
    a = np.zeros((64, 256, SLOTS), np.uint64)
    mi355x.check(lib.mi355x_server_stamps(a.ctypes.data))
    return a.astype(np.int64)


def report(name, st, host_us):
    print(f"\n{name}: {host_us:.2f} us per call (host)\n\n| point | us (slowest workgroup) |\n|---|---:|")
    for k in ORDER:
        vals = []
        for slot in range(64):
            v = (st[slot, :, k] - st[slot, 0, 0]) / 100.0
            v = v[(v > -50) & (v < 500)]
            if v.size:
                vals.append(v.max())
        if len(vals) >= 32:
            print(f"| {NAMES[k]} | {np.median(vals):.2f} |")
    sys.stdout.flush()


def main():
    lib = mi355x.load(os.path.join(HERE, "libggml-mi355x-stamps.so"))
    lib.mi355x_server_stamps.argtypes = [ctypes.c_void_p]
    lib.mi355x_server_stamps.restype = ctypes.c_int
    H, F, QKV = 2048, 11008, 2560
    rng = np.random.default_rng(1)
    with mi355x.Context(0) as ctx:
        srv = mi355x.Server(ctx, 16384)
        res = lambda N, K, seed: ctx.resident(mi355x.Q4_0, random_q4_0(N, K, seed), N, K)  # noqa: E731
        qkv, o, gate, up, down, lm = res(QKV, H, 1), res(H, H, 2), res(F, H, 3), res(F, H, 4), res(H, F, 5), \
            res(151936, H, 6)
        y = ctx.alloc(4 * 151936)
        yq = ctx.alloc(4 * QKV)
        nw = ctx.to_device(rng.uniform(0.5, 1.5, H).astype(np.float32))
        x = rng.standard_normal(H).astype(np.float32)
        resid = rng.standard_normal(H).astype(np.float32)
        cases = [
            ("q|k|v, 2560 x 2048", lambda: srv.gemv(x, [(qkv.ptr, QKV, y.ptr)])),
            ("vocabulary, 151936 x 2048", lambda: srv.gemv(x, [(lm.ptr, 151936, y.ptr)])),
            ("layer block (o, norm, gate|up, SiLU, down) + next q|k|v, residual kept",
             lambda: srv.block(x, o.ptr, H, nw.ptr, 1e-6, gate.ptr, up.ptr, F, down.ptr, 0, nw.ptr, qkv.ptr, QKV,
                               yq.ptr)),
        ]
        for variant, vname in ((mi355x.VARIANT_AUTO, "digit numerics"), (mi355x.VARIANT_GGML_Q8, "ggml numerics")):
            ctx.set_option(mi355x.OPT_VARIANT, variant)
            srv.block(x, o.ptr, resid, nw.ptr, 1e-6, gate.ptr, up.ptr, F, down.ptr, 0)  # leaves a residual
            for name, fn in cases:
                for _ in range(100):
                    fn()
                t0 = time.perf_counter()
                for _ in range(64):
                    fn()
                host = (time.perf_counter() - t0) / 64 * 1e6
                srv.stop()
                report(f"{name}, {vname}", stamps(lib), host)
        ctx.set_option(mi355x.OPT_VARIANT, mi355x.VARIANT_AUTO)
        srv.close()
        for b in (qkv, o, gate, up, down, lm, y, yq, nw):
            b.free()


if __name__ == "__main__":
    main()
