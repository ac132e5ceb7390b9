"""The C-ABI library loads and exports every symbol declared in include/*.h;
pure (device-free) entry points behave as documented."""
import os
import re

import numpy as np

import mi355x

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", fn)).read()
        names += re.findall(r"^(?:MI355X_API|GGML_MI355X_API)\s+[^;(]*?\b(\w+)\s*\(", text, re.M)
    return names


def test_every_declared_symbol_is_exported():
    lib = mi355x.load()
    names = declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_row_bytes_matches_block_geometry():
    # include/xdna/kquants.h:182-200
    assert mi355x.row_bytes(mi355x.Q4_0, 4096) == 128 * 18
    assert mi355x.row_bytes(mi355x.Q4_0, 33) == -1
    for t, bb in mi355x.BLOCK_BYTES.items():
        bv = mi355x.BLOCK_VALUES[t]
        assert mi355x.row_bytes(t, 4 * bv) == 4 * bb
        assert mi355x.row_bytes(t, bv + 1) == -1
    assert mi355x.row_bytes(99, 256) == -1


def test_type_ready_and_grid_validation():
    for t in (mi355x.Q4_0, mi355x.Q3_K, mi355x.Q4_K, mi355x.Q5_K, mi355x.Q6_K, mi355x.IQ4_XS, mi355x.IQ3_S):
        assert mi355x.type_ready(t)
    assert not mi355x.type_ready(mi355x.F32)
    lib = mi355x.load()
    bad = np.zeros(10, dtype=np.uint8)
    assert lib.mi355x_set_iq_grid(mi355x.IQ3_XXS, bad.ctypes.data, bad.nbytes) == mi355x.EINVAL
    assert "1024 bytes" in mi355x.last_error()
    assert lib.mi355x_set_iq_grid(mi355x.Q4_0, bad.ctypes.data, bad.nbytes) == mi355x.EINVAL
    # magnitudes outside 1..127 (the kernels negate bytes carry-free)
    for bad_byte in (0, 128, 255):
        g = np.full(1024, 43, dtype=np.uint8)
        g[517] = bad_byte
        assert lib.mi355x_set_iq_grid(mi355x.IQ3_XXS, g.ctypes.data, g.nbytes) == mi355x.EINVAL
        assert "1..127" in mi355x.last_error()


def test_device_count_does_not_crash_without_gpu():
    assert mi355x.device_count() >= 0
