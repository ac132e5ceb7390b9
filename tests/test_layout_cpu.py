"""The K/IQ resident layouts (xdna.cpp_amd/csrc/kq_layout.h) on the CPU: for
every type, row length and row alignment, the ggml -> resident byte map is a
bijection of the row, and every unit a GEMV lane fetches with one load
instruction lies contiguous, in ggml order, at an address aligned as that
load needs (4 for dword loads, 2 for the fp16 d).  The header is compiled
with g++ into a tiny helper; no GPU involved."""
import ctypes as C
import os
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "xdna.cpp_amd", "csrc")

HELPER = r"""
#include "kq_layout.h"
extern "C" int kq_block_bytes(int t) { return mi355x::kq_layout(t).block_bytes; }
extern "C" int kq_nfields(int t) { return mi355x::kq_layout(t).nfields; }
extern "C" int kq_grouped(int t) { return mi355x::kq_layout(t).grouped ? 1 : 0; }
extern "C" void kq_field(int t, int i, int *off, int *len) {
    auto L = mi355x::kq_layout(t); *off = L.f[i].off; *len = L.f[i].len;
}
extern "C" void kq_map_row(int t, unsigned long long B, int flipped, unsigned long long *out) {
    auto L = mi355x::kq_layout(t);
    for (unsigned long long b = 0; b < B; ++b)
        for (int e = 0; e < L.block_bytes; ++e)
            out[b * L.block_bytes + e] = mi355x::kq_row_offset(L, b, e, B, flipped != 0);
}
"""

TYPES = {"Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ3_XXS": 18, "IQ3_S": 21, "IQ2_S": 22, "IQ4_XS": 23}
BLOCK = {11: 110, 12: 144, 13: 176, 14: 210, 18: 98, 21: 110, 22: 82, 23: 136}
GROUPED = {11, 14, 18, 21, 22}


def r(a, n):
    return list(range(a, a + n))


def load_units(t, s):
    """(ggml bytes in load order, alignment) of each load slice s of a block
    issues, as the kernels' Kq<TYPE>::load does (include/xdna/kquants.h
    field order restated in kq_layout.h)."""
    hh, k = s >> 2, s & 3
    if t == 12:  # Q4_K: 16 code bytes, the 16-byte head
        return [(r(16 + 16 * s, 16), 4), (r(0, 16), 4)]
    if t == 13:  # Q5_K: codes, the 16 high-bit bytes of half h, head
        return [(r(48 + 16 * s, 16), 4), (r(16 + 16 * (s & 1), 16), 4), (r(0, 16), 4)]
    if t == 23:  # IQ4_XS
        return [(r(8 + 16 * s, 16), 4), (r(0, 8), 4)]
    if t == 11:  # Q3_K: codes + half of the shared hmask bytes, scales, d
        # scales: the low-nibble bytes as words kk = 0, 1 ([kk], [kk + 4],
        # [kk + 2], [kk + 6]), then scales[8..11]
        lo = [96 + kk + 2 * j for kk in (0, 1) for j in (0, 2, 1, 3)]
        return [(r(32 + 8 * s, 8) + r(8 * k + 4 * hh, 4), 4), (lo + r(104, 4), 4), (r(108, 2), 2)]
    if t == 14:  # Q6_K: ql, ql, qh runs; one scale word; d
        kk = k >> 1
        return [(r(64 * hh + 8 * k, 8) + r(64 * hh + 32 + 8 * k, 8) + r(128 + 32 * hh + 8 * k, 8), 4),
                ([192 + 8 * hh + kk + 2 * j for j in range(4)], 4), (r(208, 2), 2)]
    if t == 21:  # IQ3_S: qs + signs; qh byte; 4 scale bytes; d
        return [(r(2 + 8 * s, 8) + r(74 + 4 * s, 4), 4), ([66 + s], 1), (r(106, 4), 4), (r(0, 2), 2)]
    if t == 18:  # IQ3_XXS: qs + scales_and_signs word; d
        return [(r(2 + 8 * s, 8) + r(66 + 4 * s, 4), 4), (r(0, 2), 2)]
    if t == 22:  # IQ2_S: qs + signs; qh and scale bytes; d
        return [(r(2 + 4 * s, 4) + r(34 + 4 * s, 4), 4), ([66 + s, 74 + s], 2), (r(0, 2), 2)]
    raise ValueError(t)


@pytest.fixture(scope="module")
def layout():
    d = tempfile.mkdtemp(prefix="kqlayout")
    src = os.path.join(d, "h.cpp")
    so = os.path.join(d, "h.so")
    open(src, "w").write(HELPER)
    subprocess.run(["g++", "-std=c++17", "-O1", "-shared", "-fPIC", "-I", CSRC, src, "-o", so], check=True)
    lib = C.CDLL(so)
    lib.kq_map_row.argtypes = [C.c_int, C.c_ulonglong, C.c_int, C.POINTER(C.c_ulonglong)]
    return lib


def row_map(layout, t, B, flipped):
    out = (C.c_ulonglong * (B * BLOCK[t]))()
    layout.kq_map_row(t, B, int(flipped), out)
    return np.ctypeslib.as_array(out).astype(np.int64).reshape(B, BLOCK[t])


@pytest.mark.parametrize("name", list(TYPES))
def test_fields_tile_the_ggml_block(layout, name):
    t = TYPES[name]
    assert layout.kq_block_bytes(t) == BLOCK[t]
    assert layout.kq_grouped(t) == (t in GROUPED)
    covered = np.zeros(BLOCK[t], dtype=int)
    off, ln = C.c_int(), C.c_int()
    for i in range(layout.kq_nfields(t)):
        layout.kq_field(t, i, C.byref(off), C.byref(ln))
        covered[off.value:off.value + ln.value] += 1
    assert np.all(covered == 1)
    # the load units of the 8 slices cover the block (shared units repeat)
    seen = set()
    for s in range(8):
        for unit, _ in load_units(t, s):
            seen.update(unit)
    assert seen == set(range(BLOCK[t]))


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("B", [1, 2, 3, 7, 8, 9, 16, 43, 56, 61])
def test_row_map_is_a_bijection_with_aligned_load_units(layout, name, B):
    t = TYPES[name]
    row_bytes = B * BLOCK[t]
    # rows of a 256-aligned tensor start at r * row_bytes: only 0 or 2 mod 4
    for row_addr in sorted({(i * row_bytes) % 16 for i in range(8)}):
        flipped = (row_addr & 3) == 2
        m = row_map(layout, t, B, flipped)
        assert np.array_equal(np.sort(m.reshape(-1)), np.arange(row_bytes)), "not a bijection"
        for b in range(B):
            for s in range(8):
                for unit, align in load_units(t, s):
                    o = m[b, unit]
                    assert np.all(np.diff(o) == 1), (name, B, b, s, unit[:3])
                    assert (row_addr + o[0]) % align == 0, (name, B, row_addr, b, s, unit[:3])


@pytest.mark.parametrize("name", ["Q3_K", "Q6_K", "IQ3_S", "IQ3_XXS", "IQ2_S"])
@pytest.mark.parametrize("B", [8, 16, 56])
def test_lane_records_of_a_step_form_one_span(layout, name, B):
    """In a full group of 8 superblocks, the lane records of the 64 lanes
    (lane = 8 s + bl) follow one another: one load instruction per step
    covers a contiguous span."""
    t = TYPES[name]
    m = row_map(layout, t, B, False)
    for g in range(B // 8):
        starts = []
        for lane in range(64):
            s, bl = lane // 8, lane % 8
            unit, _ = load_units(t, s)[0]
            starts.append(m[8 * g + bl, unit[0]])
        d = np.diff(starts)
        assert np.all(d == len(load_units(t, 0)[0][0])), (name, g, d[:8])
