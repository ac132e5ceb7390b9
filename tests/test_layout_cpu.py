"""The K/IQ field-plane layout (xdna.cpp_amd/csrc/kq_layout.h) on the CPU:
for every type, row length and row alignment, the ggml -> resident byte map
is a bijection of the row, keeps each field's bytes together, and puts every
record of a plane at an address aligned to min(4, record size) -- the
property the kernels' dword loads rely on.  The header is compiled with g++
into a tiny helper; no GPU involved."""
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


@pytest.mark.parametrize("name", list(TYPES))
def test_fields_tile_the_ggml_block(layout, name):
    t = TYPES[name]
    assert layout.kq_block_bytes(t) == BLOCK[t]
    covered = np.zeros(BLOCK[t], dtype=int)
    off, ln = C.c_int(), C.c_int()
    for i in range(layout.kq_nfields(t)):
        layout.kq_field(t, i, C.byref(off), C.byref(ln))
        covered[off.value:off.value + ln.value] += 1
    assert np.all(covered == 1)


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("B", [1, 2, 3, 7, 16, 43, 56])
def test_row_map_is_an_aligned_bijection(layout, name, B):
    t = TYPES[name]
    bb = BLOCK[t]
    row_bytes = B * bb
    off, ln = C.c_int(), C.c_int()
    fields = []
    for i in range(layout.kq_nfields(t)):
        layout.kq_field(t, i, C.byref(off), C.byref(ln))
        fields.append((off.value, ln.value))
    # rows of a 256-aligned tensor start at r * row_bytes: only 0 or 2 mod 4
    for row_addr in sorted({(r * row_bytes) % 16 for r in range(8)}):
        flipped = (row_addr & 3) == 2
        out = (C.c_ulonglong * row_bytes)()
        layout.kq_map_row(t, B, int(flipped), out)
        m = np.ctypeslib.as_array(out).astype(np.int64)
        assert np.array_equal(np.sort(m), np.arange(row_bytes)), "not a bijection"
        m = m.reshape(B, bb)
        for fo, fl in fields:
            rec = m[:, fo:fo + fl]
            # a field's bytes stay contiguous and in order, blocks in order
            assert np.all(np.diff(rec, axis=1) == 1)
            assert np.all(np.diff(rec[:, 0]) == fl)
            align = min(4, fl)
            assert np.all((row_addr + rec[:, 0]) % align == 0), (name, B, row_addr, fo, fl)
