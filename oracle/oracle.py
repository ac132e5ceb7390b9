"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, by ``__graft_entry__.smoke()`` and by ``bench.py``'s
``cpu_baseline`` leg, and nowhere else.  Two libraries live here:

* ``liboracle.so`` -- the plain-C restatement in ``oracle.c`` (numerics
  contract in ``oracle.h``);
* ``_ref/libxdna_ref.so`` -- the reference's own CPU sources built by
  ``oracle/Makefile`` from /root/reference (optional; absent where the
  reference was never built).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libxdna_ref.so")

# ggml type ids
Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS = 2, 11, 12, 13, 14, 18, 21, 22, 23
ALL_TYPES = (Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS)
TYPE_NAMES = {Q4_0: "Q4_0", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS"}
GRID_TYPES = (IQ3_XXS, IQ2_S)

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            subprocess.run(["make", "-s", "-C", HERE, "oracle"], check=True)
        lib = ctypes.CDLL(path)
        lib.orc_fp16_to_f32.restype = ctypes.c_float
        lib.orc_fp16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_bf16_to_f32.restype = ctypes.c_float
        lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.orc_row_bytes.restype = ctypes.c_int64
        lib.orc_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        lib.orc_block_values.restype = ctypes.c_int64
        lib.orc_block_values.argtypes = [ctypes.c_int]
        lib.orc_block_bytes.restype = ctypes.c_int64
        lib.orc_block_bytes.argtypes = [ctypes.c_int]
        lib.orc_q4_0_validate_row.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        lib.orc_q4_0_validate_matrix.argtypes = [ctypes.c_uint64] * 3
        lib.orc_dequant_row.argtypes = [ctypes.c_int, _u8p, ctypes.c_int64, _f32p, ctypes.c_void_p]
        lib.orc_gemv_f32.argtypes = [ctypes.c_int, _u8p, ctypes.c_int64, ctypes.c_int64,
                                     _f32p, _f32p, ctypes.c_void_p]
        lib.orc_gemv_bf16.argtypes = [ctypes.c_int, _u8p, ctypes.c_int64, ctypes.c_int64,
                                      _u16p, _f32p, ctypes.c_void_p]
        lib.orc_row_norms.argtypes = [ctypes.c_int, _u8p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.POINTER(ctypes.c_double), ctypes.c_void_p]
        lib.orc_ksigns_iq2xs.restype = ctypes.c_uint8
        lib.orc_ksigns_iq2xs.argtypes = [ctypes.c_int]
        lib.orc_f32_to_fp16.restype = ctypes.c_uint16
        lib.orc_f32_to_fp16.argtypes = [ctypes.c_float]
        lib.orc_quantize_row_q8_0.argtypes = [_f32p, ctypes.c_int64, _u8p]
        lib.orc_gemv_q4_0_q8_0.argtypes = [_u8p, ctypes.c_int64, ctypes.c_int64, _f32p, _f32p]
        lib.orc_quantize_row_q8_K.argtypes = [_f32p, ctypes.c_int64, _u8p]
        lib.orc_gemv_q8_K.argtypes = [ctypes.c_int, _u8p, ctypes.c_int64, ctypes.c_int64, _f32p, _f32p,
                                      ctypes.c_void_p]
        self.lib = lib

    # ggml-cpu numerics (external restatement; see oracle.c)
    def f32_to_fp16(self, f: float) -> int:
        return self.lib.orc_f32_to_fp16(f)

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
        if self.lib.orc_quantize_row_q8_0(_ptr(x, _f32p), x.size, _ptr(out, _u8p)) != 0:
            raise ValueError("orc_quantize_row_q8_0 rejected the row")
        return out

    def gemv_q4_0_q8_0(self, W: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.uint8).reshape(-1)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(N, dtype=np.float32)
        if self.lib.orc_gemv_q4_0_q8_0(_ptr(W, _u8p), N, K, _ptr(x, _f32p), _ptr(y, _f32p)) != 0:
            raise ValueError("orc_gemv_q4_0_q8_0 rejected the shape")
        return y

    Q8K_BYTES = 292

    def quantize_q8_K(self, x: np.ndarray):
        """Q8_K blocks of an activation row: (d[nb] f32, qs[nb, 256] int8,
        bsums[nb, 16] int16)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        nb = x.size // 256
        out = np.zeros(nb * self.Q8K_BYTES, dtype=np.uint8)
        if self.lib.orc_quantize_row_q8_K(_ptr(x, _f32p), x.size, _ptr(out, _u8p)) != 0:
            raise ValueError("orc_quantize_row_q8_K rejected the row")
        blk = out.reshape(nb, self.Q8K_BYTES)
        return (blk[:, 0:4].copy().view(np.float32).reshape(nb), blk[:, 4:260].copy().view(np.int8),
                blk[:, 260:292].copy().view(np.int16))

    def gemv_q8_K(self, t: int, W: np.ndarray, N: int, K: int, x: np.ndarray, grid=None) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.uint8).reshape(-1)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(N, dtype=np.float32)
        g = None if grid is None else np.ascontiguousarray(grid)
        rc = self.lib.orc_gemv_q8_K(t, _ptr(W, _u8p), N, K, _ptr(x, _f32p), _ptr(y, _f32p),
                                    None if g is None else g.ctypes.data)
        if rc != 0:
            raise ValueError(f"orc_gemv_q8_K rc={rc}")
        return y

    def fp16_to_f32(self, h: int) -> float:
        return self.lib.orc_fp16_to_f32(h)

    def bf16_to_f32(self, b: int) -> float:
        return self.lib.orc_bf16_to_f32(b)

    def f32_to_bf16(self, f: float) -> int:
        return self.lib.orc_f32_to_bf16(f)

    def row_bytes(self, t: int, K: int) -> int:
        return self.lib.orc_row_bytes(t, K)

    def block_values(self, t: int) -> int:
        return self.lib.orc_block_values(t)

    def block_bytes(self, t: int) -> int:
        return self.lib.orc_block_bytes(t)

    def dequant_row(self, t: int, row: np.ndarray, K: int, grid=None) -> np.ndarray:
        row = np.ascontiguousarray(row, dtype=np.uint8)
        out = np.empty(K, dtype=np.float32)
        g = None if grid is None else np.ascontiguousarray(grid)
        rc = self.lib.orc_dequant_row(t, _ptr(row, _u8p), K, _ptr(out, _f32p),
                                      None if g is None else g.ctypes.data)
        if rc != 0:
            raise ValueError(f"orc_dequant_row rc={rc}")
        return out

    def gemv(self, t: int, W: np.ndarray, N: int, K: int, x: np.ndarray, grid=None) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.uint8)
        rb = self.row_bytes(t, K)
        if rb < 0 or W.size < N * rb:
            raise ValueError("weight buffer does not hold N rows")
        y = np.empty(N, dtype=np.float32)
        g = None if grid is None else np.ascontiguousarray(grid)
        if x.dtype == np.uint16:
            x = np.ascontiguousarray(x)
            rc = self.lib.orc_gemv_bf16(t, _ptr(W, _u8p), N, K, _ptr(x, _u16p), _ptr(y, _f32p),
                                        None if g is None else g.ctypes.data)
        else:
            x = np.ascontiguousarray(x, dtype=np.float32)
            rc = self.lib.orc_gemv_f32(t, _ptr(W, _u8p), N, K, _ptr(x, _f32p), _ptr(y, _f32p),
                                       None if g is None else g.ctypes.data)
        if rc != 0:
            raise ValueError(f"orc_gemv rc={rc}")
        return y

    def row_norms(self, t: int, W: np.ndarray, N: int, K: int, grid=None) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.uint8)
        out = np.empty(N, dtype=np.float64)
        g = None if grid is None else np.ascontiguousarray(grid)
        rc = self.lib.orc_row_norms(t, _ptr(W, _u8p), N, K, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                    None if g is None else g.ctypes.data)
        if rc != 0:
            raise ValueError(f"orc_row_norms rc={rc}")
        return out

    def ksigns(self) -> np.ndarray:
        return np.array([self.lib.orc_ksigns_iq2xs(i) for i in range(128)], dtype=np.uint8)


class RefLib:
    """The reference's own CPU code (oracle/_ref/libxdna_ref.so)."""

    def __init__(self, path: str = REF_SO):
        lib = ctypes.CDLL(path)
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_fp16_to_f32.restype = ctypes.c_float
        lib.ref_fp16_to_f32.argtypes = [ctypes.c_uint16]
        lib.ref_bf16_to_f32.restype = ctypes.c_float
        lib.ref_bf16_to_f32.argtypes = [ctypes.c_uint16]
        lib.ref_f32_to_bf16.restype = ctypes.c_uint16
        lib.ref_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.ref_q4_0_validate_row.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        lib.ref_q4_0_validate_matrix.argtypes = [ctypes.c_uint64] * 3
        lib.ref_q4_0_gemv_f32.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                          _f32p, ctypes.c_uint64, _f32p, ctypes.c_uint64]
        lib.ref_q4_0_gemv_bf16.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                           _u16p, ctypes.c_uint64, _f32p, ctypes.c_uint64]
        lib.ref_q4_0_dequantize_row.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p]
        lib.ref_gemv_kq.argtypes = [ctypes.c_int, _u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p, _f32p]
        lib.ref_dequant_kq.argtypes = [ctypes.c_int, _u8p, ctypes.c_uint64, _f32p]
        lib.ref_cpu_engine_new.restype = ctypes.c_void_p
        lib.ref_cpu_engine_free.argtypes = [ctypes.c_void_p]
        lib.ref_cpu_engine_run.argtypes = [ctypes.c_void_p, _u8p, ctypes.c_uint64, ctypes.c_uint64,
                                           ctypes.c_uint64, _f32p, _f32p]
        lib.ref_prepack_layout.argtypes = [ctypes.c_uint64] * 3 + [ctypes.POINTER(ctypes.c_uint64)]
        lib.ref_prepack_pack.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, _u8p, ctypes.c_uint64]
        lib.ref_prepack_dequant.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, _f32p, ctypes.c_uint64]
        lib.ref_iq3s_grid.argtypes = [ctypes.POINTER(ctypes.c_uint32)]
        self.lib = lib

    @staticmethod
    def available(path: str = REF_SO) -> bool:
        return os.path.exists(path)

    def error(self) -> str:
        return self.lib.ref_last_error().decode()

    def gemv(self, t: int, W: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
        W = np.ascontiguousarray(W, dtype=np.uint8)
        y = np.empty(N, dtype=np.float32)
        if t == Q4_0:
            if x.dtype == np.uint16:
                rc = self.lib.ref_q4_0_gemv_bf16(_ptr(W, _u8p), W.size, N, K, _ptr(x, _u16p), x.size,
                                                  _ptr(y, _f32p), N)
            else:
                x = np.ascontiguousarray(x, dtype=np.float32)
                rc = self.lib.ref_q4_0_gemv_f32(_ptr(W, _u8p), W.size, N, K, _ptr(x, _f32p), x.size,
                                                 _ptr(y, _f32p), N)
        else:
            x = np.ascontiguousarray(x, dtype=np.float32)
            rc = self.lib.ref_gemv_kq(t, _ptr(W, _u8p), N, K, _ptr(x, _f32p), _ptr(y, _f32p))
        if rc != 0:
            raise ValueError(self.error())
        return y

    def dequant_row(self, t: int, row: np.ndarray, K: int) -> np.ndarray:
        row = np.ascontiguousarray(row, dtype=np.uint8)
        out = np.empty(K, dtype=np.float32)
        if t == Q4_0:
            rc = self.lib.ref_q4_0_dequantize_row(_ptr(row, _u8p), row.size, K, _ptr(out, _f32p))
        else:
            rc = self.lib.ref_dequant_kq(t, _ptr(row, _u8p), K, _ptr(out, _f32p))
        if rc != 0:
            raise ValueError(self.error())
        return out

    def iq3s_grid(self) -> np.ndarray:
        g = np.empty(512, dtype=np.uint32)
        self.lib.ref_iq3s_grid(g.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
        return g


class RefCpuEngine:
    """The reference's AVX2+OpenMP Q4GemvEngine (4 threads for N > 256)."""

    THREADS = 4

    def __init__(self, ref: RefLib):
        self.ref = ref
        self.h = ref.lib.ref_cpu_engine_new()

    def run(self, W: np.ndarray, N: int, K: int, x: np.ndarray, y: np.ndarray) -> None:
        rc = self.ref.lib.ref_cpu_engine_run(self.h, _ptr(W, _u8p), W.size, N, K, _ptr(x, _f32p),
                                             _ptr(y, _f32p))
        if rc != 0:
            raise ValueError(self.ref.error())

    def close(self) -> None:
        if self.h:
            self.ref.lib.ref_cpu_engine_free(self.h)
            self.h = None


def decode_gemv(kind: str = "reference"):
    """CPU GEMV for the decode harness's callback backend (qwen2_decode.h):
    returns f(id, w, N, K, x, y) over raw addresses of ggml Q4_0 bytes, the
    f32 activation and the f32 output, and the number of threads it uses.

    kind "reference": the reference's AVX2+OpenMP Q4GemvEngine
    (src/cpu-q4-gemv-engine.cpp), from oracle/_ref;
    kind "oracle": the scalar C restatement (liboracle.so);
    kind "ggml_q8": ggml-cpu's Q8_0-activation numerics, restated in
    liboracle.so (external restatement, pinned by known answers; OpenMP over
    rows)."""
    if kind == "reference":
        ref = RefLib()
        eng = RefCpuEngine(ref)
        run = ref.lib.ref_cpu_engine_run

        def f(i, w, N, K, x, y):
            rc = run(eng.h, ctypes.cast(w, _u8p), N * (K // 32) * 18, N, K, ctypes.cast(x, _f32p),
                     ctypes.cast(y, _f32p))
            if rc != 0:
                raise ValueError(ref.error())
        f.engine = eng  # keeps the engine alive with the callable
        return f, RefCpuEngine.THREADS
    if kind == "oracle":
        o = Oracle()
        gemv = o.lib.orc_gemv_f32

        def f(i, w, N, K, x, y):
            rc = gemv(Q4_0, ctypes.cast(w, _u8p), N, K, ctypes.cast(x, _f32p), ctypes.cast(y, _f32p), None)
            if rc != 0:
                raise ValueError(f"orc_gemv_f32 rc={rc}")
        return f, 1
    if kind == "ggml_q8":
        o = Oracle()
        gemv = o.lib.orc_gemv_q4_0_q8_0

        def f(i, w, N, K, x, y):
            rc = gemv(ctypes.cast(w, _u8p), N, K, ctypes.cast(x, _f32p), ctypes.cast(y, _f32p))
            if rc != 0:
                raise ValueError(f"orc_gemv_q4_0_q8_0 rc={rc}")
        return f, os.cpu_count() or 1
    raise ValueError(kind)
