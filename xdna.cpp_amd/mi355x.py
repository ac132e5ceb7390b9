"""ctypes binding of libggml-mi355x.so (the C-ABI in include/mi355x-gemv.h).

Python is only the harness language here: tests and bench.py drive the
library through this module.  Loading fails loudly when the shared library is
missing -- there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libggml-mi355x.so")

OK, EINVAL, EUNSUPPORTED, EHIP, ENOMEM = 0, -1, -2, -3, -4

# ggml type ids
F32, Q4_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ3_S, IQ2_S, IQ4_XS = 0, 2, 11, 12, 13, 14, 18, 21, 22, 23
TYPE_NAMES = {Q4_0: "Q4_0", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
              IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S", IQ2_S: "IQ2_S", IQ4_XS: "IQ4_XS"}
BLOCK_VALUES = {Q4_0: 32, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, IQ3_XXS: 256, IQ3_S: 256,
                IQ2_S: 256, IQ4_XS: 256}
BLOCK_BYTES = {Q4_0: 18, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, IQ3_XXS: 98, IQ3_S: 110,
               IQ2_S: 82, IQ4_XS: 136}


OPT_VARIANT, OPT_ROWS_PER_WAVE, OPT_WAVES_PER_GROUP, OPT_GRID, OPT_PREFETCH, OPT_FORM, OPT_OVERLAP = 1, 2, 3, 4, 5, 6, 7
FORM_AUTO, FORM_ROWS, FORM_KSPLIT, FORM_STREAM, FORM_PIPE = 0, 1, 2, 3, 4
VARIANT_AUTO, VARIANT_EXACT_F32, VARIANT_DIGITS, VARIANT_GGML_Q8 = 0, 1, 2, 3


class Mi355xError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


_c = ctypes
_vp = _c.c_void_p
_SIGNATURES = {
    "mi355x_last_error": (_c.c_char_p, []),
    "mi355x_inject_fault": (_c.c_int, [_c.c_char_p, _c.c_int, _c.c_int]),
    "mi355x_device_count": (_c.c_int, [_c.POINTER(_c.c_int)]),
    "mi355x_ctx_create": (_c.c_int, [_c.c_int, _c.POINTER(_vp)]),
    "mi355x_ctx_destroy": (None, [_vp]),
    "mi355x_ctx_sync": (_c.c_int, [_vp]),
    "mi355x_ctx_fence": (_c.c_int, [_vp]),
    "mi355x_server_create": (_c.c_int, [_vp, _c.c_int64, _c.POINTER(_vp)]),
    "mi355x_server_gemv": (_c.c_int, [_vp, _vp, _c.c_int64, _c.c_int, _vp]),
    "mi355x_server_swiglu": (_c.c_int, [_vp, _vp, _c.c_int64, _vp, _vp, _c.c_int64, _vp, _c.c_int64, _vp]),
    "mi355x_server_block": (_c.c_int, [_vp, _vp, _c.c_int64, _vp, _vp, _c.c_int64, _vp, _c.c_float, _vp, _vp,
                                       _c.c_int64, _vp, _vp, _vp, _vp, _c.c_int64, _vp]),
    "mi355x_server_stop": (_c.c_int, [_vp]),
    "mi355x_server_running": (_c.c_int, [_vp]),
    "mi355x_server_destroy": (None, [_vp]),
    "mi355x_ctx_set_option": (_c.c_int, [_vp, _c.c_int, _c.c_int64]),
    "mi355x_ctx_stream": (_vp, [_vp]),
    "mi355x_ctx_device": (_c.c_int, [_vp]),
    "mi355x_mem_info": (_c.c_int, [_vp, _c.POINTER(_c.c_size_t), _c.POINTER(_c.c_size_t)]),
    "mi355x_device_describe": (_c.c_int, [_c.c_int, _c.c_char_p, _c.c_size_t, _c.c_char_p, _c.c_size_t]),
    "mi355x_malloc": (_c.c_int, [_vp, _c.c_size_t, _c.POINTER(_vp)]),
    "mi355x_free": (_c.c_int, [_vp, _vp]),
    "mi355x_host_malloc": (_c.c_int, [_c.c_size_t, _c.POINTER(_vp)]),
    "mi355x_host_free": (_c.c_int, [_vp]),
    "mi355x_host_device_ptr": (_c.c_int, [_vp, _c.POINTER(_vp)]),
    "mi355x_memcpy_h2d": (_c.c_int, [_vp, _vp, _vp, _c.c_size_t]),
    "mi355x_memcpy_d2h": (_c.c_int, [_vp, _vp, _vp, _c.c_size_t]),
    "mi355x_memcpy_d2d": (_c.c_int, [_vp, _vp, _vp, _c.c_size_t]),
    "mi355x_fill": (_c.c_int, [_vp, _vp, _c.c_uint8, _c.c_size_t]),
    "mi355x_row_bytes": (_c.c_int64, [_c.c_int, _c.c_int64]),
    "mi355x_type_ready": (_c.c_int, [_c.c_int]),
    "mi355x_set_iq_grid": (_c.c_int, [_c.c_int, _vp, _c.c_size_t]),
    "mi355x_prepack_from_host": (_c.c_int, [_vp, _c.c_int, _c.c_int64, _c.c_int64, _vp, _vp, _c.c_size_t,
                                            _c.c_size_t]),
    "mi355x_prepack_from_device": (_c.c_int, [_vp, _c.c_int, _c.c_int64, _c.c_int64, _vp, _vp, _c.c_size_t,
                                              _c.c_size_t]),
    "mi355x_unpack_to_host": (_c.c_int, [_vp, _c.c_int, _c.c_int64, _c.c_int64, _vp, _vp, _c.c_size_t,
                                         _c.c_size_t]),
    "mi355x_gemv": (_c.c_int, [_vp, _c.c_int, _vp, _c.c_int64, _c.c_int64, _vp, _vp]),
    "mi355x_gemv_multi": (_c.c_int, [_vp, _c.c_int, _c.c_int64, _vp, _c.c_int, _vp]),
    "mi355x_gemv_bf16": (_c.c_int, [_vp, _c.c_int, _vp, _c.c_int64, _c.c_int64, _vp, _vp]),
    "mi355x_gemv_batched": (_c.c_int, [_vp, _c.c_int, _vp, _c.c_int64, _c.c_int64, _vp, _c.c_int64, _vp,
                                       _c.c_int64, _c.c_int64]),
    "mi355x_gemv_batched_noalloc": (_c.c_int, [_vp, _c.c_int, _vp, _c.c_int64, _c.c_int64, _vp, _c.c_int64, _vp,
                                               _c.c_int64, _c.c_int64]),
    "mi355x_time_gemv": (_c.c_int, [_vp, _c.c_int, _c.POINTER(_vp), _c.c_int, _c.c_int64, _c.c_int64, _vp,
                                    _vp, _c.c_int, _c.c_int, _c.POINTER(_c.c_double)]),
}

class GemvJob(_c.Structure):
    """mi355x_gemv_job: {const void *W; int64_t N; float *y;}"""
    _fields_ = [("W", _c.c_void_p), ("N", _c.c_int64), ("y", _c.c_void_p)]


MULTI_MAX_JOBS = 8
# device id of a host-only context (no GPU; every device call fails)
DEVICE_HOST_ONLY = -1
# hipError_t values used with mi355x_inject_fault
HIP_ERROR_OUT_OF_MEMORY, HIP_ERROR_NO_DEVICE, HIP_ERROR_ILLEGAL_ADDRESS, HIP_ERROR_LAUNCH_FAILURE = 2, 100, 700, 719


def inject_fault(entry: str | None, hip_error: int = 0, skip: int = 0) -> None:
    """Arms a one-shot injected HIP error on the C-ABI entry point `entry`
    ("*": any device entry point) after `skip` more calls; None disarms."""
    check(load().mi355x_inject_fault(entry.encode() if entry else None, hip_error, skip))

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the shared library (raises if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().mi355x_last_error().decode()


def check(rc: int) -> None:
    if rc != OK:
        raise Mi355xError(rc, last_error())


def device_count() -> int:
    n = ctypes.c_int(0)
    check(load().mi355x_device_count(ctypes.byref(n)))
    return n.value


def row_bytes(t: int, K: int) -> int:
    return load().mi355x_row_bytes(t, K)


def type_ready(t: int) -> bool:
    return bool(load().mi355x_type_ready(t))


def set_iq_grid(t: int, table: np.ndarray) -> None:
    table = np.ascontiguousarray(table)
    check(load().mi355x_set_iq_grid(t, table.ctypes.data, table.nbytes))


class DeviceBuffer:
    """A device allocation owned by a Context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(ctx.lib.mi355x_malloc(ctx.h, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def free(self) -> None:
        if self.ptr:
            check(self.ctx.lib.mi355x_free(self.ctx.h, self.ptr))
            self.ptr = None

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload overruns the buffer")
        check(self.ctx.lib.mi355x_memcpy_h2d(self.ctx.h, self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download overruns the buffer")
        check(self.ctx.lib.mi355x_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr + offset, out.nbytes))
        return out


class ResidentWeights:
    """A weight tensor prepacked into the resident layout on the device."""

    def __init__(self, ctx: "Context", t: int, raw: np.ndarray, N: int, K: int, chunk: int | None = None):
        rb = row_bytes(t, K)
        if rb < 0:
            raise ValueError(f"K={K} is not a multiple of the block of type {t}")
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        if raw.size != N * rb:
            raise ValueError(f"raw weights hold {raw.size} bytes, expected {N * rb}")
        self.ctx, self.t, self.N, self.K, self.nbytes = ctx, t, N, K, N * rb
        self.buf = DeviceBuffer(ctx, max(self.nbytes, 1))
        step = chunk or max(self.nbytes, 1)
        for off in range(0, self.nbytes, step):
            n = min(step, self.nbytes - off)
            view = raw[off:off + n]
            check(ctx.lib.mi355x_prepack_from_host(ctx.h, t, N, K, self.buf.ptr, view.ctypes.data, off, n))

    @property
    def ptr(self) -> int:
        return self.buf.ptr

    def raw_bytes(self, offset: int = 0, size: int | None = None) -> np.ndarray:
        size = self.nbytes - offset if size is None else size
        out = np.empty(size, dtype=np.uint8)
        check(self.ctx.lib.mi355x_unpack_to_host(self.ctx.h, self.t, self.N, self.K, self.buf.ptr,
                                                 out.ctypes.data, offset, size))
        return out

    def free(self) -> None:
        self.buf.free()


class ServerJob(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("N", ctypes.c_int64), ("y", ctypes.c_void_p)]


class Server:
    """Persistent Q4_0 GEMV server (mi355x_server_*) on a Context's device."""

    def __init__(self, ctx: "Context", max_k: int):
        self.lib = ctx.lib
        h = ctypes.c_void_p()
        check(self.lib.mi355x_server_create(ctx.h, max_k, ctypes.byref(h)))
        self.h = h.value

    def gemv_ptr(self, x: np.ndarray, jobs) -> int:
        """jobs: [(W device pointer, N, y device-visible pointer)]; x: host f32."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        arr = (ServerJob * len(jobs))(*[ServerJob(w, n, y) for w, n, y in jobs])
        return self.lib.mi355x_server_gemv(self.h, x.ctypes.data, x.size, len(jobs), arr)

    def gemv(self, x: np.ndarray, jobs) -> None:
        check(self.gemv_ptr(x, jobs))

    def swiglu_ptr(self, x: np.ndarray, w_gate: int, w_up: int, F: int, w_down: int, N: int, y: int) -> int:
        """y = W_down (silu(W_gate x) * (W_up x)) as one command (device pointers)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        return self.lib.mi355x_server_swiglu(self.h, x.ctypes.data, x.size, w_gate, w_up, F, w_down, N, y)

    def swiglu(self, x: np.ndarray, w_gate: int, w_up: int, F: int, w_down: int, N: int, y: int) -> None:
        check(self.swiglu_ptr(x, w_gate, w_up, F, w_down, N, y))

    def block_ptr(self, x: np.ndarray, w_o: int, resid: np.ndarray, norm_w: int, eps: float, w_gate: int,
                  w_up: int, F: int, w_down: int, y: int, next_norm_w: int = 0, w_next: int = 0, N_next: int = 0,
                  y_next: int = 0) -> int:
        """y = r + W_down (silu(W_gate xn) * (W_up xn)), xn = rmsnorm(r) * norm_w,
        r = resid + W_o x, as one command (x, resid: host f32; the rest device);
        with w_next also y_next = W_next (rmsnorm(y) * next_norm_w).  resid as
        an int H: the residual the server kept from the last block command;
        y 0: y is only kept in the server."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if isinstance(resid, int):  # H, the residual the server holds
            rp, H = None, resid
        else:
            resid = np.ascontiguousarray(resid, dtype=np.float32)
            rp, H = resid.ctypes.data, resid.size
        return self.lib.mi355x_server_block(self.h, x.ctypes.data, x.size, w_o, rp, H, norm_w, eps, w_gate, w_up, F,
                                            w_down, y or None, next_norm_w or None, w_next or None, N_next,
                                            y_next or None)

    def block(self, *args) -> None:
        check(self.block_ptr(*args))

    def stop(self) -> None:
        check(self.lib.mi355x_server_stop(self.h))

    def running(self) -> bool:
        """True while the resident kernel runs (it leaves after 1 s idle)."""
        rc = self.lib.mi355x_server_running(self.h)
        if rc < 0:
            check(rc)
        return rc == 1

    def close(self) -> None:
        if self.h:
            self.lib.mi355x_server_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Context:
    """One device + one HIP stream (mi355x_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = ctypes.c_void_p()
        check(self.lib.mi355x_ctx_create(device, ctypes.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            self.lib.mi355x_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_option(self, option: int, value: int) -> None:
        check(self.lib.mi355x_ctx_set_option(self.h, option, value))

    def sync(self) -> None:
        check(self.lib.mi355x_ctx_sync(self.h))

    def fence(self) -> None:
        """Spin-wait on the context's completion word (covers device memory
        and pinned host memory)."""
        check(self.lib.mi355x_ctx_fence(self.h))

    def describe(self) -> tuple[str, str]:
        name = ctypes.create_string_buffer(256)
        pci = ctypes.create_string_buffer(64)
        check(self.lib.mi355x_device_describe(self.lib.mi355x_ctx_device(self.h), name, 256, pci, 64))
        return name.value.decode(), pci.value.decode()

    def mem_info(self) -> tuple[int, int]:
        f, t = ctypes.c_size_t(), ctypes.c_size_t()
        check(self.lib.mi355x_mem_info(self.h, ctypes.byref(f), ctypes.byref(t)))
        return f.value, t.value

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        b = DeviceBuffer(self, max(a.nbytes, 1))
        if a.nbytes:
            b.upload(a)
        return b

    def resident(self, t: int, raw: np.ndarray, N: int, K: int, chunk: int | None = None) -> ResidentWeights:
        return ResidentWeights(self, t, raw, N, K, chunk)

    def gemv_ptr(self, t: int, w_ptr: int, N: int, K: int, x_ptr: int, y_ptr: int, bf16: bool = False) -> int:
        fn = self.lib.mi355x_gemv_bf16 if bf16 else self.lib.mi355x_gemv
        return fn(self.h, t, w_ptr, N, K, x_ptr, y_ptr)

    def gemv_multi_ptr(self, t: int, K: int, x_ptr: int, jobs) -> int:
        """mi355x_gemv_multi over (w_ptr, N, y_ptr) jobs sharing x."""
        arr = (GemvJob * len(jobs))(*[GemvJob(w, n, y) for w, n, y in jobs])
        return self.lib.mi355x_gemv_multi(self.h, t, K, x_ptr, len(jobs), arr)

    def gemv_batched_ptr(self, t: int, w_ptr: int, N: int, K: int, x_ptr: int, x_stride: int, y_ptr: int,
                         y_stride: int, M: int) -> int:
        return self.lib.mi355x_gemv_batched(self.h, t, w_ptr, N, K, x_ptr, x_stride, y_ptr, y_stride, M)

    def gemv_batched(self, w: ResidentWeights, xs: np.ndarray, x_stride: int | None = None,
                     y_stride: int | None = None) -> np.ndarray:
        """M GEMVs against the same weights (xs: M x K); activation rows
        x_stride floats apart and outputs y_stride floats apart on the device."""
        M = xs.shape[0]
        xst = x_stride or w.K
        yst = y_stride or w.N
        xp = np.zeros((M, xst), np.float32)
        xp[:, :w.K] = xs
        xb = self.to_device(xp)
        yb = self.alloc(4 * max(M * yst, 1))
        try:
            check(self.gemv_batched_ptr(w.t, w.ptr, w.N, w.K, xb.ptr, xst, yb.ptr, yst, M))
            self.sync()
            return yb.download(np.float32, M * yst).reshape(M, yst)[:, :w.N]
        finally:
            xb.free()
            yb.free()

    def gemv(self, w: ResidentWeights, x: np.ndarray) -> np.ndarray:
        """One GEMV with host activations; returns the host output."""
        bf16 = x.dtype == np.uint16
        xb = self.to_device(x)
        yb = self.alloc(4 * max(w.N, 1))
        try:
            check(self.gemv_ptr(w.t, w.ptr, w.N, w.K, xb.ptr, yb.ptr, bf16))
            self.sync()
            return yb.download(np.float32, w.N)
        finally:
            xb.free()
            yb.free()

    def time_gemv(self, t: int, weight_ptrs: list[int], N: int, K: int, x_ptr: int, y_ptr: int,
                  warmup: int, iters: int) -> float:
        arr = (ctypes.c_void_p * len(weight_ptrs))(*weight_ptrs)
        ms = ctypes.c_double(0.0)
        check(self.lib.mi355x_time_gemv(self.h, t, arr, len(weight_ptrs), N, K, x_ptr, y_ptr, warmup, iters,
                                        ctypes.byref(ms)))
        return ms.value
