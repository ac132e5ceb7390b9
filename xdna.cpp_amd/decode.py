"""ctypes binding of the end-to-end decode harness (decode/libqwen2-decode.so).

The harness is a batch-1 greedy decoder of a Qwen2-shaped model with seeded
random Q4_0 weights (decode/qwen2_decode.h).  Its matrix-vector products go
either to the MI355X library (weights resident in HBM) or to a caller's
function -- the CPU reference used to check token identity.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "decode", "libqwen2-decode.so")

GEMV_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p)


class Config(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int), ("n_kv_heads", C.c_int),
                ("head_dim", C.c_int), ("ffn", C.c_int), ("vocab", C.c_int), ("rope_theta", C.c_float),
                ("norm_eps", C.c_float), ("seed", C.c_uint64)]


# Qwen2.5-3B shape
QWEN25_3B = dict(n_layers=36, hidden=2048, n_heads=16, n_kv_heads=2, head_dim=128, ffn=11008, vocab=151936,
                 rope_theta=1e6, norm_eps=1e-6, seed=20250101)

_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is missing: build with `make -C xdna.cpp_amd`")
    lib = C.CDLL(path)
    lib.qd_model_create.restype = C.c_void_p
    lib.qd_model_create.argtypes = [C.POINTER(Config), C.c_int]
    lib.qd_model_free.argtypes = [C.c_void_p]
    lib.qd_n_matrices.restype = C.c_int
    lib.qd_n_matrices.argtypes = [C.c_void_p]
    lib.qd_matrix.restype = C.c_void_p
    lib.qd_matrix.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
    lib.qd_last_error.restype = C.c_char_p
    lib.qd_vector.restype = C.POINTER(C.c_float)
    lib.qd_vector.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_int)]
    lib.qd_last_logits.restype = C.c_int
    lib.qd_last_logits.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.qd_quantize_q4_0.argtypes = [C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]
    lib.qd_silu_mul.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    lib.qd_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_float]
    lib.qd_set_block.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_swiglu.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_plugin_groups.restype = C.c_int
    lib.qd_set_plugin_groups.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_fuse.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_variant.restype = C.c_int
    lib.qd_set_variant.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_io.restype = C.c_int
    lib.qd_set_io.argtypes = [C.c_void_p, C.c_int]
    lib.qd_set_wait.restype = C.c_int
    lib.qd_set_wait.argtypes = [C.c_void_p, C.c_int]
    lib.qd_last_wait.restype = C.c_int
    lib.qd_last_wait.argtypes = [C.c_void_p]
    lib.qd_last_launches.restype = C.c_int64
    lib.qd_last_launches.argtypes = [C.c_void_p]
    lib.qd_attach_gpu.restype = C.c_int
    lib.qd_attach_gpu.argtypes = [C.c_void_p, C.c_int]
    lib.qd_generate.restype = C.c_int
    lib.qd_generate.argtypes = [C.c_void_p, C.c_int, GEMV_FN, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                C.c_void_p, C.POINTER(C.c_double)]
    _lib = lib
    return lib


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    out = np.empty(N * (K // 32) * 18, dtype=np.uint8)
    load().qd_quantize_q4_0(w.ctypes.data, N, K, out.ctypes.data)
    return out.reshape(N, -1)


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """The decoder's host SwiGLU step: silu(g) * u in the f32 steps that
    mi355x_server_swiglu states."""
    g = np.array(g, dtype=np.float32, copy=True)
    u = np.ascontiguousarray(u, dtype=np.float32)
    assert g.shape == u.shape and g.ndim == 1
    load().qd_silu_mul(g.ctypes.data, u.ctypes.data, g.size)
    return g


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The decoder's host RMSNorm (the steps mi355x_server_block states)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    assert x.shape == w.shape and x.ndim == 1
    out = np.empty_like(x)
    load().qd_rmsnorm(x.ctypes.data, w.ctypes.data, out.ctypes.data, x.size, eps)
    return out


def prompt_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """Uniform-random synthetic prompt."""
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


class Model:
    def __init__(self, threads: int = 8, **cfg):
        self.lib = load()
        self.cfg = Config(**cfg)
        self.h = self.lib.qd_model_create(C.byref(self.cfg), threads)
        if not self.h:
            raise RuntimeError(self.lib.qd_last_error().decode())

    def close(self) -> None:
        if self.h:
            self.lib.qd_model_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def n_matrices(self) -> int:
        return self.lib.qd_n_matrices(self.h)

    def matrix(self, i: int):
        """(pointer to ggml Q4_0 bytes, N, K) of matrix i."""
        N, K = C.c_int64(), C.c_int64()
        p = self.lib.qd_matrix(self.h, i, C.byref(N), C.byref(K))
        return p, N.value, K.value

    def vector(self, i: int) -> np.ndarray:
        """Copy of vector i: 5 per layer (attn norm, ffn norm, q/k/v bias),
        then the output norm."""
        n = C.c_int()
        p = self.lib.qd_vector(self.h, i, C.byref(n))
        if not p:
            raise IndexError(i)
        return np.ctypeslib.as_array(p, (n.value,)).copy()

    def weight_bytes(self) -> int:
        return sum(self.matrix(i)[1] * (self.matrix(i)[2] // 32) * 18 for i in range(self.n_matrices()))

    def last_logits(self) -> np.ndarray:
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        if self.lib.qd_last_logits(self.h, out.ctypes.data, self.cfg.vocab) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())
        return out

    def set_fuse(self, on: bool) -> None:
        self.lib.qd_set_fuse(self.h, 1 if on else 0)

    def set_block(self, on: bool) -> None:
        """Server mode: o through down as one command (default on)."""
        self.lib.qd_set_block(self.h, 1 if on else 0)

    def set_swiglu(self, on: bool) -> None:
        """Server mode: gate|up, SiLU and down as one command (default on);
        off: two GEMV commands with SiLU on the host, so only the MUL_MATs
        run on the GPU (block commands need it on)."""
        self.lib.qd_set_swiglu(self.h, 1 if on else 0)

    def set_variant(self, variant: int) -> None:
        """GEMV kernel variant on the GPU path (mi355x.VARIANT_*)."""
        if self.lib.qd_set_variant(self.h, variant) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())

    IO_STAGED, IO_MAPPED = 0, 1

    def set_io(self, mode: int) -> None:
        """IO_STAGED: activations/outputs copied through HBM around each GEMV
        group; IO_MAPPED (default): kernels read/write pinned host memory."""
        if self.lib.qd_set_io(self.h, mode) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())

    WAIT_STREAM, WAIT_FENCE, WAIT_SERVER, WAIT_PLUGIN = 0, 1, 2, 3

    def set_wait(self, mode: int) -> None:
        """WAIT_SERVER (default): GEMV groups as commands to a persistent
        server kernel (where it applies, else WAIT_FENCE); WAIT_FENCE: one
        launch per GEMV group, then a spin on a completion word; WAIT_STREAM:
        hipStreamSynchronize instead; WAIT_PLUGIN: every group through the
        ggml plugin (weights as tensors in its buffer, activation in, one
        graph_compute per group, outputs out, synchronize)."""
        if self.lib.qd_set_wait(self.h, mode) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())

    PLUGIN_GROUPS_SERVER, PLUGIN_GROUPS_LAUNCH = 0, 1

    def set_plugin_groups(self, mode: int) -> None:
        """WAIT_PLUGIN: graph_compute runs a group as one launch
        (PLUGIN_GROUPS_LAUNCH, default) or a server command (PLUGIN_GROUPS_SERVER)."""
        if self.lib.qd_set_plugin_groups(self.h, mode) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())

    def last_wait(self) -> int:
        """The wait mode the last GPU decode used."""
        return self.lib.qd_last_wait(self.h)

    def last_launches(self) -> int:
        return self.lib.qd_last_launches(self.h)

    def attach_gpu(self, device: int = 0) -> None:
        if self.lib.qd_attach_gpu(self.h, device) != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())

    def generate(self, prompt: np.ndarray, n_gen: int, cpu_gemv=None):
        """Greedy decode on the GPU (cpu_gemv None) or with cpu_gemv(id, w_ptr,
        N, K, x_ptr, y_ptr).  Returns (tokens, timings dict)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(n_gen, 1), dtype=np.int32)
        t = (C.c_double * 4)()
        if cpu_gemv is None:
            cb, backend = GEMV_FN(0), 0
        else:
            def shim(user, i, w, N, K, x, y):
                try:
                    cpu_gemv(i, w, N, K, x, y)
                    return 0
                except Exception:  # reported as a failed GEMV
                    return -1
            cb, backend = GEMV_FN(shim), 1
        rc = self.lib.qd_generate(self.h, backend, cb, None, prompt.ctypes.data, len(prompt), n_gen,
                                  out.ctypes.data, t)
        if rc != 0:
            raise RuntimeError(self.lib.qd_last_error().decode())
        return out[:n_gen], {"prompt_s": t[0], "gen_s": t[1], "gen_gemv_s": t[2], "gen_host_s": t[3],
                             "gen_passes": max(n_gen - 1, 0)}
