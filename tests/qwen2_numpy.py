"""Independent float64 numpy forward pass of the decode harness's model, used
to check that decode/qwen2_decode.cpp computes a Qwen2 decoder step.

Standard Qwen2 decoder layer (the architecture llama.cpp runs for
Qwen2.5-3B): RMSNorm; q/k/v projections with bias; NeoX-style
(rotate-half) RoPE; grouped-query softmax attention with scale 1/sqrt(d);
output projection and residual; RMSNorm; SwiGLU FFN and residual.  A final
RMSNorm and the tied embedding matrix give the logits.  Weights are the
harness's own Q4_0 bytes, dequantized by the C oracle.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

QD_Q, QD_K, QD_V, QD_O, QD_GATE, QD_UP, QD_DOWN = range(7)


def dequantized(model, oracle, i: int) -> np.ndarray:
    p, N, K = model.matrix(i)
    rb = K // 32 * 18
    raw = np.ctypeslib.as_array((C.c_uint8 * (N * rb)).from_address(p))
    return np.stack([oracle.dequant_row(2, raw[r * rb:(r + 1) * rb], K) for r in range(N)]).astype(np.float64)


class Qwen2Numpy:
    def __init__(self, model, oracle):
        c = model.cfg
        self.c = c
        L = c.n_layers
        self.W = [dequantized(model, oracle, i) for i in range(7 * L + 1)]
        self.vec = [model.vector(i).astype(np.float64) for i in range(5 * L + 1)]

    def _rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c.norm_eps) * w

    def _rope(self, v, pos):
        hd = self.c.head_dim
        half = hd // 2
        f = pos * self.c.rope_theta ** (-2.0 * np.arange(half) / hd)
        cos, sin = np.cos(f), np.sin(f)
        a, b = v[..., :half].copy(), v[..., half:].copy()
        return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1)

    def generate(self, prompt, n_gen):
        """Greedy tokens and the logits behind the last one."""
        c, W, V = self.c, self.W, self.vec
        L, hd, nh, nkv = c.n_layers, c.head_dim, c.n_heads, c.n_kv_heads
        kc = [[] for _ in range(L)]
        vc = [[] for _ in range(L)]
        out, logits = [], None
        n_pos = len(prompt) + n_gen - 1
        tok = int(prompt[0])
        for pos in range(n_pos):
            if pos < len(prompt):
                tok = int(prompt[pos])
            h = W[7 * L][tok].copy()
            for layer in range(L):
                w = W[7 * layer:7 * layer + 7]
                x = self._rms(h, V[5 * layer])
                q = (w[QD_Q] @ x + V[5 * layer + 2]).reshape(nh, hd)
                k = (w[QD_K] @ x + V[5 * layer + 3]).reshape(nkv, hd)
                v = (w[QD_V] @ x + V[5 * layer + 4]).reshape(nkv, hd)
                q, k = self._rope(q, pos), self._rope(k, pos)
                kc[layer].append(k)
                vc[layer].append(v)
                K_, V_ = np.stack(kc[layer]), np.stack(vc[layer])  # [t, nkv, hd]
                att = np.empty((nh, hd))
                for hh in range(nh):
                    g = hh // (nh // nkv)
                    s = K_[:, g, :] @ q[hh] / np.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[hh] = (p / p.sum()) @ V_[:, g, :]
                h = h + w[QD_O] @ att.reshape(-1)
                x = self._rms(h, V[5 * layer + 1])
                gt, up = w[QD_GATE] @ x, w[QD_UP] @ x
                h = h + w[QD_DOWN] @ (gt / (1.0 + np.exp(-gt)) * up)
            if pos + 1 < len(prompt):
                continue
            logits = W[7 * L] @ self._rms(h, V[5 * L])
            tok = int(np.argmax(logits))
            out.append(tok)
        return np.array(out, dtype=np.int32), logits
