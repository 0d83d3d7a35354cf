"""CPU restatement of the reference's decode attention and KV cache.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the library's paged
decode attention (garuda_amd/csrc/gmoe_attn.hip, gmoe_kv.cpp). The product never loads
it.

Follows LlamaBackend::attend_one (garuda/src/llama/mod.rs:766-821): rope q (every query
head) and k (every kv head) at pos = the cache's length (simd::rope, simd/mod.rs:196-206,
in f32 as the reference forms freq and angle), append, then per query head h with kv
head h / group: scores over [attention_start, pos] = dot(q_h, k_j) * (1/sqrt(hd)),
softmax (uniform weights when a score is NaN or +inf, or none is finite, as simd::softmax
falls back), context = sum_j p_j v_j. KVCacheState (cache/mod.rs:221-600): per-layer
lengths, the context-window cap (:348-362) and attention_start with a sliding window
(:333-338). The dot products, softmax and weighted sum are evaluated in float64 here
(the reference's f32 sums are within the layer tolerance of them).

Pinned by the reference's rope tests (simd/mod.rs:282-299), closed forms (a single
position returns its value; equal scores average the values; rope of a unit vector at
position p is (cos, sin) of p * freq) and brute force over small caches
(tests/test_attention_oracle.py).
"""
from __future__ import annotations

import numpy as np


def rope(v: np.ndarray, pos: int, theta: float) -> np.ndarray:
    """simd::rope over one head's vector (f32)."""
    v = np.asarray(v, dtype=np.float32).copy()
    hd = v.size
    for i in range(hd // 2):
        freq = np.float32(1.0) / np.float32(np.float32(theta) ** (np.float32(2.0 * i) / np.float32(hd)))
        ang = np.float32(pos) * freq
        s, c = np.float32(np.sin(np.float64(ang))), np.float32(np.cos(np.float64(ang)))
        a, b = v[2 * i], v[2 * i + 1]
        v[2 * i] = a * c - b * s
        v[2 * i + 1] = a * s + b * c
    return v


class KvOracle:
    def __init__(self, n_layers, n_heads, n_kv_heads, head_dim, max_positions=2048, sliding_window=0,
                 rope_theta=10000.0):
        self.nl, self.nh, self.nkv, self.hd = n_layers, n_heads, n_kv_heads, head_dim
        self.maxpos, self.win, self.theta = max_positions, sliding_window, rope_theta
        self.keys, self.vals = {}, {}

    def _kv(self, seq, layer):
        key = (seq, layer)
        if key not in self.keys:
            self.keys[key], self.vals[key] = [], []
        return self.keys[key], self.vals[key]

    def seq_len(self, seq, layer=0):
        return len(self._kv(seq, layer)[0])

    def attend_one(self, layer, seq, q, k, v):
        K, V = self._kv(seq, layer)
        pos = len(K)
        if pos >= self.maxpos:
            raise ValueError("context window exhausted")
        hd, group = self.hd, self.nh // self.nkv
        q = np.concatenate([rope(q[h * hd:(h + 1) * hd], pos, self.theta) for h in range(self.nh)])
        k = np.concatenate([rope(k[h * hd:(h + 1) * hd], pos, self.theta) for h in range(self.nkv)])
        K.append(k)
        V.append(np.asarray(v, dtype=np.float32).copy())
        start = max(0, pos + 1 - self.win) if self.win else 0
        Ks, Vs = np.array(K[start:], dtype=np.float64), np.array(V[start:], dtype=np.float64)
        Ks32 = np.array(K[start:], dtype=np.float32)
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        out = np.empty(self.nh * hd, dtype=np.float64)
        for h in range(self.nh):
            kh = h // group
            with np.errstate(invalid="ignore", over="ignore"):
                s = Ks[:, kh * hd:(kh + 1) * hd] @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
                # the reference's scores are f32 (simd::dot * scale): whether one is NaN or
                # +inf, or none is above -inf, is read from an f32 evaluation
                s32 = (Ks32[:, kh * hd:(kh + 1) * hd] @ q[h * hd:(h + 1) * hd]) * np.float32(scale)
            if np.isnan(s32).any() or np.isposinf(s32).any() or np.isneginf(s32).all():
                # simd/mod.rs:132-158: a NaN or +inf score, or nothing finite, gives uniform weights
                p = np.full(s.size, 1.0 / s.size)
            else:
                p = np.exp(s - s.max())
                p /= p.sum()
            out[h * hd:(h + 1) * hd] = p @ Vs[:, kh * hd:(kh + 1) * hd]
        return out

    def attention(self, layer, seqs, q, k, v):
        """Entries in order, each attending after its own append."""
        n = len(seqs)
        q = np.asarray(q, dtype=np.float32).reshape(n, -1)
        k = np.asarray(k, dtype=np.float32).reshape(n, -1)
        v = np.asarray(v, dtype=np.float32).reshape(n, -1)
        return np.stack([self.attend_one(layer, int(s), q[i], k[i], v[i]) for i, s in enumerate(seqs)])
